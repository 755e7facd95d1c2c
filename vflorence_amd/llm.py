"""``LLM``: the engine under the reference's public name (vflorence/llm.py:1-5)."""

from .engine.llm_engine import LLMEngine


class LLM(LLMEngine):
    pass
