"""MI355X (gfx950) decode-step attention path for vflorence.

Submodules:
    hip_attn                 -- torch wrappers of the C ABI (counterpart of vllm_cpu_attn)
    layers.attention         -- vflorence::self_attention / vflorence::cross_attention ops
    layers.bart              -- BART whose decoder attention calls those ops
    layers.logits_processor  -- generation rules on the GPU
    utils.context            -- per-step Context read by the ops
    engine                   -- block manager, scheduler, GPU runner, engine

``LLM``, ``Request``, ``RequestOut`` and ``SamplingParams`` are the reference's public
names (vflorence/__init__.py); they load on first use so kernel-only users do not
import the engine.
"""

__version__ = "0.1.0"
__all__ = ["LLM", "Request", "RequestOut", "SamplingParams"]


def __getattr__(name):
    if name == "LLM":
        from .llm import LLM

        return LLM
    if name in ("Request", "RequestOut"):
        from .engine import sequence

        return getattr(sequence, name)
    if name == "SamplingParams":
        from .sampling_params import SamplingParams

        return SamplingParams
    raise AttributeError(name)
