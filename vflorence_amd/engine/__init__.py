"""Host-side engine around the GPU path: block manager, scheduler, runner, engine."""

from .block_manager import BlockManager
from .llm_engine import LLMEngine, Request, RequestOut
from .model_runner import ModelRunner
from .scheduler import Scheduler
from .sequence import Sequence

__all__ = ["BlockManager", "LLMEngine", "ModelRunner", "Request", "RequestOut", "Scheduler",
           "Sequence"]
