"""Step-level engine: requests in, completions out (vflorence/engine/llm_engine.py:18-171).

Same API and request validation as the reference (``add_request``, ``step``,
``generate``, ``abort``, ``is_finished``); the runner executes each step on the GPU.
A rejected request yields an empty completion while the others run; a failed step
drops every request and returns all blocks and encoder pages.
"""

from __future__ import annotations

import gc
import logging
import math
from contextlib import contextmanager

import torch

from ..config import Config
from ..sampling_params import SamplingParams
from .model_runner import ModelRunner
from .scheduler import Scheduler
from .sequence import Request, RequestOut, Sequence

__all__ = ["LLMEngine", "Request", "RequestOut"]

logger = logging.getLogger(__name__)


class LLMEngine:
    def __init__(self, model, state_dict: dict | None = None, **kwargs):
        config = Config(model, **kwargs)
        self.config = config
        self.runner = ModelRunner(config, state_dict)
        self.scheduler = Scheduler(config)
        text = config.text_config
        self.decoder_start_token_id = text.decoder_start_token_id
        self.eos_token_id = text.eos_token_id
        self._sampling_params = SamplingParams.from_generation_config(
            config.generation_config, self.eos_token_id)
        self._next_request_id = 0

    def add_request(self, request: Request, sampling_params: SamplingParams | None = None) -> int:
        if sampling_params is None:
            sampling_params = self._sampling_params
        else:
            sampling_params = sampling_params.with_defaults(self._sampling_params)
        self._validate(request, sampling_params)
        request_id = self._next_request_id
        self._next_request_id += 1
        self.scheduler.add(Sequence(request_id, [self.decoder_start_token_id], request.input_ids,
                                    sampling_params, request.pixel_values))
        return request_id

    def step(self) -> list[tuple[int, RequestOut]]:
        seqs, copies = self.scheduler.schedule()
        sample_out = self.runner.run(seqs, copies)
        outputs = self.scheduler.postprocess(seqs, sample_out)
        for request_id, _ in outputs:
            self.runner.clear_request(request_id)
        return outputs

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    @contextmanager
    def _abort_on_failure(self):
        try:
            yield
        except BaseException:
            self.abort()
            raise

    def abort(self) -> None:
        """Drop every waiting and running request; release blocks and encoder pages."""
        self.scheduler.reset()
        self.runner.reset()

    @torch.inference_mode()
    def generate(self, requests, sampling_params: SamplingParams | None = None,
                 use_tqdm: bool = False) -> list[RequestOut]:
        requests = [requests] if isinstance(requests, Request) else list(requests)
        if not requests:
            return []
        slots: list = []
        for request in requests:
            try:
                slots.append(self.add_request(request, sampling_params))
            except ValueError as e:
                logger.error("request rejected: %s", e)
                slots.append(RequestOut(request.input_ids, [], request.pixel_values))
        outputs: dict[int, RequestOut] = {}
        # Every step allocates and drops one Sequence per running row; they hold no
        # reference cycles, so reference counting frees them and the cyclic collector
        # would only add pauses to the step loop.
        collecting = gc.isenabled()
        gc.disable()
        try:
            with self._abort_on_failure():
                while not self.is_finished():
                    for request_id, out in self.step():
                        outputs[request_id] = out
        finally:
            if collecting:
                gc.enable()
        return [outputs[s] if isinstance(s, int) else s for s in slots]

    def _validate(self, request: Request, sampling_params: SamplingParams) -> None:
        """Reject a request that would fail or run out of KV cache mid-step."""
        cfg = self.config
        if request.pixel_values is not None:
            raise ValueError("pixel_values are only supported for Florence-2 checkpoints")
        active = self.scheduler.waiting or self.scheduler.running
        if active and active[0].sampling_params != sampling_params:
            raise ValueError("all active requests must share the same SamplingParams")
        if sampling_params.max_tokens > cfg.max_decoder_len:
            raise ValueError(f"max_tokens ({sampling_params.max_tokens}) exceeds the engine's "
                             f"max_decoder_len ({cfg.max_decoder_len})")
        if len(request.input_ids) > cfg.max_encoder_len:
            raise ValueError(f"encoder prompt has {len(request.input_ids)} tokens; the engine "
                             f"supports at most max_encoder_len={cfg.max_encoder_len}")
        if not request.input_ids:
            raise ValueError("encoder prompt is empty")
        if sampling_params.num_beams > cfg.max_num_seqs:
            raise ValueError(f"num_beams ({sampling_params.num_beams}) exceeds "
                             f"max_num_seqs ({cfg.max_num_seqs})")
        need = sampling_params.num_beams * math.ceil(sampling_params.max_tokens / cfg.block_size)
        if need > cfg.num_blocks:
            raise ValueError(f"one request may need {need} KV blocks but num_blocks is "
                             f"{cfg.num_blocks}; increase num_blocks")
