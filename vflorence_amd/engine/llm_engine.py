"""Requests in, completions out: the step loop of vflorence/engine/llm_engine.py:18-171.

``add_request`` validates a request against the engine's limits and queues it;
``step`` runs one decode step (schedule on the host core -> GPU step -> feed the
result back) and returns the requests that finished; ``generate`` steps until every
accepted request is done.  A rejected request yields an empty completion while the
others run; a step that raises drops every request and frees every block and
encoder page before the exception propagates.
"""

from __future__ import annotations

import gc
import logging
import math

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
        text = config.text_config
        self.config = config
        self.decoder_start_token_id = text.decoder_start_token_id
        self.eos_token_id = text.eos_token_id
        # the checkpoint's generation config fills whatever a request leaves unset
        self._sampling_params = SamplingParams.from_generation_config(
            config.generation_config, self.eos_token_id)
        self.scheduler = Scheduler(config)
        self.runner = ModelRunner(config, state_dict)
        self._next_request_id = 0

    # -- requests ------------------------------------------------------------------------

    def _limits_violated(self, request: Request, params: SamplingParams) -> str | None:
        """Why the engine cannot run ``request`` with ``params`` (None if it can)."""
        cfg = self.config
        if request.pixel_values is not None:
            return "pixel_values are only supported for Florence-2 checkpoints"
        shared = self.scheduler.active_params()
        if shared is not None and shared != params:
            return "all active requests must share the same SamplingParams"
        if params.max_tokens > cfg.max_decoder_len:
            return (f"max_tokens ({params.max_tokens}) exceeds the engine's max_decoder_len "
                    f"({cfg.max_decoder_len})")
        n = len(request.input_ids)
        if n > cfg.max_encoder_len:
            return (f"encoder prompt has {n} tokens; the engine supports at most "
                    f"max_encoder_len={cfg.max_encoder_len}")
        if n == 0:
            return "encoder prompt is empty"
        if params.num_beams > cfg.max_num_seqs:
            return f"num_beams ({params.num_beams}) exceeds max_num_seqs ({cfg.max_num_seqs})"
        blocks = params.num_beams * math.ceil(params.max_tokens / cfg.block_size)
        if blocks > cfg.num_blocks:
            return (f"one request may need {blocks} KV blocks but num_blocks is "
                    f"{cfg.num_blocks}; increase num_blocks")
        return None

    def add_request(self, request: Request, sampling_params: SamplingParams | None = None) -> int:
        """Queue ``request``; parameters left None take the checkpoint's generation
        config.  Raises ValueError when the engine cannot run it."""
        params = (self._sampling_params if sampling_params is None
                  else sampling_params.with_defaults(self._sampling_params))
        problem = self._limits_violated(request, params)
        if problem is not None:
            raise ValueError(problem)
        rid = self._next_request_id
        self._next_request_id += 1
        self.scheduler.add(Sequence(rid, [self.decoder_start_token_id], request.input_ids,
                                    params, request.pixel_values))
        return rid

    # -- stepping ------------------------------------------------------------------------

    def step(self) -> list[tuple[int, RequestOut]]:
        batch = self.scheduler.schedule()
        result = self.runner.run(batch)
        finished = self.scheduler.postprocess(batch, result)
        for rid, _ in finished:
            self.runner.clear_request(rid)
        return finished

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    def abort_request(self, request_id: int) -> bool:
        """Cancel one request between steps: its blocks and encoder pages return to
        their pools and it yields no output."""
        known = self.scheduler.abort_request(request_id)
        self.runner.clear_request(request_id)
        return known

    def abort(self) -> None:
        """Drop every waiting and running request; free blocks and encoder pages."""
        self.scheduler.reset()
        self.runner.reset()

    @torch.inference_mode()
    def generate(self, requests, sampling_params: SamplingParams | None = None,
                 use_tqdm: bool = False) -> list[RequestOut]:
        """Run ``requests`` (one or a list) to completion; one RequestOut each, in order.
        A request the engine rejects gets an empty completion.  ``use_tqdm`` shows a
        progress bar over the accepted requests."""
        batch = [requests] if isinstance(requests, Request) else list(requests)
        ids = [self._admit(r, sampling_params) for r in batch]
        bar = None
        if use_tqdm:
            from tqdm.auto import tqdm

            bar = tqdm(total=sum(i is not None for i in ids), desc="Generating", unit="req")
        try:
            finished = self._drain(bar)
        finally:
            if bar is not None:
                bar.close()
        return [finished[i] if i is not None else RequestOut(r.input_ids, [], r.pixel_values)
                for r, i in zip(batch, ids)]

    def _admit(self, request: Request, params: SamplingParams | None) -> int | None:
        """Queue one request of a ``generate`` call; None (logged) when it is rejected."""
        try:
            return self.add_request(request, params)
        except ValueError as exc:
            logger.error("request rejected: %s", exc)
            return None

    def _drain(self, bar=None) -> dict[int, RequestOut]:
        """Step until no request is left; on any exception every request is dropped and
        its blocks and pages freed before the exception propagates.  The step loop makes
        no reference cycles, so the cyclic collector is paused around it."""
        finished: dict[int, RequestOut] = {}
        paused = gc.isenabled()
        gc.disable()
        try:
            while not self.is_finished():
                done = self.step()
                finished.update(done)
                if bar is not None and done:
                    bar.update(len(done))
        except BaseException:
            self.abort()
            raise
        finally:
            if paused:
                gc.enable()
        return finished
