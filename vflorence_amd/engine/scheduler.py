"""Continuous batching on the native host core (vflorence/engine/scheduler.py:8-127).

The running hypotheses, their block tables and the beam bookkeeping live in the
engine core (``engine/core.py``, include/vfl_engine.h); this class submits requests
to it, starts steps, feeds each step's sampled tokens or beam candidates back and
turns finished requests into ``RequestOut``.  The policy is the reference's:

* admission is FIFO while the running requests' beams plus the next request's fit
  ``max_num_seqs``;
* a step first makes every running row's next position writable (a fresh block, or
  a private copy of a block other rows still hold), and fails with "KV cache is full"
  if the pool cannot cover that;
* greedy steps append each row's token and retire finished rows;
* beam steps keep each request's best live continuations, collect finished
  hypotheses by length-penalised score and end the request when no continuation lives
  or the early-stopping test passes; a request's beams stay adjacent.
"""

from __future__ import annotations

from collections import deque

from .block_manager import BlockManager
from .core import EngineCore, RowView
from .sequence import RequestOut, Sequence


class StepBatch:
    """A scheduled step: how many rows run and how many copy-on-write pairs precede
    them, the requests admitted this step (their encoders run first), the shared
    sampling parameters, and the core that holds the rows."""

    __slots__ = ("core", "num_rows", "num_pairs", "fresh", "sampling_params")

    def __init__(self, core, num_rows, num_pairs, fresh, sampling_params):
        self.core = core
        self.num_rows = num_rows
        self.num_pairs = num_pairs
        self.fresh = fresh
        self.sampling_params = sampling_params


class Scheduler:
    def __init__(self, config):
        self.max_num_seqs = config.max_num_seqs
        self.core = EngineCore(config.num_blocks, config.block_size, config.max_num_seqs)
        self.block_manager = BlockManager.view(self.core.pool)
        self.waiting: deque[Sequence] = deque()
        self._requests: dict[int, Sequence] = {}  # submitted, not yet finished

    def is_finished(self) -> bool:
        return not self.waiting and self.core.num_running == 0

    def reset(self) -> None:
        """Drop every request and free every block (after an aborted step)."""
        self.core.reset()
        self.waiting.clear()
        self._requests.clear()

    def add(self, seq: Sequence) -> None:
        p = seq.sampling_params
        self.core.add_request(seq.request_id, seq.token_ids, p.num_beams, p.max_tokens,
                              sorted(p.eos_ids()), p.length_penalty, p.early_stopping)
        self.waiting.append(seq)
        self._requests[seq.request_id] = seq

    def active_params(self):
        """The sampling parameters the submitted requests share (None when idle)."""
        for seq in self._requests.values():
            return seq.sampling_params
        return None

    @property
    def num_running(self) -> int:
        """Running rows (hypotheses)."""
        return self.core.num_running

    @property
    def running(self) -> list[RowView]:
        """Snapshots of the running rows, in row order."""
        return self.core.rows()

    @property
    def num_pending_beams(self) -> int:
        """Requests holding finished beam hypotheses while other beams still run."""
        return self.core.num_pending_beams

    def abort_request(self, request_id: int) -> bool:
        """Drop a waiting or running request between steps (its blocks are freed, it is
        not reported as finished); False if it is not known."""
        known = self.core.abort_request(request_id)
        self.waiting = deque(s for s in self.waiting if s.request_id != request_id)
        return self._requests.pop(request_id, None) is not None or known

    def schedule(self) -> StepBatch:
        admitted = self.core.schedule()
        fresh = []
        for rid in admitted:
            seq = self.waiting.popleft()
            if seq.request_id != rid:
                raise RuntimeError(f"admission order diverged: {seq.request_id} != {rid}")
            fresh.append(seq)
        return StepBatch(self.core, self.core.num_rows, self.core.num_pairs, fresh,
                         self.active_params())

    def postprocess(self, batch: StepBatch, sample_out) -> list[tuple[int, RequestOut]]:
        """Feed the step's result back: greedy, one token per row; beam search, each
        row's best ``k`` (scores, token ids) as two [rows, k] arrays."""
        if batch.num_rows == 0:
            return []
        if batch.sampling_params.num_beams > 1:
            scores, ids = sample_out
            self.core.beam_update(scores, ids)
        else:
            self.core.greedy_update(sample_out)
        outputs = []
        for rid, completion in self.core.finished():
            seq = self._requests.pop(rid)
            outputs.append((rid, RequestOut(seq.encoder_token_ids, completion, seq.pixel_values)))
        return outputs
