"""Continuous batching and beam bookkeeping on the host.

Same policy as vflorence/engine/scheduler.py:8-127, because block tables, copy pairs
and beam selection must come out exactly as the reference's for token parity:

* admission is FIFO while the running requests' beam counts fit ``max_num_seqs``;
* before a step every running sequence gets a writable slot
  (``BlockManager.ensure_capacity``), and the step fails if the pool cannot cover it;
* greedy steps append each sampled token and retire finished sequences;
* beam steps walk each request's candidates best first: a stopped candidate becomes a
  finished hypothesis only if it ranks within the top ``num_beams``, live ones fill up
  to ``num_beams`` running children, finished hypotheses are kept by length-penalised
  score, and the request ends when no live beam remains or the early-stopping test
  passes.  Children share their parent's blocks (``fork``) and every parent is retired,
  so a request's beams stay adjacent in ``running``, which the cross-attention beam
  groups rely on.
"""

from __future__ import annotations

from collections import defaultdict, deque
from operator import attrgetter

from .block_manager import BlockManager
from .sequence import RequestOut, Sequence

_score = attrgetter("score")


class Scheduler:
    def __init__(self, config):
        self.max_num_seqs = config.max_num_seqs
        self.block_manager = BlockManager(config.num_blocks, config.block_size)
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []
        self._finished_beams: dict[int, list[Sequence]] = defaultdict(list)

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def reset(self) -> None:
        self.waiting.clear()
        self.running.clear()
        self._finished_beams.clear()
        self.block_manager.reset()

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def remove(self, seq: Sequence) -> None:
        self.running.remove(seq)
        self.block_manager.deallocate(seq)

    def schedule(self) -> tuple[list[Sequence], list[tuple[int, int]]]:
        """Admit waiting requests, give every running sequence a slot; return the step's
        sequences and its copy-on-write pairs."""
        if self.waiting:  # admission needs the running requests' beam counts
            beams = {seq.request_id: seq.sampling_params.num_beams for seq in self.running}
            used = sum(beams.values())
            while (self.waiting
                   and used + self.waiting[0].sampling_params.num_beams <= self.max_num_seqs):
                seq = self.waiting.popleft()
                self.running.append(seq)
                used += seq.sampling_params.num_beams
        seqs = list(self.running)
        bm = self.block_manager
        if bm.required_new_blocks(seqs) > bm.num_free_blocks:
            raise RuntimeError("KV cache is full; increase num_blocks")
        copies = []
        for seq in seqs:
            pair = bm.ensure_capacity(seq)
            if pair is not None:
                copies.append(pair)
        return seqs, copies

    def postprocess(self, seqs: list[Sequence], sample_out) -> list[tuple[int, RequestOut]]:
        for seq in seqs:
            seq.num_cached_tokens += 1
        if seqs and seqs[0].sampling_params.num_beams > 1:
            return self._postprocess_beam(seqs, sample_out)
        return self._postprocess_greedy(seqs, sample_out)

    def _postprocess_greedy(self, seqs, token_ids) -> list[tuple[int, RequestOut]]:
        outputs = []
        for seq, token in zip(seqs, token_ids):
            seq.append_token(token)
            if seq.is_finished:
                self.remove(seq)
                outputs.append((seq.request_id, seq.to_output()))
        return outputs

    def _postprocess_beam(self, seqs, candidates_by_request) -> list[tuple[int, RequestOut]]:
        outputs = []
        eos_of: dict[int, set[int]] = {}
        for request_id, candidates in candidates_by_request.items():
            sp = candidates[0][0].sampling_params
            num_beams = sp.num_beams
            eos = eos_of.get(id(sp))
            if eos is None:
                eos = eos_of[id(sp)] = sp.eos_ids()
            max_tokens = sp.max_tokens
            finished = self._finished_beams[request_id]
            live: list[tuple[Sequence, Sequence]] = []
            for rank, (parent, token, cum_logprob) in enumerate(candidates):
                if rank >= num_beams and len(live) >= num_beams:
                    break
                # Sequence.is_finished of the child (the parent's tokens plus ``token``),
                # decided before the child exists: only kept candidates are forked
                generated = len(parent.token_ids) + 1 - len(parent.decoder_token_ids)
                if token in eos or generated >= max_tokens:
                    if rank < num_beams:
                        finished.append(parent.fork(token, cum_logprob))
                elif len(live) < num_beams:
                    live.append((parent, parent.fork(token, cum_logprob)))
            if finished:
                finished.sort(key=_score, reverse=True)
                del finished[num_beams:]
            # the early-stopping test compares with the best live beam only when the
            # finished list is full (the live scores are not needed otherwise)
            done = not live or (len(finished) >= num_beams and (
                sp.early_stopping
                or finished[-1].score >= max(child.score for _, child in live)))
            if done:
                self._finished_beams.pop(request_id, None)
                outputs.append((request_id, finished[0].to_output()))
            else:
                # A parent's first live child takes over its block table; further
                # children fork from that child.  The reference forks every child and
                # then deallocates every parent (scheduler.py:120-126): per block that
                # is +1 per child and -1 per parent, so the reference counts, the blocks
                # freed below and their order come out the same.
                holder: dict[int, Sequence] = {}
                for parent, child in live:
                    owner = holder.get(id(parent))
                    if owner is None:
                        child.block_table = parent.block_table
                        parent.block_table = []
                        holder[id(parent)] = child
                    else:
                        self.block_manager.fork(owner, child)
                    self.running.append(child)
        # retire every parent: blocks freed in step order, one pass over ``running``
        for seq in seqs:
            self.block_manager.deallocate(seq)
        retired = set(map(id, seqs))
        self.running = [s for s in self.running if id(s) not in retired]
        return outputs
