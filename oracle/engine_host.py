"""TEST INFRASTRUCTURE, NOT PRODUCT CODE: pure-Python restatement of vflorence's
host-side decode bookkeeping, the checker of the engine's native host core
(vflorence_amd/csrc/host/engine_core.cpp).

Only tests/ use this module.  It restates, step for step and in the reference's own
order of operations:

* the block manager (vflorence/engine/block_manager.py:4-73): reference counts, a FIFO
  free list (allocate from the front, free to the back, a table freed last block
  first), ``required_new_blocks`` (:28-42), ``ensure_capacity`` (:44-59), ``fork`` (:61-65);
* admission and capacity (vflorence/engine/scheduler.py:35-58);
* the step metadata formulas of ModelRunner._prepare (model_runner.py:288-305);
* greedy postprocessing (scheduler.py:69-79);
* the beam candidate merge (model_runner.py:383-410: per-row top-k plus the row's
  cumulative log-prob added in float32, a request's candidates sorted best first,
  stably, keeping max(2, 1 + n_eos) * num_beams) and the beam postprocessing
  (scheduler.py:81-127) with the reference's literal block handling: fork every live
  child from its parent, then deallocate every parent in row order.

How it is pinned (tests/test_engine_host.py): the reference's known answers for the
block budget (tests/test_engine.py:182-189, 361-380) and for the beam gate
(tests/test_beam.py:22-32), and brute-force invariants (holder counts equal table
entries, free + held = pool).
"""

from __future__ import annotations

import math
from collections import deque

import numpy as np


class Pool:
    """block_manager.py:4-73."""

    def __init__(self, num_blocks: int, block_size: int):
        self.block_size = block_size
        self.refs = [0] * num_blocks
        self.free = deque(range(num_blocks))

    def allocate(self) -> int:
        if not self.free:
            raise RuntimeError("KV cache is full; increase num_blocks")
        b = self.free.popleft()
        self.refs[b] = 1
        return b

    def required(self, rows) -> int:
        need, left = 0, {}
        for h in rows:
            i = h.cached // self.block_size
            if i >= len(h.table):
                need += 1
                continue
            b = h.table[i]
            r = left.get(b, self.refs[b])
            if r > 1:
                need += 1
                left[b] = r - 1
        return need

    def ensure(self, h):
        i = h.cached // self.block_size
        if i >= len(h.table):
            h.table.append(self.allocate())
            return None
        b = h.table[i]
        if self.refs[b] == 1:
            return None
        new = self.allocate()
        self.refs[b] -= 1
        h.table[i] = new
        return (b, new)

    def fork(self, parent, child) -> None:
        child.table = list(parent.table)
        for b in child.table:
            self.refs[b] += 1

    def free_table(self, h) -> None:
        for b in reversed(h.table):
            self.refs[b] -= 1
            if self.refs[b] == 0:
                self.free.append(b)
        h.table = []


class Hyp:
    def __init__(self, rid, tokens, req):
        self.rid, self.tokens, self.req = rid, list(tokens), req
        self.table: list[int] = []
        self.cached = 0
        self.cum = 0.0

    def child(self, token, cum):
        c = Hyp(self.rid, self.tokens + [token], self.req)
        c.cached, c.cum = self.cached, cum
        return c

    def generated(self):
        return len(self.tokens) - self.req["prompt_len"]

    def done(self):
        return self.tokens[-1] in self.req["eos"] or self.generated() >= self.req["max_tokens"]

    def score(self):
        return self.cum / (max(self.generated(), 1) ** self.req["length_penalty"])


class HostOracle:
    def __init__(self, num_blocks: int, block_size: int, max_num_seqs: int):
        self.pool = Pool(num_blocks, block_size)
        self.max_num_seqs = max_num_seqs
        self.waiting: deque[Hyp] = deque()
        self.running: list[Hyp] = []
        self.finished_beams: dict[int, list[Hyp]] = {}
        self.pairs: list[tuple[int, int]] = []

    def add(self, rid, prompt, num_beams, max_tokens, eos, length_penalty, early_stopping):
        req = dict(num_beams=num_beams, max_tokens=max_tokens, eos=set(eos),
                   length_penalty=length_penalty, early_stopping=early_stopping,
                   prompt_len=len(prompt))
        self.waiting.append(Hyp(rid, prompt, req))

    def schedule(self):
        """Returns the admitted request ids; sets ``pairs``."""
        used = sum({h.rid: h.req["num_beams"] for h in self.running}.values())
        admitted = []
        while self.waiting and used + self.waiting[0].req["num_beams"] <= self.max_num_seqs:
            h = self.waiting.popleft()
            self.running.append(h)
            used += h.req["num_beams"]
            admitted.append(h.rid)
        if self.pool.required(self.running) > len(self.pool.free):
            raise RuntimeError("KV cache is full; increase num_blocks")
        self.pairs = [p for h in self.running if (p := self.pool.ensure(h)) is not None]
        return admitted

    def metadata(self):
        """model_runner.py:288-305 per running row."""
        bs = self.pool.block_size
        rows = self.running
        return dict(
            input_ids=[h.tokens[-1] for h in rows],
            positions=[h.cached for h in rows],
            slots=[h.table[h.cached // bs] * bs + h.cached % bs for h in rows],
            lengths=[len(h.tokens) for h in rows],
            context_lens=[h.cached + 1 for h in rows],
            tables=[list(h.table) for h in rows],
            row_requests=[h.rid for h in rows],
        )

    def greedy(self, tokens):
        for h in self.running:
            h.cached += 1
        out = []
        for h, t in zip(list(self.running), tokens):
            h.tokens.append(int(t))
            if h.done():
                self.running.remove(h)
                self.pool.free_table(h)
                out.append((h.rid, h.tokens[h.req["prompt_len"]:]))
        return out

    def beam(self, scores: np.ndarray, ids: np.ndarray):
        """model_runner.py:383-410 (merge) then scheduler.py:81-127 (``walk``)."""
        cands: dict[int, list] = {}
        for r, h in enumerate(self.running):
            vals = scores[r].astype(np.float32) + np.float32(h.cum)
            cands.setdefault(h.rid, []).extend(
                (h, int(t), float(v)) for t, v in zip(ids[r].tolist(), vals))
        for cs in cands.values():
            cs.sort(key=lambda c: c[2], reverse=True)
            del cs[max(2, 1 + len(cs[0][0].req["eos"])) * cs[0][0].req["num_beams"]:]
        return self.walk(cands)

    def walk(self, cands: dict[int, list]):
        """scheduler.py:81-127 over each request's candidates (parent, token, cum),
        taken in the given order."""
        rows = self.running
        for h in rows:
            h.cached += 1
        out = []
        children = []
        for rid, cs in cands.items():
            req = cs[0][0].req
            nb = req["num_beams"]
            done = self.finished_beams.setdefault(rid, [])
            live = []
            for rank, (parent, tok, cum) in enumerate(cs):
                if rank >= nb and len(live) >= nb:
                    break
                c = parent.child(tok, cum)
                if c.done():
                    if rank < nb:
                        done.append(c)
                elif len(live) < nb:
                    live.append((parent, c))
            done.sort(key=lambda c: c.score(), reverse=True)
            del done[nb:]
            best = max((c.score() for _, c in live), default=-math.inf)
            if not live or (len(done) >= nb and (req["early_stopping"]
                                                 or done[-1].score() >= best)):
                self.finished_beams.pop(rid, None)
                out.append((rid, done[0].tokens[req["prompt_len"]:]))
            else:
                for parent, c in live:
                    self.pool.fork(parent, c)
                    children.append(c)
        for h in rows:
            self.pool.free_table(h)
        self.running = children
        return out
