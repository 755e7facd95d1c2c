"""The group-plan builder (``vfl_build_group_plan``, host code, no device): its output
against a plain restatement of the definition on random beam-like tables, the
coverage property every planned launch relies on (each (row, position) a row reads
is in exactly one entry of its position, with the row's bit), and its refusals."""

import math

import numpy as np
import pytest
import torch

BS = 16


def hip():
    from vflorence_amd import hip_attn

    return hip_attn


def restated(table, lens, starts, order, slots, width, num_blocks):
    """Slot list [(first row, rows, widest, [(id, pos, tokens, cols)])] from the
    definition: tokens = how many of the block's tokens the longest listing row attends
    to."""
    out = []
    groups = len(starts) - 1
    for s in range(slots):
        if s >= groups:
            out.append((0, 0, 0, []))
            continue
        g = order[s] if order is not None else s
        r0, r1 = starts[g], starts[g + 1]
        nblk = [min(math.ceil(lens[r] / BS), width) if lens[r] > 0 else 0 for r in range(r0, r1)]
        widest = max(nblk, default=0)
        ents = []
        for p in range(widest):
            here = []
            for c in range(r1 - r0):
                if p >= nblk[c]:
                    continue
                i = int(table[r0 + c][p])
                if not 0 <= i < num_blocks:
                    continue
                toks = min(BS, min(int(lens[r0 + c]), nblk[c] * BS) - p * BS)
                for e in here:
                    if e[0] == i:
                        e[2] = max(e[2], toks)
                        e[3] |= 1 << c
                        break
                else:
                    here.append([i, p, toks, 1 << c])
            ents += [tuple(e) for e in here]
        out.append((r0, r1 - r0, widest, ents))
    return out


def decoded(plan):
    w = plan.words.numpy()
    out = []
    for s in range(plan.slots):
        rec = w[4 + s * plan.stride:]
        n = int(rec[2])
        ents = [(int(rec[4 + 2 * e]), int(np.uint32(rec[5 + 2 * e]) >> 16),
                 int((np.uint32(rec[5 + 2 * e]) >> 8) & 0xFF),
                 int(np.uint32(rec[5 + 2 * e]) & 0xFF)) for e in range(n)]
        out.append((int(rec[0]), int(rec[1]), int(rec[3]), ents))
    return int(w[0]), out


def beam_like_case(seed, groups=12, max_rows=8, max_len=200):
    rnd = np.random.default_rng(seed)
    sizes = [int(x) for x in rnd.integers(1, max_rows + 1, size=groups)]
    nxt = 0
    tables, lens = [], []
    for G in sizes:
        base = []
        for r in range(G):
            if r == 0 or rnd.random() < 0.2:
                L = int(rnd.integers(0, max_len + 1))
                nb = math.ceil(L / BS)
                t = list(range(nxt, nxt + nb))
                nxt += nb
            else:
                pt = base[int(rnd.integers(0, r))][0]
                k = int(rnd.integers(0, len(pt) + 1))
                extra = int(rnd.integers(0, 4))
                t = pt[:k] + list(range(nxt, nxt + extra))
                nxt += extra
                L = max(0, (len(t) - 1) * BS + int(rnd.integers(1, BS + 1))) if t else 0
            base.append((t, L))
        for t, L in base:
            tables.append(t)
            lens.append(L)
    width = max(1, max(len(t) for t in tables))
    table = np.full((len(tables), width), 0, dtype=np.int32)
    for i, t in enumerate(tables):
        table[i, : len(t)] = t
        if rnd.random() < 0.1 and len(t):
            table[i, int(rnd.integers(0, len(t)))] = -1 if rnd.random() < 0.5 else nxt + 50
    starts = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    return table, np.array(lens, dtype=np.int32), starts, nxt


@pytest.mark.parametrize("seed", range(8))
def test_plan_matches_its_definition(seed):
    table, lens, starts, nb = beam_like_case(seed)
    groups = len(starts) - 1
    order = np.random.default_rng(100 + seed).permutation(groups).astype(np.int32)
    use_order = seed % 2 == 1
    slots = groups + (seed % 3) * 5
    narrow = seed % 4 == 3  # a table narrower than some contexts: positions clamp
    width = max(1, table.shape[1] - 2) if narrow else table.shape[1]
    t = torch.from_numpy(np.ascontiguousarray(table[:, :width]))
    plan = hip().build_group_plan(t, torch.from_numpy(lens), torch.from_numpy(starts),
                                  group_order=torch.from_numpy(order) if use_order else None,
                                  num_slots=slots, num_blocks=nb)
    used, got = decoded(plan)
    assert used == groups and plan.slots == slots and plan.max_blocks == width
    assert plan.stride % 4 == 0 and plan.stride >= 4 + 2 * 8 * width
    want = restated(table[:, :width], lens, starts, order if use_order else None, slots, width,
                    nb)
    assert got == want


@pytest.mark.parametrize("seed", range(4))
def test_every_read_is_in_exactly_one_entry(seed):
    table, lens, starts, nb = beam_like_case(seed + 50, groups=20)
    plan = hip().build_group_plan(torch.from_numpy(table), torch.from_numpy(lens),
                                  torch.from_numpy(starts), num_blocks=nb)
    _, slots = decoded(plan)
    for (r0, n, widest, ents) in slots:
        seen = {}
        for (i, p, toks, cols) in ents:
            assert cols != 0 and cols < (1 << n) and 1 <= toks <= BS
            assert (i, p) not in seen, "an id listed twice at one position"
            seen[(i, p)] = (toks, cols)
        for c in range(n):
            L = int(lens[r0 + c])
            for p in range(math.ceil(L / BS) if L > 0 else 0):
                i = int(table[r0 + c, p])
                hits = [cols for (j, q, _, cols) in ents if q == p and (cols >> c) & 1]
                if 0 <= i < nb:
                    assert len(hits) == 1
                    toks, cols = seen[(i, p)]
                    assert cols >> c & 1 and toks >= min(BS, L - p * BS)  # covers the row
                else:
                    assert hits == []


def test_plan_refusals():
    ha = hip()
    t = torch.zeros(9, 2, dtype=torch.int32)
    lens = torch.full((9,), 20, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="at most 8 rows"):
        ha.build_group_plan(t, lens, torch.tensor([0, 9], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="group order entry out of range"):
        ha.build_group_plan(t, lens, torch.tensor([0, 4, 9], dtype=torch.int32),
                            group_order=torch.tensor([0, 2], dtype=torch.int32))
    with pytest.raises(ValueError, match="CPU int32"):
        ha.build_group_plan(t.long(), lens, torch.tensor([0, 4, 9], dtype=torch.int32))
    with pytest.raises(ValueError, match="at most"):
        ha.group_plan_stride(9, 4)
    # a stride too small for a group's distinct blocks (the library's own check)
    from vflorence_amd._lib import lib

    words = torch.zeros(4 + 8, dtype=torch.int32)
    t2 = torch.arange(8, dtype=torch.int32).reshape(4, 2)
    starts = torch.tensor([0, 4], dtype=torch.int32)
    rc = lib.vfl_build_group_plan(t2.data_ptr(), 2, 2, lens.data_ptr(), 4, starts.data_ptr(),
                                  None, 1, BS, 1 << 30, words.data_ptr(), 1, 8)
    assert rc != 0
    assert b"more distinct blocks" in lib.vfl_last_error()
