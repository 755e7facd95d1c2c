"""The group-plan builder (``vfl_build_group_plan``, host code, no device): its output
against a plain restatement of the definition on random beam-like tables, the
coverage property every planned launch relies on (each (row, position) a row reads
is in exactly one entry of its position, with the row's bit), and its refusals; the
copy-on-write fold (``vfl_fold_plan_copies``) on the block tables and copy pairs of a
beam search through the BlockManager, and its refusals (plan unchanged)."""

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


HEADER, ENTRY = 4, 2  # words of a slot's header, of an entry


def decoded(plan, copies=False):
    """(used slots, [(first row, rows, widest, entries)]); an entry is (id, position,
    tokens, rows) -- with ``copies``, plus whether it is flagged as a fork block whose id
    is its copy source.  Without ``copies`` no entry may be flagged."""
    w = plan.words.numpy()
    out = []
    for s in range(plan.slots):
        rec = w[4 + s * plan.stride:]
        n = int(rec[2])
        ents = []
        for e in range(n):
            x = rec[HEADER + ENTRY * e: HEADER + ENTRY * (e + 1)]
            word = np.uint32(x[1])
            flagged = bool(word >> 31)
            ent = (int(x[0]), int((word >> 16) & 0x7FFF), int((word >> 8) & 0xFF),
                   int(word & 0xFF))
            if copies:
                ent += (flagged,)
            else:
                assert not flagged
            ents.append(ent)
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
    assert plan.stride % 4 == 0 and plan.stride >= HEADER + ENTRY * 8 * width
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

    words = torch.zeros(4 + HEADER + 4, dtype=torch.int32)  # room for two entries
    t2 = torch.arange(8, dtype=torch.int32).reshape(4, 2)
    starts = torch.tensor([0, 4], dtype=torch.int32)
    rc = lib.vfl_build_group_plan(t2.data_ptr(), 2, 2, lens.data_ptr(), 4, starts.data_ptr(),
                                  None, 1, BS, 1 << 30, words.data_ptr(), 1, HEADER + 4)
    assert rc != 0
    assert b"more distinct blocks" in lib.vfl_last_error()


def beam_step_plan(step, beams=4, requests=5):
    """A beam-search step's tables, lengths and copy pairs (BlockManager forks) and its
    group plan, one group per request."""
    from vflorence_amd.workloads import beam_decode_schedule

    p = beam_decode_schedule(num_requests=requests, beams=beams, steps=step + 1,
                             cow_fraction=0.3, seed=beams + step)[step]
    n = len(p.context_lens)
    width = max(len(t) for t in p.block_tables)
    table = torch.zeros(n, width, dtype=torch.int32)
    for i, t in enumerate(p.block_tables):
        table[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    nb = 1 + int(table.max())
    starts = torch.arange(0, n + 1, beams, dtype=torch.int32)
    plan = hip().build_group_plan(table, torch.tensor(p.context_lens, dtype=torch.int32),
                                  starts, num_blocks=nb)
    return p, table, nb, plan


@pytest.mark.parametrize("step", [17, 30, 45])
def test_fold_marks_each_copy_destination_with_its_source(step):
    p, table, nb, plan = beam_step_plan(step)
    assert p.copies, "the schedule forks at this step"
    before = decoded(plan)
    src = [a for a, _ in p.copies]
    dst = [b for _, b in p.copies]
    assert hip().fold_plan_copies(plan, src, dst, num_blocks=nb)
    used, slots = decoded(plan, copies=True)
    want = dict(zip(dst, src))
    found = {}
    for (r0, n, widest, ents), (_, _, _, plain) in zip(slots, before[1]):
        for (i, pos, toks, cols, flagged), (i0, pos0, toks0, cols0) in zip(ents, plain):
            assert (pos, toks, cols) == (pos0, toks0, cols0)  # only ids and flags change
            if i0 in want:
                # the fork's block (one row's, at its last position) names its source
                assert flagged and i == want[i0] and cols & (cols - 1) == 0
                r = r0 + cols.bit_length() - 1
                assert pos == (p.context_lens[r] - 1) // BS
                assert table[r, pos] == i0
                found[i0] = i
            else:
                assert not flagged and i == i0
    assert found == want


def test_fold_refusals_leave_the_plan_unchanged():
    p, table, nb, plan = beam_step_plan(30)
    src = [a for a, _ in p.copies]
    dst = [b for _, b in p.copies]
    from vflorence_amd._lib import lib

    words = plan.words.clone()
    # a block several rows of a group read at one position (a shared prefix block)
    shared = next(i for (_, _, _, ents) in decoded(plan)[1] for (i, _, _, cols) in ents
                  if cols & (cols - 1))
    absent = nb + 5
    cases = [
        (src + [src[0]], dst + [absent], nb + 10, b"not a block of the plan"),
        (src + [src[0]], dst + [dst[0]], nb, b"destination of two copies"),
        (src + [dst[0]], dst + [absent], nb + 10, b"both a copy source and a destination"),
        (src, dst[:-1] + [nb], nb, b"out of range"),
        (src + [src[0]], dst + [shared], nb, b"listed by several rows"),
    ]
    for s, d, n, why in cases:
        assert not hip().fold_plan_copies(plan, s, d, num_blocks=n), (s, d)
        assert why in lib.vfl_last_error()
        assert torch.equal(plan.words, words)
    assert hip().fold_plan_copies(plan, [], [], num_blocks=nb)
    assert torch.equal(plan.words, words)
    # one row, two private blocks: only the last one, where the new token goes, can be
    # its fork block (the fused launch stores the copy to the block of the row's slot)
    one = hip().build_group_plan(torch.tensor([[5, 6]], dtype=torch.int32),
                                 torch.tensor([20], dtype=torch.int32),
                                 torch.tensor([0, 1], dtype=torch.int32), num_blocks=10)
    before = one.words.clone()
    for s_, d_ in (([1, 2], [5, 6]), ([1], [5])):
        assert not hip().fold_plan_copies(one, s_, d_, num_blocks=10)
        assert b"not its row's last block" in lib.vfl_last_error()
        assert torch.equal(one.words, before)
    assert hip().fold_plan_copies(one, [2], [6], num_blocks=10)
    assert decoded(one, copies=True)[1][0][3] == [(5, 0, 16, 1, False), (2, 1, 4, 1, True)]


def restated_descriptors(table, lens, starts, order, slots, width):
    out = []
    groups = len(starts) - 1
    for s in range(slots):
        if s >= groups:
            out.append([0, 0, 0, 0])
            continue
        g = order[s] if order is not None else s
        r0, r1 = int(starts[g]), int(starts[g + 1])
        if r1 == r0:
            out.append([0, 0, 0, 0])
            continue
        out.append([r0, r1 - r0, int(lens[r0]), 0] + [int(x) for x in table[r0, :width]])
    return out


@pytest.mark.parametrize("seed", range(4))
def test_slot_descriptors_match_their_definition(seed):
    """Slot descriptors of shared-table groups (cross-attention beams): per dispatch slot,
    the group's first row, rows, length and the first row's table row; empty slots and
    empty groups zero."""
    rnd = np.random.default_rng(seed)
    sizes = [int(x) for x in rnd.integers(0, 9, size=10)]
    starts = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    rows = int(starts[-1])
    width = int(rnd.integers(1, 70))
    table = rnd.integers(0, 5000, size=(rows, width)).astype(np.int32)
    lens = rnd.integers(0, width * BS + 1, size=rows).astype(np.int32)
    order = rnd.permutation(len(sizes)).astype(np.int32) if seed % 2 else None
    slots = len(sizes) + seed
    d = hip().build_slot_descriptors(
        torch.from_numpy(table), torch.from_numpy(lens), torch.from_numpy(starts),
        group_order=None if order is None else torch.from_numpy(order), num_slots=slots)
    assert d.stride % 4 == 0 and d.stride >= 4 + width and d.slots == slots
    w = d.words.numpy()
    got = []
    for s in range(slots):
        rec = w[s * d.stride: (s + 1) * d.stride]
        got.append([int(x) for x in rec[:4]] + ([int(x) for x in rec[4: 4 + width]]
                                                if rec[1] else []))
    assert got == restated_descriptors(table, lens, starts, order, slots, width)


def test_slot_descriptor_refusals():
    ha = hip()
    t = torch.zeros(4, 2, dtype=torch.int32)
    lens = torch.full((4,), 20, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="group order entry out of range"):
        ha.build_slot_descriptors(t, lens, torch.tensor([0, 2, 4], dtype=torch.int32),
                                  group_order=torch.tensor([0, 5], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="group rows out of range"):
        ha.build_slot_descriptors(t, lens, torch.tensor([0, 2, 9], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="bad sizes"):  # fewer slots than groups
        ha.build_slot_descriptors(t, lens, torch.tensor([0, 2, 4], dtype=torch.int32),
                                  num_slots=1)
