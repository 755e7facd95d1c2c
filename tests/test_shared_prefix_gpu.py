"""Self-attention over row groups whose rows keep their own block tables
(VFL_GROUP_OWN_TABLES): the beams of a request, whose copy-on-write forks share
prefix blocks, are served by one workgroup that reads every distinct block once.

Checks: with one wave the grouped kernel is bit-identical to the one-row kernel (every
row still folds exactly its own blocks, in order); any partition of the rows gives the
same results; every wave count matches the float64 oracle; the fused KV write equals
reshape_and_cache + attention bit for bit, also on beam-search block tables produced by
the real BlockManager; shared partial blocks with stale NaN tails, invalid ids,
zero-length rows and clamped tables behave as in the one-row kernel.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"
BS = 16
TOL = {
    torch.float32: dict(rtol=1e-5, atol=1e-6),
    torch.bfloat16: dict(rtol=0.0, atol=2e-2),
    torch.float16: dict(rtol=0.0, atol=2e-2),
}


def hip():
    from vflorence_amd import hip_attn

    return hip_attn


def bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


def prefix_tree_case(group_sizes, seed, H=16, D=64, dtype=torch.bfloat16, max_len=300):
    """Rows in groups; within a group each row after the first copies a random prefix of
    an earlier row's table (whole blocks, never that row's last one) and appends private
    blocks, so rows share prefixes of different lengths and every last block is private
    (the block manager's invariant).  Slots are position L-1 of each row."""
    g = torch.Generator().manual_seed(seed)
    rnd = np.random.default_rng(seed)
    next_block = 0
    tables, lens = [], []
    for G in group_sizes:
        group = []
        for r in range(G):
            if r == 0 or rnd.random() < 0.15:
                L = int(rnd.integers(1, max_len + 1))
                nb = math.ceil(L / BS)
                t = list(range(next_block, next_block + nb))
                next_block += nb
            else:
                pt, _ = group[int(rnd.integers(0, r))]
                s = int(rnd.integers(0, len(pt)))  # shared whole blocks, < len(pt)
                extra = int(rnd.integers(1, 5))
                t = pt[:s] + list(range(next_block, next_block + extra))
                next_block += extra
                L = (len(t) - 1) * BS + int(rnd.integers(1, BS + 1))
            group.append((t, L))
        for t, L in group:
            tables.append(t)
            lens.append(L)
    NB = next_block + 5
    perm = torch.randperm(NB, generator=g)
    width = max(len(t) for t in tables)
    table = torch.zeros(len(tables), width, dtype=torch.int32)
    for i, t in enumerate(tables):
        table[i, : len(t)] = perm[torch.tensor(t)].to(torch.int32)
    N = len(lens)
    L = torch.tensor(lens, dtype=torch.int32)
    slots = torch.tensor([int(table[i, (lens[i] - 1) // BS]) * BS + (lens[i] - 1) % BS
                          for i in range(N)], dtype=torch.int64)
    fused = torch.randn(N, 3 * H * D, generator=g).to(dtype)
    kc = torch.randn(NB, H, BS, D, generator=g).to(dtype)
    vc = torch.randn(NB, H, BS, D, generator=g).to(dtype)
    starts = torch.tensor(np.concatenate([[0], np.cumsum(group_sizes)]), dtype=torch.int32)
    return fused, kc, vc, L, table, slots, starts


def metadata(N, H, D, dtype, starts=None, waves=0, fuse=False, lens=None, gmax=8):
    hip_attn = hip()
    order = None
    if starts is not None and lens is not None:
        firsts = [max(lens[starts[i]:starts[i + 1]].tolist(), default=0)
                  for i in range(len(starts) - 1)]
        order = torch.tensor(hip_attn.longest_first(firsts), dtype=torch.int32, device=DEV)
    return hip_attn.get_scheduler_metadata(
        num_reqs=N, num_heads=H, num_kv_heads=H, head_dim=D, dtype=dtype, block_size=BS,
        group_start=None if starts is None else starts.to(DEV), group_order=order,
        max_group_size=gmax if starts is not None else 1, waves_per_workgroup=waves,
        fuse_kv_write=fuse, own_tables=starts is not None)


def attend(fused, kc, vc, L, table, starts, waves, H=16, D=64):
    """Two-step-free attention (no KV write) over the given caches."""
    hip_attn = hip()
    N = fused.shape[0]
    q = fused.to(DEV)[:, : H * D].reshape(N, H, D)
    kd, vd = kc.to(DEV), vc.to(DEV)
    out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
    sm = metadata(N, H, D, q.dtype, starts, waves, lens=L)
    hip_attn.attention_with_kv_cache(q, kd, vd, out, None, L.to(DEV), scale=D**-0.5,
                                     block_table=table.to(DEV), scheduler_metadata=sm)
    torch.cuda.synchronize()
    return out.cpu()


def write_and_attend(fused, kc, vc, L, table, slots, starts, waves, fuse, H=16, D=64):
    hip_attn = hip()
    N = fused.shape[0]
    f = fused.to(DEV)
    q, k, v = (t.reshape(N, H, D) for t in f.chunk(3, dim=-1))
    kd, vd = kc.to(DEV), vc.to(DEV)
    out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
    sm = metadata(N, H, D, q.dtype, starts, waves, fuse=fuse, lens=L)
    if fuse:
        hip_attn.self_attention_with_kv_write(q, k, v, kd, vd, out, L.to(DEV), slots.to(DEV),
                                              scale=D**-0.5, block_table=table.to(DEV),
                                              scheduler_metadata=sm)
    else:
        hip_attn.reshape_and_cache(k, v, kd, vd, slots.to(DEV))
        hip_attn.attention_with_kv_cache(q, kd, vd, out, None, L.to(DEV), scale=D**-0.5,
                                         block_table=table.to(DEV), scheduler_metadata=sm)
    torch.cuda.synchronize()
    return out.cpu(), kd.cpu(), vd.cpu()


def oracle_check(out, fused, kc, vc, L, table, H=16, D=64):
    q = fused[:, : H * D].reshape(len(L), H, D)
    want = orc.paged_attention(q.double().numpy(), kc.double().numpy(),
                               hip().v_cache_logical(vc).double().numpy(), L.numpy(),
                               table.numpy(), D**-0.5)
    np.testing.assert_allclose(out.double().numpy(), want, **TOL[fused.dtype])


GROUPS = [[4] * 8, [1, 2, 3, 4, 5, 6, 7, 8], [8, 8], [3] * 7, [2, 5, 1, 7]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", range(len(GROUPS)))
def test_one_wave_grouped_is_bit_identical_to_one_row_kernel(dtype, case):
    fused, kc, vc, L, table, _, starts = prefix_tree_case(GROUPS[case], seed=case, dtype=dtype)
    grouped = attend(fused, kc, vc, L, table, starts, waves=1)
    single = attend(fused, kc, vc, L, table, None, waves=1)
    assert np.array_equal(bits(grouped), bits(single))
    oracle_check(grouped, fused, kc, vc, L, table)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("waves", [1, 2, 4, 8, 0])
def test_grouped_matches_oracle(dtype, head_dim, waves):
    fused, kc, vc, L, table, _, starts = prefix_tree_case([4, 4, 3, 8, 1, 5], seed=waves + 7,
                                                          dtype=dtype, D=head_dim, max_len=700)
    out = attend(fused, kc, vc, L, table, starts, waves, D=head_dim)
    oracle_check(out, fused, kc, vc, L, table, D=head_dim)


def test_any_partition_gives_the_same_rows():
    """Grouping only shares loads: cutting the same rows into other groups (including
    groups of rows that share nothing) changes no output bit with one wave."""
    fused, kc, vc, L, table, _, starts = prefix_tree_case([4] * 6, seed=3)
    ref = attend(fused, kc, vc, L, table, starts, waves=1)
    # the last cut has empty groups (a padded launch grid): they write nothing
    for cut in ([0, 3, 5, 11, 12, 20, 24], [0, 8, 16, 24], list(range(0, 25, 2)),
                [0, 4, 4, 8, 12, 20, 24, 24, 24]):
        other = attend(fused, kc, vc, L, table, torch.tensor(cut, dtype=torch.int32), waves=1)
        assert np.array_equal(bits(other), bits(ref)), cut


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("waves", [1, 2, 4])
def test_fused_grouped_equals_two_steps(dtype, waves):
    fused, kc, vc, L, table, slots, starts = prefix_tree_case([4, 4, 2, 8, 3, 1], seed=11 + waves,
                                                              dtype=dtype)
    o2, k2, v2 = write_and_attend(fused, kc, vc, L, table, slots, starts, waves, fuse=False)
    o1, k1, v1 = write_and_attend(fused, kc, vc, L, table, slots, starts, waves, fuse=True)
    assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
    assert np.array_equal(bits(o1), bits(o2))
    oracle_check(o1, fused, k1, v1, L, table)
    if waves == 1:  # and the grouped fused launch equals the one-row fused launch
        o0, k0, v0 = write_and_attend(fused, kc, vc, L, table, slots, None, 1, fuse=True)
        assert np.array_equal(bits(o0), bits(o1))
        assert np.array_equal(bits(k0), bits(k1)) and np.array_equal(bits(v0), bits(v1))


def test_fused_grouped_slot_outside_the_context():
    fused, kc, vc, L, table, slots, starts = prefix_tree_case([4, 3], seed=5)
    used = set(table.flatten().tolist())
    free = [b for b in range(kc.shape[0]) if b not in used]
    slots = slots.clone()
    slots[1] = free[0] * BS + 7  # a block nobody reads: written without substitution
    slots[5] = -1  # padding: not written
    o2, k2, v2 = write_and_attend(fused, kc, vc, L, table, slots, starts, 2, fuse=False)
    o1, k1, v1 = write_and_attend(fused, kc, vc, L, table, slots, starts, 2, fuse=True)
    assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
    assert np.array_equal(bits(o1), bits(o2))


def test_shared_partial_block_with_stale_nan_tail():
    """Two rows of a group list the same partial last block with different lengths (a
    fork before its copy-on-write); tokens past the longer length hold NaN."""
    hip_attn = hip()
    H, D = 16, 64
    g = torch.Generator().manual_seed(2)
    kc = torch.randn(8, H, BS, D, generator=g).to(torch.bfloat16)
    vlog = torch.randn(8, H, BS, D, generator=g).to(torch.bfloat16)
    kc[3, :, 9:] = float("nan")
    vlog[3, :, 9:] = float("nan")
    vc = hip_attn.v_cache_from_logical(vlog)
    table = torch.tensor([[1, 3], [1, 3], [5, 3], [1, 6]], dtype=torch.int32)
    L = torch.tensor([25, 23, 19, 32], dtype=torch.int32)  # block 3 holds 9, 7, 3 tokens
    fused = torch.randn(4, 3 * H * D, generator=g).to(torch.bfloat16)
    starts = torch.tensor([0, 4], dtype=torch.int32)
    for waves in (1, 2):
        out = attend(fused, kc, vc, L, table, starts, waves)
        assert torch.isfinite(out.float()).all()
        oracle_check(out, fused, kc, vc, L, table)
    assert np.array_equal(bits(attend(fused, kc, vc, L, table, starts, 1)),
                          bits(attend(fused, kc, vc, L, table, None, 1)))


def test_invalid_ids_zero_lengths_and_clamped_tables():
    fused, kc, vc, L, table, _, starts = prefix_tree_case([4, 4, 4], seed=9)
    L = L.clone()
    table = table.clone()
    L[2] = 0  # zero-length row inside a group
    table[5, 0] = -3  # invalid ids contribute nothing
    table[6, 1] = kc.shape[0] + 10
    for waves in (1, 4):
        grouped = attend(fused, kc, vc, L, table, starts, waves)
        assert (grouped[2] == 0).all()
        if waves == 1:
            assert np.array_equal(bits(grouped), bits(attend(fused, kc, vc, L, table, None, 1)))
    # a table narrower than the contexts: both kernels clamp to its width
    narrow = table[:, :3].contiguous()
    a = attend(fused, kc, vc, L, narrow, starts, 1)
    b = attend(fused, kc, vc, L, narrow, None, 1)
    assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("beams", [4, 3])
def test_beam_search_tables_fused_grouped_equals_two_steps(beams):
    """Block tables of a beam search driven through the BlockManager (forks share
    blocks, copy-on-write makes each row's last block private): at several steps, the
    fused grouped launch equals the two steps, and the oracle."""
    from vflorence_amd.workloads import beam_decode_schedule

    R, H, D = 6, 16, 64
    plans = beam_decode_schedule(num_requests=R, beams=beams, steps=70, cow_fraction=0.2,
                                 seed=beams)
    g = torch.Generator().manual_seed(beams)
    NB = 1 + max(max(max(t) for t in p.block_tables) for p in plans)
    kc = torch.randn(NB, H, BS, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(NB, H, BS, D, generator=g).to(torch.bfloat16)
    starts = torch.arange(0, R * beams + 1, beams, dtype=torch.int32)
    shared = 0
    for step in (0, 1, 15, 16, 17, 40, 69):
        p = plans[step]
        N = len(p.context_lens)
        width = max(len(t) for t in p.block_tables)
        table = torch.zeros(N, width, dtype=torch.int32)
        for i, t in enumerate(p.block_tables):
            table[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
        listed = [b for t in p.block_tables for b in t]
        shared += len(listed) - len(set(listed))
        L = torch.tensor(p.context_lens, dtype=torch.int32)
        slots = torch.tensor(p.slot_mapping, dtype=torch.int64)
        fused = torch.randn(N, 3 * H * D, generator=g).to(torch.bfloat16)
        for waves in (1, 2):
            o2, k2, v2 = write_and_attend(fused, kc, vc, L, table, slots, starts, waves, False)
            o1, k1, v1 = write_and_attend(fused, kc, vc, L, table, slots, starts, waves, True)
            assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
            assert np.array_equal(bits(o1), bits(o2))
        oracle_check(o1, fused, k1, v1, L, table)
    assert shared > 0  # the schedule did share blocks between beams
