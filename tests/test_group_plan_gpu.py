"""Self-attention over own-table row groups driven by a group plan (the per-step
schedule ``build_group_plan`` makes on the host; vflorence/engine/model_runner.py:308-319
is where the reference makes its per-step scheduler metadata).

Checks: with one wave the planned launch is bit-identical to the table-walking grouped
launch and to the one-row kernel (each row folds exactly its own blocks, in order);
every wave count matches the float64 oracle, including groups whose plans hold more
than one 64-entry window; the fused KV write equals reshape_and_cache + attention bit
for bit (and the table-walking fused launch at one wave), also for slots outside the
context and padding rows, and on beam-search tables from the BlockManager; a plan
with a dispatch order and padded empty slots writes exactly the rows of its groups;
invalid ids, zero lengths, stale NaN tails and clamped tables behave as in the other
kernels.
"""

import numpy as np
import pytest
import torch

from test_shared_prefix_gpu import (BS, DEV, attend, bits, oracle_check, prefix_tree_case,
                                    write_and_attend)

pytestmark = pytest.mark.gpu


def hip():
    from vflorence_amd import hip_attn

    return hip_attn


def plan_for(table, L, starts, num_blocks, order=None, slots=None, gmax=8):
    return hip().build_group_plan(table, L, starts, group_order=order, num_slots=slots,
                                  max_group_size=gmax, block_size=BS,
                                  num_blocks=num_blocks).to(DEV)


def planned_metadata(N, H, D, dtype, starts, plan, waves, fuse, order=None, gmax=8):
    return hip().get_scheduler_metadata(
        num_reqs=N, num_heads=H, num_kv_heads=H, head_dim=D, dtype=dtype, block_size=BS,
        group_start=starts.to(DEV), group_order=None if order is None else order.to(DEV),
        max_group_size=gmax, waves_per_workgroup=waves, fuse_kv_write=fuse, own_tables=True,
        group_plan=plan)


def planned_attend(fused, kc, vc, L, table, starts, waves, H=16, D=64, order=None, slots=None,
                   out=None):
    hip_attn = hip()
    N = fused.shape[0]
    q = fused.to(DEV)[:, : H * D].reshape(N, H, D)
    kd, vd = kc.to(DEV), vc.to(DEV)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
    plan = plan_for(table, L, starts, kc.shape[0], order=order, slots=slots)
    sm = planned_metadata(N, H, D, q.dtype, starts, plan, waves, False, order=order)
    hip_attn.attention_with_kv_cache(q, kd, vd, out, None, L.to(DEV), scale=D**-0.5,
                                     block_table=table.to(DEV), scheduler_metadata=sm)
    torch.cuda.synchronize()
    return out.cpu()


def planned_write_and_attend(fused, kc, vc, L, table, slots, starts, waves, fuse, H=16, D=64):
    hip_attn = hip()
    N = fused.shape[0]
    f = fused.to(DEV)
    q, k, v = (t.reshape(N, H, D) for t in f.chunk(3, dim=-1))
    kd, vd = kc.to(DEV), vc.to(DEV)
    out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
    plan = plan_for(table, L, starts, kc.shape[0])
    sm = planned_metadata(N, H, D, q.dtype, starts, plan, waves, fuse)
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


GROUPS = [[4] * 8, [1, 2, 3, 4, 5, 6, 7, 8], [8, 8], [3] * 7, [2, 5, 1, 7]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", range(len(GROUPS)))
def test_one_wave_planned_is_bit_identical_to_table_walk_and_one_row(dtype, case):
    fused, kc, vc, L, table, _, starts = prefix_tree_case(GROUPS[case], seed=case, dtype=dtype)
    planned = planned_attend(fused, kc, vc, L, table, starts, waves=1)
    walked = attend(fused, kc, vc, L, table, starts, waves=1)
    single = attend(fused, kc, vc, L, table, None, waves=1)
    assert np.array_equal(bits(planned), bits(walked))
    assert np.array_equal(bits(planned), bits(single))
    oracle_check(planned, fused, kc, vc, L, table)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("waves", [1, 2, 4, 8, 0])
def test_planned_matches_oracle(dtype, head_dim, waves):
    """Contexts up to 700 tokens in groups of up to 8 rows: plans of 15 to 158 entries
    per group."""
    fused, kc, vc, L, table, _, starts = prefix_tree_case([4, 4, 3, 8, 1, 5], seed=waves + 7,
                                                          dtype=dtype, D=head_dim, max_len=700)
    out = planned_attend(fused, kc, vc, L, table, starts, waves, D=head_dim)
    oracle_check(out, fused, kc, vc, L, table, D=head_dim)


@pytest.mark.parametrize("waves", [1, 2, 8])
def test_planned_groups_of_private_blocks_over_many_windows(waves):
    """Groups of 8 rows that share nothing, contexts up to 640 tokens: ~300 entries per
    group, five 64-entry windows."""
    H, D = 16, 64
    rnd = np.random.default_rng(31 + waves)
    g = torch.Generator().manual_seed(31 + waves)
    lens = [int(x) for x in rnd.integers(400, 641, size=16)]
    nbs = [-(-x // BS) for x in lens]
    NB = sum(nbs) + 3
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    table = torch.zeros(16, max(nbs), dtype=torch.int32)
    at = 0
    for i, nb in enumerate(nbs):
        table[i, :nb] = perm[at:at + nb]
        at += nb
    L = torch.tensor(lens, dtype=torch.int32)
    starts = torch.tensor([0, 8, 16], dtype=torch.int32)
    fused = torch.randn(16, 3 * H * D, generator=g).to(torch.bfloat16)
    kc = torch.randn(NB, H, BS, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(NB, H, BS, D, generator=g).to(torch.bfloat16)
    plan = hip().build_group_plan(table, L, starts, num_blocks=NB)
    counts = [int(plan.words[4 + s * plan.stride + 2]) for s in range(plan.slots)]
    assert min(counts) > 256
    out = planned_attend(fused, kc, vc, L, table, starts, waves)
    oracle_check(out, fused, kc, vc, L, table)
    if waves == 1:
        assert np.array_equal(bits(out), bits(attend(fused, kc, vc, L, table, None, 1)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("waves", [1, 2, 4])
def test_planned_fused_equals_two_steps(dtype, waves):
    fused, kc, vc, L, table, slots, starts = prefix_tree_case([4, 4, 2, 8, 3, 1], seed=11 + waves,
                                                              dtype=dtype)
    o2, k2, v2 = planned_write_and_attend(fused, kc, vc, L, table, slots, starts, waves, False)
    o1, k1, v1 = planned_write_and_attend(fused, kc, vc, L, table, slots, starts, waves, True)
    assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
    assert np.array_equal(bits(o1), bits(o2))
    oracle_check(o1, fused, k1, v1, L, table)
    if waves == 1:  # and the table-walking fused launch
        o0, k0, v0 = write_and_attend(fused, kc, vc, L, table, slots, starts, 1, fuse=True)
        assert np.array_equal(bits(o0), bits(o1))
        assert np.array_equal(bits(k0), bits(k1)) and np.array_equal(bits(v0), bits(v1))


@pytest.mark.parametrize("waves", [1, 2])
def test_planned_fused_slot_outside_the_context(waves):
    fused, kc, vc, L, table, slots, starts = prefix_tree_case([4, 3], seed=5)
    used = set(table.flatten().tolist())
    free = [b for b in range(kc.shape[0]) if b not in used]
    slots = slots.clone()
    slots[1] = free[0] * BS + 7  # a block nobody reads: written without substitution
    slots[4] = free[1] * BS  # in the second group, owned by a wave other than wave 0
    slots[5] = -1  # padding: not written
    o2, k2, v2 = planned_write_and_attend(fused, kc, vc, L, table, slots, starts, waves, False)
    o1, k1, v1 = planned_write_and_attend(fused, kc, vc, L, table, slots, starts, waves, True)
    assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
    assert np.array_equal(bits(o1), bits(o2))


def test_plan_order_and_padded_slots_write_only_their_rows():
    """Slots in a dispatch order, then empty slots up to a larger launch: every row is
    written once, with the same bits as the natural order; rows outside the groups keep
    what the output buffer held."""
    fused, kc, vc, L, table, _, starts = prefix_tree_case([3, 4, 2, 4], seed=21)
    ref = planned_attend(fused, kc, vc, L, table, starts, waves=1)
    order = torch.tensor([2, 0, 3, 1], dtype=torch.int32)
    N, H, D = fused.shape[0], 16, 64
    sentinel = torch.full((N, H, D), 7.0, dtype=fused.dtype, device=DEV)
    got = planned_attend(fused, kc, vc, L, table, starts, waves=1, order=order, slots=9,
                         out=sentinel)
    assert np.array_equal(bits(got), bits(ref))
    # groups over rows 0..8 only: rows 9.. stay untouched
    part = torch.tensor([0, 3, 7, 9], dtype=torch.int32)
    sentinel = torch.full((N, H, D), 7.0, dtype=fused.dtype, device=DEV)
    got = planned_attend(fused, kc, vc, L, table, part, waves=2, slots=6, out=sentinel)
    assert (got[9:].float() == 7.0).all()
    oracle_check(got[:9], fused[:9], kc, vc, L[:9], table[:9])


def test_planned_invalid_ids_zero_lengths_and_clamped_tables():
    fused, kc, vc, L, table, _, starts = prefix_tree_case([4, 4, 4], seed=9)
    L = L.clone()
    table = table.clone()
    L[2] = 0  # zero-length row inside a group
    table[5, 0] = -3  # invalid ids contribute nothing
    table[6, 1] = kc.shape[0] + 10
    for waves in (1, 4):
        planned = planned_attend(fused, kc, vc, L, table, starts, waves)
        assert (planned[2] == 0).all()
        if waves == 1:
            assert np.array_equal(bits(planned), bits(attend(fused, kc, vc, L, table, None, 1)))
    narrow = table[:, :3].contiguous()
    a = planned_attend(fused, kc, vc, L, narrow, starts, 1)
    b = attend(fused, kc, vc, L, narrow, None, 1)
    assert np.array_equal(bits(a), bits(b))


def test_planned_shared_partial_block_with_stale_nan_tail():
    hip_attn = hip()
    H, D = 16, 64
    g = torch.Generator().manual_seed(2)
    kc = torch.randn(8, H, BS, D, generator=g).to(torch.bfloat16)
    vlog = torch.randn(8, H, BS, D, generator=g).to(torch.bfloat16)
    kc[3, :, 9:] = float("nan")
    vlog[3, :, 9:] = float("nan")
    vc = hip_attn.v_cache_from_logical(vlog)
    table = torch.tensor([[1, 3], [1, 3], [5, 3], [1, 6]], dtype=torch.int32)
    L = torch.tensor([25, 23, 19, 32], dtype=torch.int32)
    fused = torch.randn(4, 3 * H * D, generator=g).to(torch.bfloat16)
    starts = torch.tensor([0, 4], dtype=torch.int32)
    for waves in (1, 2):
        out = planned_attend(fused, kc, vc, L, table, starts, waves)
        assert torch.isfinite(out.float()).all()
        oracle_check(out, fused, kc, vc, L, table)
    assert np.array_equal(bits(planned_attend(fused, kc, vc, L, table, starts, 1)),
                          bits(attend(fused, kc, vc, L, table, None, 1)))


@pytest.mark.parametrize("beams", [4, 3])
def test_planned_beam_search_tables_fused_equals_two_steps(beams):
    from vflorence_amd.workloads import beam_decode_schedule

    R, H, D = 6, 16, 64
    plans = beam_decode_schedule(num_requests=R, beams=beams, steps=70, cow_fraction=0.2,
                                 seed=beams)
    g = torch.Generator().manual_seed(beams)
    NB = 1 + max(max(max(t) for t in p.block_tables) for p in plans)
    kc = torch.randn(NB, H, BS, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(NB, H, BS, D, generator=g).to(torch.bfloat16)
    starts = torch.arange(0, R * beams + 1, beams, dtype=torch.int32)
    for step in (0, 1, 15, 16, 17, 40, 69):
        p = plans[step]
        N = len(p.context_lens)
        width = max(len(t) for t in p.block_tables)
        table = torch.zeros(N, width, dtype=torch.int32)
        for i, t in enumerate(p.block_tables):
            table[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
        L = torch.tensor(p.context_lens, dtype=torch.int32)
        slots = torch.tensor(p.slot_mapping, dtype=torch.int64)
        fused = torch.randn(N, 3 * H * D, generator=g).to(torch.bfloat16)
        for waves in (1, 2):
            o2, k2, v2 = planned_write_and_attend(fused, kc, vc, L, table, slots, starts, waves,
                                                  False)
            o1, k1, v1 = planned_write_and_attend(fused, kc, vc, L, table, slots, starts, waves,
                                                  True)
            assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
            assert np.array_equal(bits(o1), bits(o2))
        oracle_check(o1, fused, k1, v1, L, table)


def beam_step(beams, step, seed):
    from vflorence_amd.workloads import beam_decode_schedule

    R = 6
    plans = beam_decode_schedule(num_requests=R, beams=beams, steps=step + 1, cow_fraction=0.3,
                                 seed=seed)
    p = plans[step]
    N = len(p.context_lens)
    width = max(len(t) for t in p.block_tables)
    table = torch.zeros(N, width, dtype=torch.int32)
    for i, t in enumerate(p.block_tables):
        table[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    NB = 1 + max(max(max(t) for t in q.block_tables) for q in plans)
    starts = torch.arange(0, R * beams + 1, beams, dtype=torch.int32)
    return p, table, NB, starts


@pytest.mark.parametrize("beams", [4, 3])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("waves", [1, 2, 4])
def test_fused_launch_with_folded_copies_equals_copy_then_fused_launch(beams, head_dim, waves):
    """Copy-on-write folded into the plan: the fused launch reads each fork's source
    block, stores it whole to the fork's block with the new token in place and attends
    to it -- caches and outputs bit-identical to copy_blocks followed by the same fused
    launch (the reference's order, model_runner.py:284-286), stale tails included."""
    hip_attn = hip()
    H, D = 16, head_dim
    for step in (17, 33, 50):
        p, table, NB, starts = beam_step(beams, step, seed=10 * beams + step)
        assert p.copies
        N = len(p.context_lens)
        g = torch.Generator().manual_seed(step)
        kc = torch.randn(NB, H, BS, D, generator=g).to(torch.bfloat16)
        vc = torch.randn(NB, H, BS, D, generator=g).to(torch.bfloat16)
        fused = torch.randn(N, 3 * H * D, generator=g).to(torch.bfloat16).to(DEV)
        q, k, v = (t.reshape(N, H, D) for t in fused.chunk(3, dim=-1))
        L = torch.tensor(p.context_lens, dtype=torch.int32)
        slots = torch.tensor(p.slot_mapping, dtype=torch.int64).to(DEV)
        src = [a for a, _ in p.copies]
        dst = [b for _, b in p.copies]
        results = []
        for fold in (False, True):
            kd, vd = kc.to(DEV), vc.to(DEV)
            plan = hip_attn.build_group_plan(table, L, starts, block_size=BS, num_blocks=NB)
            if fold:
                assert hip_attn.fold_plan_copies(plan, src, dst, num_blocks=NB)
            else:
                hip_attn.copy_blocks([kd, vd], torch.tensor(src, device=DEV),
                                     torch.tensor(dst, device=DEV), staged=False)
            sm = planned_metadata(N, H, D, q.dtype, starts, plan.to(DEV), waves, True)
            out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
            hip_attn.self_attention_with_kv_write(q, k, v, kd, vd, out, L.to(DEV), slots,
                                                  scale=D**-0.5, block_table=table.to(DEV),
                                                  scheduler_metadata=sm)
            torch.cuda.synchronize()
            results.append((out.cpu(), kd.cpu(), vd.cpu()))
        (o0, k0, v0), (o1, k1, v1) = results
        assert np.array_equal(bits(k0), bits(k1)) and np.array_equal(bits(v0), bits(v1))
        assert np.array_equal(bits(o0), bits(o1))
        # the copies happened: every fork's block holds its source's tokens
        for a, b in p.copies:
            assert not np.array_equal(bits(kc[b]), bits(k1[b]))


def test_plain_launch_refuses_a_plan_with_copies_folded_in():
    """A folded plan names each fork block's copy source in its place, which only the
    fused launch acts on: the plain attention launch refuses it."""
    hip_attn = hip()
    H, D = 16, 64
    p, table, NB, starts = beam_step(4, 33, seed=5)
    N = len(p.context_lens)
    L = torch.tensor(p.context_lens, dtype=torch.int32)
    plan = hip_attn.build_group_plan(table, L, starts, block_size=BS, num_blocks=NB)
    assert hip_attn.fold_plan_copies(plan, [a for a, _ in p.copies], [b for _, b in p.copies],
                                     num_blocks=NB)
    sm = planned_metadata(N, H, D, torch.bfloat16, starts, plan.to(DEV), 2, False)
    q = torch.zeros(N, H, D, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(NB, H, BS, D, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="only self_attention_with_kv_write"):
        hip_attn.attention_with_kv_cache(q, kv, kv, torch.empty_like(q), None, L.to(DEV),
                                         scale=D**-0.5, block_table=table.to(DEV),
                                         scheduler_metadata=sm)


def test_plan_for_another_table_width_is_refused():
    fused, kc, vc, L, table, _, starts = prefix_tree_case([4, 4], seed=1)
    N, H, D = fused.shape[0], 16, 64
    plan = plan_for(table, L, starts, kc.shape[0])
    sm = planned_metadata(N, H, D, fused.dtype, starts, plan, 1, False)
    q = fused.to(DEV)[:, : H * D].reshape(N, H, D)
    out = torch.empty_like(q)
    wider = torch.zeros(N, table.shape[1] + 1, dtype=torch.int32)
    wider[:, : table.shape[1]] = table
    with pytest.raises(ValueError, match="group plan was made for block tables"):
        hip().attention_with_kv_cache(q, kc.to(DEV), vc.to(DEV), out, None, L.to(DEV),
                                      scale=D**-0.5, block_table=wider.to(DEV),
                                      scheduler_metadata=sm)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("waves", [1, 2, 4, 8])
@pytest.mark.parametrize("width", [40, 100])
def test_slot_descriptors_equal_the_group_start_path(dtype, head_dim, waves, width):
    """Shared-table groups (cross-attention beams) read through slot descriptors --
    each slot's group, length and page row in one load level -- give outputs
    bit-identical to the dispatch-order / group-start path, with a random dispatch
    order, empty groups and padded slots, and match the oracle.  Width 100: page rows
    past the 64 ids a wave holds at a time, read on from the descriptor."""
    from oracle import oracle as orc

    hip_attn = hip()
    rnd = np.random.default_rng(waves + head_dim + width)
    H, D, NB = 12, head_dim, 900
    sizes = [int(x) for x in rnd.integers(0, 9, size=14)]
    starts = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]), dtype=torch.int32)
    N = int(starts[-1])
    table = torch.zeros(N, width, dtype=torch.int32)
    lens = torch.zeros(N, dtype=torch.int32)
    for g, n in enumerate(sizes):  # a group's rows share one page row and length
        E = int(rnd.integers(0, width * BS + 1))
        pages = rnd.permutation(NB)[: -(-E // BS)]
        for r in range(int(starts[g]), int(starts[g + 1])):
            table[r, : len(pages)] = torch.from_numpy(pages.astype(np.int32))
            lens[r] = E
    order = torch.from_numpy(rnd.permutation(len(sizes)).astype(np.int32))
    slots = len(sizes) + 3
    g = torch.Generator().manual_seed(waves)
    kc = torch.randn(NB, H, BS, D, generator=g).to(dtype)
    vc = torch.randn(NB, H, BS, D, generator=g).to(dtype)
    q = torch.randn(N, H, D, generator=g).to(dtype)
    gs = torch.cat([starts, torch.full((slots - len(sizes),), N, dtype=torch.int32)])
    order_p = torch.cat([order, torch.full((slots - len(sizes),), -1, dtype=torch.int32)])
    desc = hip_attn.build_slot_descriptors(table, lens, starts, group_order=order,
                                           num_slots=slots).to(DEV)
    outs = []
    for use in (False, True):
        sm = hip_attn.get_scheduler_metadata(
            num_reqs=N, num_heads=H, num_kv_heads=H, head_dim=D, dtype=dtype, block_size=BS,
            group_start=gs.to(DEV), group_order=order_p.to(DEV), max_group_size=8,
            waves_per_workgroup=waves, slot_descriptors=desc if use else None)
        out = torch.full((N, H, D), float("nan"), dtype=dtype, device=DEV)
        hip_attn.attention_with_kv_cache(q.to(DEV), kc.to(DEV), vc.to(DEV), out, None,
                                         lens.to(DEV), scale=D**-0.5, block_table=table.to(DEV),
                                         scheduler_metadata=sm)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    want = orc.paged_attention(q.double().numpy(), kc.double().numpy(),
                               hip_attn.v_cache_logical(vc).double().numpy(), lens.numpy(),
                               table.numpy(), D**-0.5)
    np.testing.assert_allclose(outs[1].double().numpy(), want, rtol=0, atol=2e-2)
