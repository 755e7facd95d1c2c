"""Parity of the gfx950 kernels with the CPU oracle, through the C ABI.

Bars: bit-exact for the KV slot write and the copy-on-write block copy; attention
outputs within 1e-5 relative (plus 1e-6 absolute, for outputs near zero) in fp32 and
2e-2 absolute in bf16 / fp16, against the float64 oracle on identical inputs.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {
    torch.float32: dict(rtol=1e-5, atol=1e-6),
    torch.bfloat16: dict(rtol=0.0, atol=2e-2),
    torch.float16: dict(rtol=0.0, atol=2e-2),
}


def hip():
    from vflorence_amd import hip_attn

    return hip_attn


def as_f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy()


def raw_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.view(torch.int32).numpy().view(np.uint32)


# ---------------------------------------------------------------------------
# KV slot write
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_reshape_and_cache_bit_exact(dtype, head_dim):
    g = torch.Generator().manual_seed(11)
    T, H, bs, NB = 37, 16, 16, 50
    fused = torch.randn(T, 3 * H * head_dim, generator=g).to(dtype)
    key = fused[:, H * head_dim : 2 * H * head_dim].reshape(T, H, head_dim)
    value = fused[:, 2 * H * head_dim :].reshape(T, H, head_dim)
    kc = torch.randn(NB, H, bs, head_dim, generator=g).to(dtype)
    vc = torch.randn(NB, H, bs, head_dim, generator=g).to(dtype)
    slots = torch.randperm(NB * bs, generator=g)[:T].to(torch.int64)
    slots[5] = -1  # padding token
    kd, vd = kc.to(DEV), hip().v_cache_from_logical(vc).to(DEV)
    fd = fused.to(DEV)
    keyd = fd[:, H * head_dim : 2 * H * head_dim].reshape(T, H, head_dim)
    vald = fd[:, 2 * H * head_dim :].reshape(T, H, head_dim)
    hip().reshape_and_cache(keyd, vald, kd, vd, slots.to(DEV))
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(key), raw_bits(value), ko, vo, slots.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    assert np.array_equal(raw_bits(hip().v_cache_logical(vd)), vo)


def test_reshape_and_cache_unaligned_source():
    """A source whose rows start off a 16-byte boundary takes the element-wise path."""
    g = torch.Generator().manual_seed(12)
    T, H, D, bs, NB = 9, 16, 64, 16, 20
    fused = torch.randn(T, 2 * H * D + 1, generator=g).to(torch.bfloat16).to(DEV)
    key = fused[:, 1 : 1 + H * D].reshape(T, H, D)
    value = fused[:, 1 + H * D :].reshape(T, H, D)
    kc = torch.zeros(NB, H, bs, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([3, 100, 17, 250, 0, 319, 16, 15, 200], dtype=torch.int64, device=DEV)
    hip().reshape_and_cache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    vl = hip().v_cache_logical(vc)
    for t, s in enumerate(slots.tolist()):
        assert torch.equal(kc[s // bs, :, s % bs], key[t])
        assert torch.equal(vl[s // bs, :, s % bs], value[t])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("offset", [0, 1])
def test_reshape_and_cache_v_groups(dtype, head_dim, offset):
    """V of 16-bit pools is written a whole 4-token group at a time when four tokens
    take four consecutive slots starting at a multiple of 4, else token by token: runs
    that start on and off a group, a padding slot inside a run, a ragged tail, repeated
    blocks in another order; 16-byte aligned and unaligned source rows (``offset``)."""
    g = torch.Generator().manual_seed(14 + head_dim + offset)
    H, bs, NB = 16, 16, 40
    slots = (list(range(32, 48)) + list(range(66, 74)) + [100, 101, -1, 103]
             + list(range(200, 207)) + [5, 4, 7, 6] + list(range(400, 404)))
    T = len(slots)
    fused = torch.randn(T, 2 * H * head_dim + offset, generator=g).to(dtype)
    key = fused[:, offset: offset + H * head_dim].reshape(T, H, head_dim)
    value = fused[:, offset + H * head_dim:].reshape(T, H, head_dim)
    kc = torch.randn(NB, H, bs, head_dim, generator=g).to(dtype)
    vc = torch.randn(NB, H, bs, head_dim, generator=g).to(dtype)
    kd, vd = kc.to(DEV), hip().v_cache_from_logical(vc).to(DEV)
    fd = fused.to(DEV)
    keyd = fd[:, offset: offset + H * head_dim].reshape(T, H, head_dim)
    vald = fd[:, offset + H * head_dim:].reshape(T, H, head_dim)
    st = torch.tensor(slots, dtype=torch.int64)
    hip().reshape_and_cache(keyd, vald, kd, vd, st.to(DEV))
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(key), raw_bits(value), ko, vo, st.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    assert np.array_equal(raw_bits(hip().v_cache_logical(vd)), vo)


def test_reshape_and_cache_large_encoder_write():
    """The encoder path writes G * enc_len rows at once (model_runner.py:248-259)."""
    g = torch.Generator().manual_seed(13)
    G, E, H, D, bs = 4, 777, 16, 64, 16
    pages = torch.randperm(400, generator=g)[: G * math.ceil(E / bs)].view(G, -1)
    slots = torch.from_numpy(orc.cross_slots(pages.numpy(), E, bs))
    key = torch.randn(G * E, H, D, generator=g).to(torch.bfloat16)
    value = torch.randn(G * E, H, D, generator=g).to(torch.bfloat16)
    kc = torch.zeros(400, H, bs, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kd, vd = kc.to(DEV), vc.to(DEV)
    hip().reshape_and_cache(key.to(DEV), value.to(DEV), kd, vd, slots.to(DEV))
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(key), raw_bits(value), ko, vo, slots.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    assert np.array_equal(raw_bits(hip().v_cache_logical(vd)), vo)


# ---------------------------------------------------------------------------
# copy-on-write block copy
# ---------------------------------------------------------------------------
def test_copy_blocks_reference_kat():
    """tests/test_engine.py:382-405 of the reference: blocks hold their id, copy
    (0,2),(1,3) in every cache, blocks 0..3 then read [0, 1, 0, 1]."""
    caches = [
        torch.stack([torch.full((16, 16, 64), b, dtype=torch.bfloat16) for b in range(8)]).to(DEV)
        for _ in range(24)
    ]
    src = torch.tensor([0, 1], dtype=torch.int64, device=DEV)
    dst = torch.tensor([2, 3], dtype=torch.int64, device=DEV)
    hip().copy_blocks(caches, src, dst, staged=False)
    torch.cuda.synchronize()
    for c in caches:
        assert [c[b].unique().item() for b in range(4)] == [0, 1, 0, 1]


@pytest.mark.parametrize("staged", [False, True])
def test_copy_blocks_random_pairs_bit_exact(staged):
    g = torch.Generator().manual_seed(21)
    NB, ncache = 300, 6
    caches = [torch.randn(NB, 16, 16, 64, generator=g).to(torch.bfloat16) for _ in range(ncache)]
    perm = torch.randperm(NB, generator=g).tolist()
    if staged:
        # chains: a destination is also a later source -> must gather before scatter
        pairs = [(perm[i], perm[i + 1]) for i in range(0, 80)]
    else:
        pairs = [(perm[i], perm[100 + i]) for i in range(80)]
    hip_attn = hip()
    assert hip_attn.copy_pairs_need_staging(pairs) == staged
    dcaches = [c.to(DEV) for c in caches]
    src = torch.tensor([s for s, _ in pairs], dtype=torch.int64, device=DEV)
    dst = torch.tensor([d for _, d in pairs], dtype=torch.int64, device=DEV)
    hip_attn.copy_blocks(dcaches, src, dst, staged=staged)
    torch.cuda.synchronize()
    want = [raw_bits(c) for c in caches]
    orc.copy_blocks(want, pairs)
    for d, w in zip(dcaches, want):
        assert np.array_equal(raw_bits(d), w)


def test_copy_blocks_rejects_repeated_destination():
    with pytest.raises(ValueError):
        hip().copy_pairs_need_staging([(1, 5), (2, 5)])


# ---------------------------------------------------------------------------
# paged attention (self: one row per group)
# ---------------------------------------------------------------------------
def make_case(lens, H=16, D=64, bs=16, NB=None, dtype=torch.bfloat16, seed=0, std=1.0,
              strided=True):
    g = torch.Generator().manual_seed(seed)
    N = len(lens)
    nblk = [max(1, math.ceil(max(L, 0) / bs)) for L in lens]
    if NB is None:
        NB = sum(nblk) + 7
    perm = torch.randperm(NB, generator=g).tolist()
    width = max(nblk)
    table = torch.zeros(N, width, dtype=torch.int32)
    pos = 0
    for r, nb in enumerate(nblk):
        table[r, :nb] = torch.tensor(perm[pos : pos + nb], dtype=torch.int32)
        pos += nb
    kc = (torch.randn(NB, H, bs, D, generator=g) * std).to(dtype)
    vc = (torch.randn(NB, H, bs, D, generator=g) * std).to(dtype)
    if strided:
        fused = (torch.randn(N, 3 * H * D, generator=g) * std).to(dtype)
        q = fused[:, : H * D].reshape(N, H, D)
    else:
        q = (torch.randn(N, H, D, generator=g) * std).to(dtype)
    return q, kc, vc, torch.tensor(lens, dtype=torch.int32), table


def run_gpu(q, kc, vc, lens, table, scale, waves=0, group_start=None, gmax=1, order=False):
    hip_attn = hip()
    qd = q.to(DEV) if q.is_contiguous() else None
    if qd is None:  # keep the strided layout on the device
        base = q.as_strided((q.shape[0], q.stride(0)), (q.stride(0), 1), q.storage_offset())
        fused = torch.empty(q.shape[0], q.stride(0), dtype=q.dtype)
        fused.copy_(base)
        qd = fused.to(DEV).as_strided(q.shape, q.stride(), 0)
    kd, vd = kc.to(DEV), hip_attn.v_cache_from_logical(vc).to(DEV)
    out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
    meta = hip_attn.get_scheduler_metadata(
        num_reqs=q.shape[0], num_heads=q.shape[1], num_kv_heads=q.shape[1], head_dim=q.shape[2],
        dtype=q.dtype, block_size=kc.shape[2], waves_per_workgroup=waves,
        group_start=None if group_start is None else group_start.to(DEV), max_group_size=gmax,
        group_order=group_order(lens, group_start) if order else None,
    )
    hip_attn.attention_with_kv_cache(
        qd, kd, vd, out, torch.arange(q.shape[0] + 1, dtype=torch.int32, device=DEV),
        lens.to(DEV), scale=scale, causal=False, block_table=table.to(DEV),
        scheduler_metadata=meta,
    )
    torch.cuda.synchronize()
    return out.cpu()


def group_order(lens, group_start):
    firsts = lens.tolist() if group_start is None else [lens[i].item() for i in group_start[:-1]]
    order = hip().longest_first(firsts)
    return torch.tensor(order, dtype=torch.int32, device=DEV)


def check(out, q, kc, vc, lens, table, scale):
    want = orc.paged_attention(as_f64(q), as_f64(kc), as_f64(vc), lens.numpy(), table.numpy(),
                               scale)
    np.testing.assert_allclose(as_f64(out), want, **TOL[q.dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("waves", [1, 2, 4, 8, 0])
def test_self_attention_matches_oracle(dtype, head_dim, waves):
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 100, 255, 256, 257, 511, 700, 1024, 64]
    q, kc, vc, L, table = make_case(lens, D=head_dim, dtype=dtype, seed=1)
    scale = head_dim**-0.5
    out = run_gpu(q, kc, vc, L, table, scale, waves=waves, order=waves == 4)
    check(out, q, kc, vc, L, table, scale)


@pytest.mark.parametrize("H", [12, 16, 5])
def test_self_attention_head_counts(H):
    """Florence-2-base has 12 heads; 5 leaves a partly filled workgroup."""
    lens = [40, 300, 1, 129]
    q, kc, vc, L, table = make_case(lens, H=H, seed=2)
    out = run_gpu(q, kc, vc, L, table, 0.125, waves=4)
    check(out, q, kc, vc, L, table, 0.125)


def test_one_token_context_returns_value_exactly():
    lens = [1] * 8
    q, kc, vc, L, table = make_case(lens, dtype=torch.float32, seed=3)
    out = run_gpu(q, kc, vc, L, table, 0.125)
    want = vc[table[:, 0].long(), :, 0, :]
    assert torch.equal(out, want)


def test_zero_length_rows_give_zeros():
    lens = [0, 50, 0, 7]
    q, kc, vc, L, table = make_case(lens, seed=4)
    out = run_gpu(q, kc, vc, L, table, 0.125, waves=2)
    assert not out[0].any() and not out[2].any()
    check(out, q, kc, vc, L, table, 0.125)


def test_stale_tail_values_are_ignored():
    """Recycled blocks keep old data past the context (model_runner.py:64-65 zeroes
    pools only once); NaN there must not reach the output."""
    lens = [5, 21, 40]
    q, kc, vc, L, table = make_case(lens, dtype=torch.float32, seed=5)
    bs = 16
    for r, n in enumerate(lens):
        last = table[r, (n - 1) // bs]
        kc[last, :, n % bs or bs :, :] = float("nan")
        vc[last, :, n % bs or bs :, :] = float("nan")
    out = run_gpu(q, kc, vc, L, table, 0.125)
    assert torch.isfinite(out).all()
    kc2, vc2 = kc.nan_to_num(0.0), vc.nan_to_num(0.0)
    check(out, q, kc2, vc2, L, table, 0.125)


def test_context_longer_than_table_is_clamped():
    lens = [40, 40]
    q, kc, vc, L, table = make_case(lens, seed=6)
    L2 = torch.tensor([40, 40 + 16 * 5], dtype=torch.int32)  # row 1 claims more than its 3 blocks
    out = run_gpu(q, kc, vc, L2, table, 0.125)
    check(out, q, kc, vc, torch.tensor([40, 48], dtype=torch.int32), table, 0.125)


def test_invalid_block_ids_contribute_nothing():
    lens = [48, 48]
    q, kc, vc, L, table = make_case(lens, dtype=torch.float32, seed=7)
    NB = kc.shape[0]
    bad = table.clone()
    bad[1, 1] = NB + 1000  # out of the pool: skipped, not dereferenced
    out = run_gpu(q, kc, vc, L, bad, 0.125)
    check(out[:1], q[:1], kc, vc, L[:1], table[:1], 0.125)
    # row 1 attends to blocks 0 and 2 only
    keep = [table[1, 0].item(), table[1, 2].item()]
    kk = torch.cat([kc[keep[0]], kc[keep[1]]], dim=1)  # [H, 32, D]
    vv = torch.cat([vc[keep[0]], vc[keep[1]]], dim=1)
    p = torch.softmax(torch.einsum("hd,hld->hl", q[1].double(), kk.double()) * 0.125, dim=-1)
    want = torch.einsum("hl,hld->hd", p, vv.double())
    np.testing.assert_allclose(out[1].double().numpy(), want.numpy(), rtol=1e-5, atol=1e-6)


def test_deterministic():
    lens = torch.randint(1, 1025, (64,), generator=torch.Generator().manual_seed(8)).tolist()
    q, kc, vc, L, table = make_case(lens, seed=8)
    a = run_gpu(q, kc, vc, L, table, 0.125)
    b = run_gpu(q, kc, vc, L, table, 0.125)
    assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# paged attention with row groups (cross-attention beams)
# ---------------------------------------------------------------------------
def grouped_case(group_sizes, enc_lens, H=16, D=64, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    bs = 16
    need = [math.ceil(E / bs) for E in enc_lens]
    NB = sum(need) + 3
    perm = torch.randperm(NB, generator=g)
    width = max(need)
    rows_table, rows_len, starts, pos = [], [], [0], 0
    for gs, E, n in zip(group_sizes, enc_lens, need):
        pages = torch.zeros(width, dtype=torch.int32)
        pages[:n] = perm[pos : pos + n].to(torch.int32)
        pos += n
        for _ in range(gs):
            rows_table.append(pages)
            rows_len.append(E)
        starts.append(starts[-1] + gs)
    table = torch.stack(rows_table)
    N = len(rows_len)
    q = torch.randn(N, H, D, generator=g).to(dtype)
    kc = torch.randn(NB, H, bs, D, generator=g).to(dtype)
    vc = torch.randn(NB, H, bs, D, generator=g).to(dtype)
    return q, kc, vc, torch.tensor(rows_len, dtype=torch.int32), table, torch.tensor(
        starts, dtype=torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("group_sizes", [[4] * 6, [1, 2, 3, 4], [8, 8, 1], [3] * 5, [2, 7, 5]])
@pytest.mark.parametrize("waves", [1, 8, 0])
def test_grouped_attention_matches_oracle(dtype, group_sizes, waves):
    enc = [256 + 97 * i for i in range(len(group_sizes))]
    q, kc, vc, L, table, starts = grouped_case(group_sizes, enc, dtype=dtype, seed=9)
    gmax = max(group_sizes)
    out = run_gpu(q, kc, vc, L, table, 0.125, waves=waves, group_start=starts, gmax=gmax,
                  order=waves == 0)
    check(out, q, kc, vc, L, table, 0.125)


def test_grouped_equals_ungrouped():
    q, kc, vc, L, table, starts = grouped_case([4] * 8, [300 + 50 * i for i in range(8)], seed=10)
    a = run_gpu(q, kc, vc, L, table, 0.125, group_start=starts, gmax=4)
    b = run_gpu(q, kc, vc, L, table, 0.125)
    np.testing.assert_allclose(as_f64(a), as_f64(b), atol=2e-2)


# ---------------------------------------------------------------------------
# full-size workloads
# ---------------------------------------------------------------------------
def test_config_self_attention_256_ragged_sequences():
    """256 sequences, ctx U[1,1024], 20k-block pool, bf16, with the KV slot write."""
    from vflorence_amd import workloads

    case = workloads.self_attention_case(device=DEV, seed=0)
    hip_attn = hip()
    kc0, vc0 = raw_bits(case.k_cache), raw_bits(hip_attn.v_cache_logical(case.v_cache))
    hip_attn.reshape_and_cache(case.key, case.value, case.k_cache, case.v_cache, case.slot_mapping)
    out = torch.empty(case.query.shape, dtype=case.query.dtype, device=DEV)
    hip_attn.attention_with_kv_cache(
        case.query, case.k_cache, case.v_cache, out, None, case.context_lens, scale=case.scale,
        block_table=case.block_tables,
    )
    torch.cuda.synchronize()
    orc.reshape_and_cache(raw_bits(case.key), raw_bits(case.value), kc0, vc0,
                          case.slot_mapping.cpu().numpy())
    assert np.array_equal(raw_bits(case.k_cache), kc0)
    assert np.array_equal(raw_bits(hip_attn.v_cache_logical(case.v_cache)), vc0)
    table = case.block_tables.cpu().numpy()
    used, remapped = np.unique(table, return_inverse=True)
    want = orc.paged_attention(
        as_f64(case.query), orc.bf16_bits_to_f64(kc0[used]), orc.bf16_bits_to_f64(vc0[used]),
        case.context_lens.cpu().numpy(), remapped.reshape(table.shape).astype(np.int32),
        case.scale)
    np.testing.assert_allclose(as_f64(out.cpu()), want, rtol=0, atol=2e-2)
