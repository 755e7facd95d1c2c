"""Pools of 32-token blocks, the reference's block size on x86 (vflorence/config.py:42),
through the C ABI against the float64 oracle (bars of test_kernels_gpu: KV write and
block copy bit-exact, attention within 1e-5 relative in fp32 and 2e-2 absolute in
bf16 / fp16).

The one-row and VALU attention kernels read a 32-token block as two 16-token parts at
the same offset in K and in the 4-token-interleaved V; beam groups keeping their own
tables and the fused KV write fall back to one row per group and a separate write, so
those calls must give the oracle's results too.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from test_kernels_gpu import DEV, as_f64, check, hip, make_case, raw_bits, run_gpu

pytestmark = pytest.mark.gpu

BS = 32
LENS = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 500, 0, 257]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128, 48])
def test_reshape_and_cache_bit_exact(dtype, head_dim):
    g = torch.Generator().manual_seed(41 + head_dim)
    H, NB = 8, 10
    slots = torch.tensor(list(range(64, 96)) + [3, 200, -1, 31, 32, 33, 34, 35, 319, 7, 6],
                         dtype=torch.int64)
    T = slots.numel()
    key = torch.randn(T, H, head_dim, generator=g).to(dtype)
    value = torch.randn(T, H, head_dim, generator=g).to(dtype)
    kc = torch.randn(NB, H, BS, head_dim, generator=g).to(dtype)
    vc = torch.randn(NB, H, BS, head_dim, generator=g).to(dtype)
    kd, vd = kc.to(DEV), hip().v_cache_from_logical(vc).to(DEV)
    hip().reshape_and_cache(key.to(DEV), value.to(DEV), kd, vd, slots.to(DEV))
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(key), raw_bits(value), ko, vo, slots.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    assert np.array_equal(raw_bits(hip().v_cache_logical(vd)), vo)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128, 48])
@pytest.mark.parametrize("waves", [1, 4, 0])
def test_self_attention_matches_oracle(dtype, head_dim, waves):
    q, kc, vc, L, table = make_case(LENS, H=8, D=head_dim, bs=BS, dtype=dtype, seed=head_dim)
    scale = head_dim**-0.5
    out = run_gpu(q, kc, vc, L, table, scale, waves=waves)
    check(out, q, kc, vc, L, table, scale)


def grouped_case32(group_sizes, enc_lens, H=8, D=64, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    need = [math.ceil(E / BS) for E in enc_lens]
    NB = sum(need) + 3
    perm = torch.randperm(NB, generator=g)
    width = max(need)
    rows_table, rows_len, starts, pos = [], [], [0], 0
    for gs, E, n in zip(group_sizes, enc_lens, need):
        pages = torch.zeros(width, dtype=torch.int32)
        pages[:n] = perm[pos: pos + n].to(torch.int32)
        pos += n
        rows_table += [pages] * gs
        rows_len += [E] * gs
        starts.append(starts[-1] + gs)
    q = torch.randn(len(rows_len), H, D, generator=g).to(dtype)
    kc = torch.randn(NB, H, BS, D, generator=g).to(dtype)
    vc = torch.randn(NB, H, BS, D, generator=g).to(dtype)
    return (q, kc, vc, torch.tensor(rows_len, dtype=torch.int32), torch.stack(rows_table),
            torch.tensor(starts, dtype=torch.int32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 80])
def test_cross_attention_beam_groups(dtype, head_dim):
    sizes = [4, 1, 3, 8]
    q, kc, vc, L, table, starts = grouped_case32(sizes, [47, 300, 64, 129], D=head_dim,
                                                 dtype=dtype, seed=5)
    out = run_gpu(q, kc, vc, L, table, 0.125, group_start=starts, gmax=8, order=True)
    check(out, q, kc, vc, L, table, 0.125)


def test_table_clamp_and_invalid_ids():
    """Contexts longer than the table are clamped to its width in 32-token blocks; an id
    outside the pool contributes nothing."""
    q, kc, vc, L, table = make_case([70, 70], H=4, bs=BS, dtype=torch.float32, seed=9)
    L2 = torch.tensor([70, 70 + 32 * 4], dtype=torch.int32)  # row 1 claims 4 more blocks
    out = run_gpu(q, kc, vc, L2, table, 0.125)
    check(out, q, kc, vc, torch.tensor([70, 96], dtype=torch.int32), table, 0.125)
    bad = table.clone()
    bad[1, 1] = kc.shape[0] + 50
    out = run_gpu(q, kc, vc, L, bad, 0.125)
    check(out[:1], q[:1], kc, vc, L[:1], table[:1], 0.125)
    keep = [bad[1, 0].item(), bad[1, 2].item()]
    kk = torch.cat([kc[keep[0]], kc[keep[1], :, :6]], dim=1).double()  # tokens 0-31, 64-69
    vv = torch.cat([vc[keep[0]], vc[keep[1], :, :6]], dim=1).double()
    p = torch.softmax(torch.einsum("hd,hld->hl", q[1].double(), kk) * 0.125, dim=-1)
    want = torch.einsum("hl,hld->hd", p, vv)
    np.testing.assert_allclose(out[1].double().numpy(), want.numpy(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_entry_point_and_beam_groups_fall_back(dtype):
    """The fused write over beam groups keeping their own tables (the engine's call) on
    32-token blocks: cache bit-exact against the oracle's write, output against the
    oracle."""
    hip_attn = hip()
    g = torch.Generator().manual_seed(17)
    H, D = 8, 64
    table = torch.tensor([[0, 1, 0], [0, 2, 0], [3, 4, 5], [3, 4, 6]], dtype=torch.int32)
    lens = torch.tensor([40, 40, 70, 70], dtype=torch.int32)
    slots = torch.tensor([table[r, (n - 1) // BS].item() * BS + (n - 1) % BS
                          for r, n in enumerate(lens.tolist())], dtype=torch.int64)
    NB = 8
    kc = torch.randn(NB, H, BS, D, generator=g).to(dtype)
    vc = torch.randn(NB, H, BS, D, generator=g).to(dtype)
    q, k, v = (torch.randn(4, H, D, generator=g).to(dtype) for _ in range(3))
    kd, vd = kc.to(DEV), hip_attn.v_cache_from_logical(vc).to(DEV)
    out = torch.empty(4, H, D, dtype=dtype, device=DEV)
    meta = hip_attn.get_scheduler_metadata(
        num_reqs=4, num_heads=H, num_kv_heads=H, head_dim=D, dtype=dtype, block_size=BS,
        group_start=torch.tensor([0, 2, 4], dtype=torch.int32, device=DEV), max_group_size=2,
        own_tables=True, fuse_kv_write=True)
    hip_attn.self_attention_with_kv_write(q.to(DEV), k.to(DEV), v.to(DEV), kd, vd, out,
                                          lens.to(DEV), slots.to(DEV), scale=0.125,
                                          block_table=table.to(DEV), scheduler_metadata=meta)
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(k), raw_bits(v), ko, vo, slots.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    assert np.array_equal(raw_bits(hip_attn.v_cache_logical(vd)), vo)
    np_int = np.int16 if dtype != torch.float32 else np.int32
    kw = torch.from_numpy(ko.view(np_int)).view(dtype)
    vw = torch.from_numpy(vo.view(np_int)).view(dtype)
    check(out.cpu(), q, kw, vw, lens, table, 0.125)


@pytest.mark.parametrize("staged", [False, True])
def test_copy_blocks_32_token_blocks(staged):
    g = torch.Generator().manual_seed(23)
    NB = 60
    caches = [torch.randn(NB, 8, BS, 64, generator=g).to(torch.bfloat16) for _ in range(4)]
    perm = torch.randperm(NB, generator=g).tolist()
    pairs = ([(perm[i], perm[i + 1]) for i in range(12)] if staged
             else [(perm[i], perm[30 + i]) for i in range(12)])
    assert hip().copy_pairs_need_staging(pairs) == staged
    dcaches = [c.to(DEV) for c in caches]
    src = torch.tensor([s for s, _ in pairs], dtype=torch.int64, device=DEV)
    dst = torch.tensor([d for _, d in pairs], dtype=torch.int64, device=DEV)
    hip().copy_blocks(dcaches, src, dst, staged=staged)
    torch.cuda.synchronize()
    want = [raw_bits(c) for c in caches]
    orc.copy_blocks(want, pairs)
    for d, w in zip(dcaches, want):
        assert np.array_equal(raw_bits(d), w)


def test_self_attention_op_through_context():
    """vflorence::self_attention as the reference's runner calls it on x86 (32-token
    tables from its block manager, metadata for block_size 32)."""
    from vflorence_amd.layers import attention
    from vflorence_amd.utils.context import set_context

    hip_attn = hip()
    g = torch.Generator().manual_seed(29)
    lens = [3, 33, 64, 65, 1]
    N, H, D = len(lens), 16, 64
    q, kc, vc, L, table = make_case(lens, H=H, D=D, bs=BS, seed=29, strided=False)
    slots = torch.tensor([table[r, (n - 1) // BS].item() * BS + (n - 1) % BS
                          for r, n in enumerate(lens)], dtype=torch.int64)
    k = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kd, vd = kc.to(DEV), hip_attn.v_cache_from_logical(vc).to(DEV)
    meta = hip_attn.get_scheduler_metadata(num_reqs=N, num_heads=H, num_kv_heads=H,
                                           head_dim=D, dtype=torch.bfloat16, block_size=BS)
    set_context(context_lens=L.to(DEV), block_tables=table.to(DEV), slot_mapping=slots.to(DEV),
                query_start_loc=torch.arange(N + 1, dtype=torch.int32, device=DEV),
                self_metadata=meta, isa="gfx950")
    try:
        out = attention.decoder_self_attention(q.to(DEV), k.to(DEV), v.to(DEV), kd, vd, 0.125)
    finally:
        set_context()
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(k), raw_bits(v), ko, vo, slots.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    kw = torch.from_numpy(ko.view(np.int16)).view(torch.bfloat16)
    vw = torch.from_numpy(vo.view(np.int16)).view(torch.bfloat16)
    want = orc.paged_attention(as_f64(q), as_f64(kw), as_f64(vw), L.numpy(), table.numpy(), 0.125)
    np.testing.assert_allclose(as_f64(out.cpu()), want, rtol=0.0, atol=2e-2)
