"""The reference's other head sizes (vflorence/layers/attention.py:6: 32, 48, 80, 96,
112, 160, 192, 224, 256, 512 besides 64 and 128) through the C ABI, against the
float64 oracle with the bars of test_kernels_gpu: the KV slot write bit-exact,
attention within 1e-5 relative in fp32 and 2e-2 absolute in bf16 / fp16.

These sizes run the one-row / shared-table kernels: the fp32 VALU kernel with its
lanes padded to a power of two per token row, and the matrix-core kernel with a half
empty last K chunk for 48, 80 and 112.  Beam groups keeping their own tables, group
plans and the fused KV write have no kernel for them; the entry points then run every
row as its own group and the write as its own launch, with the same results -- which
the last tests check through the op and the fused entry point.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from test_kernels_gpu import DEV, as_f64, check, grouped_case, hip, make_case, raw_bits, run_gpu

pytestmark = pytest.mark.gpu

OTHER_DIMS = [32, 48, 80, 96, 112, 160, 192, 224, 256, 512]
DTYPES = [torch.bfloat16, torch.float32, torch.float16]


def heads_for(d):
    return 4 if d >= 256 else 8


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", OTHER_DIMS)
def test_reshape_and_cache_bit_exact(dtype, head_dim):
    g = torch.Generator().manual_seed(31 + head_dim)
    T, H, bs, NB = 23, heads_for(head_dim), 16, 12
    key = torch.randn(T, H, head_dim, generator=g).to(dtype)
    value = torch.randn(T, H, head_dim, generator=g).to(dtype)
    kc = torch.randn(NB, H, bs, head_dim, generator=g).to(dtype)
    vc = torch.randn(NB, H, bs, head_dim, generator=g).to(dtype)
    # a run of whole 4-token groups, scattered slots and a padding slot
    slots = torch.tensor(list(range(32, 44)) + [100, 3, -1, 77, 150, 151, 152, 9, 8, 10, 191],
                         dtype=torch.int64)
    kd, vd = kc.to(DEV), hip().v_cache_from_logical(vc).to(DEV)
    hip().reshape_and_cache(key.to(DEV), value.to(DEV), kd, vd, slots.to(DEV))
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(key), raw_bits(value), ko, vo, slots.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    assert np.array_equal(raw_bits(hip().v_cache_logical(vd)), vo)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", OTHER_DIMS)
@pytest.mark.parametrize("waves", [1, 0])
def test_self_attention_matches_oracle(dtype, head_dim, waves):
    lens = [1, 15, 16, 17, 33, 100, 255, 300, 0, 64]
    q, kc, vc, L, table = make_case(lens, H=heads_for(head_dim), D=head_dim, dtype=dtype,
                                    seed=head_dim)
    scale = head_dim**-0.5
    out = run_gpu(q, kc, vc, L, table, scale, waves=waves)
    check(out, q, kc, vc, L, table, scale)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("head_dim", OTHER_DIMS)
def test_cross_attention_beam_groups(dtype, head_dim):
    """Beams sharing one encoder table in the tile columns (one read for the group)."""
    sizes = [4, 3, 1, 8]
    enc = [40 + 61 * i for i in range(len(sizes))]
    q, kc, vc, L, table, starts = grouped_case(sizes, enc, H=heads_for(head_dim), D=head_dim,
                                               dtype=dtype, seed=head_dim + 1)
    scale = head_dim**-0.5
    out = run_gpu(q, kc, vc, L, table, scale, group_start=starts, gmax=max(sizes), order=True)
    check(out, q, kc, vc, L, table, scale)


@pytest.mark.parametrize("head_dim", [48, 80, 112])
def test_stale_tail_nan_ignored_half_chunk(head_dim):
    """A half-empty last K chunk reads nothing past the head: NaN in the next token's
    dims (the stale tail of the block) must not reach the output."""
    lens = [5, 21]
    q, kc, vc, L, table = make_case(lens, H=4, D=head_dim, dtype=torch.bfloat16, seed=3)
    for r, n in enumerate(lens):
        last = table[r, (n - 1) // 16]
        kc[last, :, n % 16:, :] = float("nan")
        vc[last, :, n % 16:, :] = float("nan")
    out = run_gpu(q, kc, vc, L, table, head_dim**-0.5)
    assert torch.isfinite(out.float()).all()
    check(out, q, kc.nan_to_num(0.0), vc.nan_to_num(0.0), L, table, head_dim**-0.5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("head_dim", [48, 96, 256])
def test_fused_entry_point_runs_two_steps(dtype, head_dim):
    """vfl_self_attention_with_kv_write on beam groups keeping their own tables: for these
    head sizes it writes the slots and then attends row by row; cache bit-exact against
    the oracle's write, output against the oracle."""
    hip_attn = hip()
    g = torch.Generator().manual_seed(head_dim)
    H, bs = 4, 16
    # two requests x 3 beams sharing their first block; each beam's own last block
    table = torch.tensor([[0, 1], [0, 2], [0, 3], [4, 5], [4, 6], [4, 7]], dtype=torch.int32)
    lens = torch.tensor([20, 20, 20, 31, 31, 31], dtype=torch.int32)
    slots = torch.tensor([table[r, (n - 1) // bs].item() * bs + (n - 1) % bs
                          for r, n in enumerate(lens.tolist())], dtype=torch.int64)
    NB = 9
    kc = torch.randn(NB, H, bs, head_dim, generator=g).to(dtype)
    vc = torch.randn(NB, H, bs, head_dim, generator=g).to(dtype)
    q = torch.randn(6, H, head_dim, generator=g).to(dtype)
    k = torch.randn(6, H, head_dim, generator=g).to(dtype)
    v = torch.randn(6, H, head_dim, generator=g).to(dtype)
    kd, vd = kc.to(DEV), hip_attn.v_cache_from_logical(vc).to(DEV)
    out = torch.empty(6, H, head_dim, dtype=dtype, device=DEV)
    starts = torch.tensor([0, 3, 6], dtype=torch.int32, device=DEV)
    meta = hip_attn.get_scheduler_metadata(
        num_reqs=6, num_heads=H, num_kv_heads=H, head_dim=head_dim, dtype=dtype, block_size=bs,
        group_start=starts, max_group_size=3, own_tables=True, fuse_kv_write=True)
    hip_attn.self_attention_with_kv_write(q.to(DEV), k.to(DEV), v.to(DEV), kd, vd, out,
                                          lens.to(DEV), slots.to(DEV), scale=head_dim**-0.5,
                                          block_table=table.to(DEV), scheduler_metadata=meta)
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(k), raw_bits(v), ko, vo, slots.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    assert np.array_equal(raw_bits(hip_attn.v_cache_logical(vd)), vo)
    kw = torch.from_numpy(ko.view(np.int16 if dtype != torch.float32 else np.int32))
    vw = torch.from_numpy(vo.view(np.int16 if dtype != torch.float32 else np.int32))
    kw, vw = kw.view(dtype), vw.view(dtype)
    check(out.cpu(), q, kw, vw, lens, table, head_dim**-0.5)


@pytest.mark.parametrize("head_dim", [32, 112, 192])
def test_ops_through_context(head_dim):
    """The custom ops (vflorence::self_attention and vflorence::cross_attention) at
    these head sizes, as a model with such heads would call them."""
    from vflorence_amd.layers import attention
    from vflorence_amd.utils.context import set_context

    hip_attn = hip()
    g = torch.Generator().manual_seed(7 + head_dim)
    H, bs, N = 4, 16, 5
    lens = [3, 17, 40, 1, 64]
    q, kc, vc, L, table = make_case(lens, H=H, D=head_dim, seed=head_dim, strided=False)
    slots = torch.tensor([table[r, (n - 1) // bs].item() * bs + (n - 1) % bs
                          for r, n in enumerate(lens)], dtype=torch.int64)
    k = torch.randn(N, H, head_dim, generator=g).to(torch.bfloat16)
    v = torch.randn(N, H, head_dim, generator=g).to(torch.bfloat16)
    kd, vd = kc.to(DEV), hip_attn.v_cache_from_logical(vc).to(DEV)
    meta = hip_attn.get_scheduler_metadata(
        num_reqs=N, num_heads=H, num_kv_heads=H, head_dim=head_dim, dtype=torch.bfloat16,
        block_size=bs)
    set_context(context_lens=L.to(DEV), block_tables=table.to(DEV), slot_mapping=slots.to(DEV),
                query_start_loc=torch.arange(N + 1, dtype=torch.int32, device=DEV),
                self_metadata=meta, isa="gfx950")
    try:
        out = attention.decoder_self_attention(q.to(DEV), k.to(DEV), v.to(DEV), kd, vd,
                                               head_dim**-0.5)
    finally:
        set_context()
    torch.cuda.synchronize()
    ko, vo = raw_bits(kc), raw_bits(vc)
    orc.reshape_and_cache(raw_bits(k), raw_bits(v), ko, vo, slots.numpy())
    assert np.array_equal(raw_bits(kd), ko)
    kw = torch.from_numpy(ko.view(np.int16)).view(torch.bfloat16)
    vw = torch.from_numpy(vo.view(np.int16)).view(torch.bfloat16)
    check(out.cpu(), q, kw, vw, L, table, head_dim**-0.5)

    # cross-attention over staged pages, 2 requests x 2 beams
    class _Attn:
        pass

    class _Layer:
        pass

    E = [70, 33]
    npg = [math.ceil(e / bs) for e in E]
    NBc = sum(npg) + 2
    kcc = torch.randn(NBc, H, bs, head_dim, generator=g).to(torch.bfloat16)
    vcc = torch.randn(NBc, H, bs, head_dim, generator=g).to(torch.bfloat16)
    perm = torch.randperm(NBc, generator=g).to(torch.int32)
    pages = [perm[: npg[0]], perm[npg[0]: npg[0] + npg[1]]]
    row_pages = [pages[0], pages[0], pages[1], pages[1]]
    row_E = [E[0], E[0], E[1], E[1]]
    layer = _Layer()
    layer.encoder_attn = _Attn()
    layer.encoder_attn.k_cache = kcc.to(DEV)
    layer.encoder_attn.v_cache = hip_attn.v_cache_from_logical(vcc).to(DEV)
    layer.encoder_attn.num_heads, layer.encoder_attn.head_dim = H, head_dim
    staged = attention.stage_cross([layer], [p.to(DEV) for p in row_pages], row_E, bs, "gfx950")
    qc = torch.randn(4, H, head_dim, generator=g).to(torch.bfloat16)
    set_context(query_start_loc=torch.arange(5, dtype=torch.int32, device=DEV),
                cross_staged=staged)
    try:
        co = attention.decoder_cross_attention(qc.to(DEV), 0, head_dim**-0.5)
    finally:
        set_context()
    torch.cuda.synchronize()
    tab = torch.nn.utils.rnn.pad_sequence(row_pages, batch_first=True)
    want = orc.paged_attention(as_f64(qc), as_f64(kcc), as_f64(vcc), np.array(row_E),
                               tab.numpy(), head_dim**-0.5)
    np.testing.assert_allclose(as_f64(co.cpu()), want, rtol=0.0, atol=2e-2)
