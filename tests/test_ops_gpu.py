"""The vflorence::self_attention / vflorence::cross_attention ops on the GPU: the fused
KV-write path equals the reference's two steps, the ops read the Context as the
reference's do, and they compile inside torch.compile without copying the caches."""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def hip():
    from vflorence_amd import hip_attn

    return hip_attn


def bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


def self_case(lens, dtype, seed, H=16, D=64, bs=16, extra_blocks=9):
    """Rows with private last blocks; slot = position L-1, as the block manager gives."""
    g = torch.Generator().manual_seed(seed)
    nblk = [math.ceil(L / bs) for L in lens]
    NB = sum(nblk) + extra_blocks
    perm = torch.randperm(NB, generator=g).tolist()
    width = max(nblk)
    table = torch.zeros(len(lens), width, dtype=torch.int32)
    slots, pos = [], 0
    for r, (L, nb) in enumerate(zip(lens, nblk)):
        ids = perm[pos : pos + nb]
        pos += nb
        table[r, :nb] = torch.tensor(ids, dtype=torch.int32)
        slots.append(ids[(L - 1) // bs] * bs + (L - 1) % bs)
    free = perm[pos:]
    fused = torch.randn(len(lens), 3 * H * D, generator=g).to(dtype)
    kc = torch.randn(NB, H, bs, D, generator=g).to(dtype)
    vc = torch.randn(NB, H, bs, D, generator=g).to(dtype)
    return fused, kc, vc, torch.tensor(lens, dtype=torch.int32), table, torch.tensor(
        slots, dtype=torch.int64), free


def run_both(fused, kc, vc, lens, table, slots, waves, H=16, D=64):
    hip_attn = hip()
    N = fused.shape[0]
    outs, caches = [], []
    for fuse in (False, True):
        f = fused.to(DEV)
        q, k, v = (t.reshape(N, H, D) for t in f.chunk(3, dim=-1))
        kd, vd = kc.to(DEV), vc.to(DEV)
        out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
        order = torch.tensor(hip_attn.longest_first(lens.tolist()), dtype=torch.int32, device=DEV)
        sm = hip_attn.get_scheduler_metadata(
            num_reqs=N, num_heads=H, num_kv_heads=H, head_dim=D, dtype=q.dtype, block_size=16,
            group_order=order, waves_per_workgroup=waves, fuse_kv_write=fuse)
        if fuse:
            hip_attn.self_attention_with_kv_write(q, k, v, kd, vd, out, lens.to(DEV),
                                                  slots.to(DEV), scale=D**-0.5,
                                                  block_table=table.to(DEV),
                                                  scheduler_metadata=sm)
        else:
            hip_attn.reshape_and_cache(k, v, kd, vd, slots.to(DEV))
            hip_attn.attention_with_kv_cache(q, kd, vd, out, None, lens.to(DEV), scale=D**-0.5,
                                             block_table=table.to(DEV), scheduler_metadata=sm)
        torch.cuda.synchronize()
        outs.append(out.cpu())
        caches.append((kd.cpu(), vd.cpu()))
    return outs, caches


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("waves", [1, 2, 4, 8])
def test_fused_kv_write_equals_two_steps(dtype, waves):
    lens = [1, 15, 16, 17, 32, 33, 100, 256, 1000, 1024, 2, 48]
    fused, kc, vc, L, table, slots, _ = self_case(lens, dtype, seed=waves)
    (o2, o1), ((k2, v2), (k1, v1)) = run_both(fused, kc, vc, L, table, slots, waves)
    assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
    torch.testing.assert_close(o1, o2, rtol=0, atol=0)
    # and both match the oracle
    hip_attn = hip()
    q = fused[:, : 16 * 64].reshape(len(lens), 16, 64)
    want = orc.paged_attention(q.double().numpy(), k1.double().numpy(),
                               hip_attn.v_cache_logical(v1).double().numpy(), L.numpy(),
                               table.numpy(), 64**-0.5)
    tol = dict(rtol=1e-5, atol=1e-6) if dtype == torch.float32 else dict(rtol=0, atol=2e-2)
    np.testing.assert_allclose(o1.double().numpy(), want, **tol)


def test_fused_slot_outside_the_context_is_written_without_substitution():
    lens = [40, 17, 64]
    fused, kc, vc, L, table, slots, free = self_case(lens, torch.bfloat16, seed=3)
    slots = slots.clone()
    slots[1] = free[0] * 16 + 5  # a free block nobody reads
    slots[2] = -1  # padding row: no write
    (o2, o1), ((k2, v2), (k1, v1)) = run_both(fused, kc, vc, L, table, slots, 4)
    assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
    torch.testing.assert_close(o1, o2, rtol=0, atol=0)


class _Attn:
    pass


class _Layer:
    def __init__(self, H, D, kc, vc, ck, cv):
        self.self_attn = _Attn()
        self.encoder_attn = _Attn()
        self.self_attn.k_cache, self.self_attn.v_cache = kc, vc
        self.encoder_attn.k_cache, self.encoder_attn.v_cache = ck, cv
        self.encoder_attn.num_heads, self.encoder_attn.head_dim = H, D


def test_ops_read_the_context_and_compile():
    from vflorence_amd import hip_attn
    from vflorence_amd.layers import attention
    from vflorence_amd.utils.context import set_context

    H, D = 16, 64
    lens = [5, 33, 70, 16]
    fused, kc, vc, L, table, slots, _ = self_case(lens, torch.bfloat16, seed=5)
    N = len(lens)
    g = torch.Generator().manual_seed(9)
    enc = [30, 30, 30, 50]
    pages = [torch.tensor([0, 1], dtype=torch.int32)] * 3 + [torch.tensor([2, 3, 4],
                                                                           dtype=torch.int32)]
    ck = torch.randn(8, H, 16, D, generator=g).to(torch.bfloat16).to(DEV)
    cv = torch.randn(8, H, 16, D, generator=g).to(torch.bfloat16).to(DEV)
    qc = torch.randn(N, H, D, generator=g).to(torch.bfloat16).to(DEV)

    def run(compiled: bool, fuse: bool):
        kd, vd = kc.to(DEV), vc.to(DEV)
        layer = _Layer(H, D, kd, vd, ck, cv)
        staged = attention.stage_cross([layer], pages, enc, 16, "gfx950")
        # one wave count for both paths: then they agree bit for bit
        sm = hip_attn.get_scheduler_metadata(
            num_reqs=N, num_heads=H, num_kv_heads=H, head_dim=D, dtype=torch.bfloat16,
            block_size=16, fuse_kv_write=fuse, waves_per_workgroup=2)
        set_context(context_lens=L.to(DEV), block_tables=table.to(DEV),
                    slot_mapping=slots.to(DEV),
                    query_start_loc=torch.arange(N + 1, dtype=torch.int32, device=DEV),
                    self_metadata=sm, isa="gfx950", cross_staged=staged)

        def step(qkv, qcross):
            q, k, v = (t.reshape(N, H, D) for t in qkv.chunk(3, dim=-1))
            a = attention.decoder_self_attention(q, k, v, kd, vd, D**-0.5)
            b = attention.decoder_cross_attention(qcross, 0, D**-0.5)
            return a.float().sum(-1) + b.float().sum(-1), a, b

        fn = torch.compile(step, fullgraph=True, dynamic=False) if compiled else step
        try:
            _, a, b = fn(fused.to(DEV), qc)
        finally:
            set_context()
        torch.cuda.synchronize()
        return a.cpu(), b.cpu(), kd.cpu(), vd.cpu()

    ref = run(False, False)
    for compiled, fuse in ((False, True), (True, False), (True, True)):
        got = run(compiled, fuse)
        for x, y in zip(got, ref):
            torch.testing.assert_close(x, y, rtol=0, atol=0)
    want = orc.paged_attention(qc.double().cpu().numpy(), ck.double().cpu().numpy(),
                               hip_attn.v_cache_logical(cv).double().cpu().numpy(),
                               np.array(enc), torch.nn.utils.rnn.pad_sequence(
                                   pages, batch_first=True).numpy(), D**-0.5)
    np.testing.assert_allclose(ref[1].double().numpy(), want, rtol=0, atol=2e-2)
