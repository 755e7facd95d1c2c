"""Cross-attention at the workload shapes, through ``stage_cross`` (both staging paths),
against the float64 oracle:

* BART-large 4-beam: 64 requests x 4 beams, 16 heads, encoder lengths U[256, 1024];
* Florence-2-base 3-beam: 128 requests x 3 beams, 12 heads, 577 visual + 10 prompt
  tokens of encoder K/V per request.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _Attn:
    pass


class _Layer:
    def __init__(self, k, v, heads, head_dim):
        self.encoder_attn = _Attn()
        self.encoder_attn.k_cache, self.encoder_attn.v_cache = k, v
        self.encoder_attn.num_heads, self.encoder_attn.head_dim = heads, head_dim


def bf16_bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def run_cross(case, heads, fixed_buffers: bool):
    from vflorence_amd import hip_attn
    from vflorence_amd.layers import attention

    layer = _Layer(case.k_cache, case.v_cache, heads, case.query.shape[-1])
    buffers = None
    if fixed_buffers:
        max_pages = max(len(p) for p in case.pages)
        buffers = attention.CrossStagingBuffers(len(case.pages) + 5, max_pages + 3, DEV)
    (k, v, table, lens, meta), = attention.stage_cross([layer], case.pages, case.enc_lens, 16,
                                                       "gfx950", buffers=buffers)
    out = torch.empty_like(case.query)
    hip_attn.attention_with_kv_cache(case.query, k, v, out, None, lens, scale=case.scale,
                                     block_table=table, scheduler_metadata=meta)
    torch.cuda.synchronize()
    return out


def oracle_cross(case):
    table = torch.nn.utils.rnn.pad_sequence(case.pages, batch_first=True).numpy()
    used, remapped = np.unique(table, return_inverse=True)
    from vflorence_amd import hip_attn

    kc = orc.bf16_bits_to_f64(bf16_bits(case.k_cache)[used])
    vc = orc.bf16_bits_to_f64(bf16_bits(hip_attn.v_cache_logical(case.v_cache))[used])
    q = orc.bf16_bits_to_f64(bf16_bits(case.query))
    return orc.paged_attention(q, kc, vc, np.array(case.enc_lens),
                               remapped.reshape(table.shape).astype(np.int32), case.scale)


@pytest.mark.parametrize("fixed", [False, True], ids=["fresh", "fixed-buffers"])
def test_bart_large_4beam_cross_attention(fixed):
    from vflorence_amd import workloads

    case = workloads.cross_attention_case(device=DEV, seed=3)
    out = run_cross(case, 16, fixed)
    want = oracle_cross(case)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, rtol=0, atol=2e-2)


@pytest.mark.parametrize("fixed", [False, True], ids=["fresh", "fixed-buffers"])
def test_florence2_base_3beam_cross_attention(fixed):
    """Florence-2-base text decoder: d_model 768 -> 12 heads x 64; each request's
    encoder output is 577 visual tokens + a 10-token prompt, N(0,1) features."""
    from vflorence_amd import workloads

    case = workloads.cross_attention_case(num_requests=128, beams=3, num_heads=12,
                                          enc_lens=[587] * 128, device=DEV, seed=4,
                                          pool_blocks=128 * math.ceil(587 / 16))
    out = run_cross(case, 12, fixed)
    want = oracle_cross(case)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, rtol=0, atol=2e-2)


def test_fixed_buffers_serve_changing_batches_at_one_address():
    """Successive batches of the same row count reuse the staging addresses; each
    batch's result matches the oracle (the staging is refreshed, not stale)."""
    from vflorence_amd import hip_attn, workloads
    from vflorence_amd.layers import attention

    buffers = attention.CrossStagingBuffers(64, 70, DEV)
    ptrs = set()
    for seed, beams in ((5, 4), (6, 2), (7, 1)):
        case = workloads.cross_attention_case(num_requests=64 // beams, beams=beams, device=DEV,
                                              seed=seed)
        layer = _Layer(case.k_cache, case.v_cache, 16, 64)
        (k, v, table, lens, meta), = attention.stage_cross([layer], case.pages, case.enc_lens, 16,
                                                           "gfx950", buffers=buffers)
        ptrs.add((table.data_ptr(), lens.data_ptr(), meta.group_start.data_ptr(),
                  meta.group_order.data_ptr()))
        out = torch.empty_like(case.query)
        hip_attn.attention_with_kv_cache(case.query, k, v, out, None, lens, scale=case.scale,
                                         block_table=table, scheduler_metadata=meta)
        torch.cuda.synchronize()
        np.testing.assert_allclose(out.double().cpu().numpy(), oracle_cross(case), rtol=0,
                                   atol=2e-2)
    assert len(ptrs) == 1
