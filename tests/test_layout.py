"""The device layout of V pools: the logical view helpers invert each other and agree
with the element formula the kernels use (include/vflorence_amd.h)."""

import pytest
import torch

from vflorence_amd import hip_attn


def vtile_index(t, d, D):
    return ((t >> 2) * D + d) * 4 + (t & 3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_v_layout_helpers(dtype, D):
    nb, h, bs = 3, 2, 16
    logical = torch.randn(nb, h, bs, D).to(dtype)
    phys = hip_attn.v_cache_from_logical(logical)
    assert phys.shape == logical.shape and phys.is_contiguous()
    assert torch.equal(hip_attn.v_cache_logical(phys), logical)
    flat = phys.view(nb, h, -1)
    for t in range(bs):
        for d in (0, 1, 17, D - 1):
            idx = vtile_index(t, d, D) if hip_attn.v_tile_interleaved(dtype) else t * D + d
            assert torch.equal(flat[:, :, idx], logical[:, :, t, d])


def test_whole_block_fill_is_layout_independent():
    """The reference's copy-on-write test fills blocks with their id
    (tests/test_engine.py:396-405); such fills read the same in any layout."""
    v = torch.zeros(4, 2, 16, 64, dtype=torch.bfloat16)
    for b in range(4):
        v[b] = b
    assert [hip_attn.v_cache_logical(v)[b].unique().item() for b in range(4)] == [0, 1, 2, 3]
