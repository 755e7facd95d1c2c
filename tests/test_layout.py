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


def test_balanced_order_pairs_long_and_short_groups_per_cu():
    """balanced_order is longest_first with alternate runs reversed: a permutation whose
    per-CU position sets (p, p + run, p + 2 run, ...) carry near-equal total length."""
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(256, 1025, (64,), generator=g).tolist()
    lf = hip_attn.longest_first(lens)
    for run in (1, 5, 16, 64, 100):
        order = hip_attn.balanced_order(lens, run)
        assert sorted(order) == list(range(64))
        assert order[:run] == lf[:run]  # the first run is still longest first
    order = hip_attn.balanced_order(lens, 16)
    assert order[16:32] == lf[16:32][::-1] and order[32:48] == lf[32:48]
    spread = lambda o: (lambda t: max(t) - min(t))(
        [sum(lens[o[p + 16 * k]] for k in range(4)) for p in range(16)])
    assert spread(order) < spread(lf)
    assert hip_attn.balanced_order(lens, 1) == lf
