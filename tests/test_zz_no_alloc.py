"""vfl_copy_blocks_noalloc (the copy-on-write entry point that allocates nothing: its
staging buffer is the library's per-GPU array) against vfl_copy_blocks with a
caller-allocated staging buffer, through the C ABI: two calls in a row on the same
pools, the second smaller, staged (destinations that are also sources) and direct,
bit for bit, and against the oracle's gather-then-scatter."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy()


def overlapping_pairs(rng, num_blocks, n):
    """``n`` pairs whose destinations are distinct and include sources of other pairs
    (chains and cycles of a permutation), so only gather-then-scatter is right."""
    blocks = rng.permutation(num_blocks)[: n + 1]
    src = blocks[:n].copy()
    dst = np.roll(blocks[:n], 1)
    dst[0] = blocks[n]  # one chain end outside the sources
    return [(int(s), int(d)) for s, d in zip(src, dst)]


def copy_with(entry, caches, ptrs, pairs, staged):
    from vflorence_amd._lib import check, lib

    src = torch.tensor([s for s, _ in pairs], dtype=torch.int64, device=DEV)
    dst = torch.tensor([d for _, d in pairs], dtype=torch.int64, device=DEV)
    block_bytes = caches[0][0].numel() * caches[0].element_size()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (ptrs.data_ptr(), len(caches), src.data_ptr(), dst.data_ptr(), len(pairs),
            block_bytes, caches[0].shape[0])
    if entry == "noalloc":
        check(lib.vfl_copy_blocks_noalloc(*args, int(staged), stream))
    else:
        staging = (torch.empty(len(caches) * len(pairs) * block_bytes, dtype=torch.uint8,
                               device=DEV) if staged else None)
        check(lib.vfl_copy_blocks(*args, None if staging is None else staging.data_ptr(),
                                  stream))
        torch.cuda.synchronize()
        del staging
    torch.cuda.synchronize()


@pytest.mark.parametrize("shape,counts", [
    ((24, 256, 16, 16, 64), (85, 10)),  # BART-large pools: 24 x 85 x 32 KiB fills 64 MiB
    ((6, 64, 4, 16, 64), (40, 7)),
])
def test_noalloc_copy_equals_the_allocating_copy(shape, counts):
    from vflorence_amd import hip_attn
    from vflorence_amd._lib import NOALLOC_STAGING_BYTES

    num_caches, nb, h, bs, d = shape
    g = torch.Generator(device=DEV).manual_seed(sum(shape))
    base = [torch.randn(nb, h, bs, d, generator=g, device=DEV).to(torch.bfloat16)
            for _ in range(num_caches)]
    a = [c.clone() for c in base]
    b = [c.clone() for c in base]
    host = [bits(c) for c in base]
    pa, pb = hip_attn.cache_pointer_table(a), hip_attn.cache_pointer_table(b)
    rng = np.random.default_rng(nb)
    block_bytes = h * bs * d * 2
    for n in counts:  # two calls in a row, the second smaller
        assert num_caches * n * block_bytes <= NOALLOC_STAGING_BYTES
        pairs = overlapping_pairs(rng, nb, n)
        assert hip_attn.copy_pairs_need_staging(pairs)
        copy_with("alloc", a, pa, pairs, staged=True)
        copy_with("noalloc", b, pb, pairs, staged=True)
        orc.copy_blocks(host, pairs)
        for ca, cb, ch in zip(a, b, host):
            assert np.array_equal(bits(ca), bits(cb))
            assert np.array_equal(bits(cb), ch)
    # a direct pass (no destination is a source) after the staged ones
    free = sorted(set(range(nb)) - {s for s, _ in pairs} - {d for _, d in pairs})
    direct = [(s, dd) for (s, _), dd in zip(pairs, free[: len(pairs)])]
    assert not hip_attn.copy_pairs_need_staging(direct)
    copy_with("alloc", a, pa, direct, staged=False)
    copy_with("noalloc", b, pb, direct, staged=False)
    orc.copy_blocks(host, direct)
    for ca, cb, ch in zip(a, b, host):
        assert np.array_equal(bits(ca), bits(cb)) and np.array_equal(bits(cb), ch)


def test_noalloc_copy_refuses_staging_beyond_its_buffer():
    from vflorence_amd import hip_attn
    from vflorence_amd._lib import NOALLOC_STAGING_BYTES, lib

    caches = [torch.zeros(128, 16, 16, 64, dtype=torch.bfloat16, device=DEV) for _ in range(24)]
    ptrs = hip_attn.cache_pointer_table(caches)
    n = NOALLOC_STAGING_BYTES // (24 * 32768) + 1
    idx = torch.arange(n, dtype=torch.int64, device=DEV)
    rc = lib.vfl_copy_blocks_noalloc(ptrs.data_ptr(), 24, idx.data_ptr(), (idx + 1).data_ptr(),
                                     n, 32768, 128, 1, None)
    assert rc == -1 and b"exceeds" in lib.vfl_last_error()
