"""TEST INFRASTRUCTURE, NOT PRODUCT CODE: CPU oracle of vflorence's decode attention path.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg use this
module, as the reference results the tests compare against and as the timed CPU
baseline.  ``vflorence_amd`` never imports it.

Two restatements of the same algorithm:

* numpy, float64 (``paged_attention``, ``reshape_and_cache``, ``copy_blocks``): the
  parity reference for tests.
* C, float32 accumulation, OpenMP (``paged_attention_c`` ...; oracle/paged_attention.c,
  built by oracle/Makefile into oracle/_build/liboracle.so): cross-checks the numpy
  version and is the CPU baseline bench.py times.

What each function restates (the reference's arithmetic is in the external package
vllm-cpu-attn 0.1.0, git 79b2eb02549b3e047bc80df51321bc7281f851c9, uv.lock:1091-1093,
absent from /root/reference; these follow its call sites):

* ``reshape_and_cache``: vflorence/layers/attention.py:55-57 and
  vflorence/engine/model_runner.py:252-259 -- cache[slot // bs, h, slot % bs] = key[t, h].
* ``paged_attention``: vflorence/layers/attention.py:61-72 (self) and :98-109 (cross) --
  out[r] = softmax(scale q K^T) V over the first seq_lens[r] tokens of the pages in
  block_table[r]; one query per sequence (query_start_loc = arange(N+1),
  vflorence/engine/model_runner.py:306).
* ``copy_blocks``: vflorence/engine/model_runner.py:162-167 -- per cache,
  index_copy_(0, dst, index_select(0, src)).
* ``slot_for``/``context_len_for``: vflorence/engine/model_runner.py:296-299.
* ``cross_slots``: vflorence/engine/model_runner.py:233-242.

How they are pinned (tests/test_oracle.py): torch.nn.functional.scaled_dot_product_attention
on densely gathered K/V, closed forms (a one-token context returns v; equal keys
return the mean of the values), block-permutation invariance, pure-Python brute force
on tiny inputs, the copy-on-write known answer of the reference's
tests/test_engine.py:382-405, and planted mistakes that must fail those checks.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

F32, BF16, F16 = 0, 1, 2


# ---------------------------------------------------------------------------
# element conversions (numpy has no bfloat16)
# ---------------------------------------------------------------------------
def bf16_bits_to_f64(bits: np.ndarray) -> np.ndarray:
    """uint16/int16 bfloat16 bit patterns -> float64 values (exact)."""
    u = bits.astype(np.uint16).astype(np.uint32) << 16
    with np.errstate(invalid="ignore"):  # NaN payloads survive as NaN
        return u.view(np.float32).astype(np.float64)


def f64_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float -> bfloat16 bits, round to nearest even (NaN -> 0x7fc0)."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


# ---------------------------------------------------------------------------
# numpy float64 restatement
# ---------------------------------------------------------------------------
def slot_for(block_table: list[int], pos: int, block_size: int) -> int:
    """Cache slot of position ``pos`` (vflorence/engine/model_runner.py:296-298)."""
    return block_table[pos // block_size] * block_size + pos % block_size


def context_len_for(pos: int) -> int:
    """Tokens attended by the token at ``pos``, itself included (model_runner.py:299)."""
    return pos + 1


def cross_slots(pages: np.ndarray, enc_len: int, block_size: int) -> np.ndarray:
    """Slots of a group's encoder tokens (vflorence/engine/model_runner.py:240-242).

    ``pages`` is [G, ceil(enc_len / bs)]; returns int64 [G * enc_len].
    """
    token = np.arange(enc_len)
    slots = pages[:, token // block_size].astype(np.int64) * block_size
    return (slots + token % block_size).reshape(-1)


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping) -> None:
    """In place: cache[slot // bs, h, slot % bs, :] = key[t, h, :]; negative slots skipped."""
    num_blocks, _, block_size, _ = k_cache.shape
    for t, slot in enumerate(np.asarray(slot_mapping).tolist()):
        if slot < 0 or slot >= num_blocks * block_size:
            continue
        k_cache[slot // block_size, :, slot % block_size, :] = key[t]
        v_cache[slot // block_size, :, slot % block_size, :] = value[t]


def copy_blocks(caches, pairs) -> None:
    """In place, per cache: gather every src block, then write them to the dst blocks."""
    if not pairs:
        return
    src = np.array([s for s, _ in pairs], dtype=np.int64)
    dst = np.array([d for _, d in pairs], dtype=np.int64)
    for cache in caches:
        gathered = cache[src].copy()
        cache[dst] = gathered


def gather_context(cache: np.ndarray, block_row, length: int) -> np.ndarray:
    """[H, length, D] view of one sequence's first ``length`` tokens."""
    num_blocks, H, bs, D = cache.shape
    nb = -(-length // bs)
    blocks = np.asarray(block_row[:nb], dtype=np.int64)
    dense = cache[blocks]  # [nb, H, bs, D]
    return dense.transpose(1, 0, 2, 3).reshape(H, nb * bs, D)[:, :length]


def paged_attention(q, k_cache, v_cache, seq_lens, block_table, scale) -> np.ndarray:
    """float64 paged decode attention; q [N, H, D] -> out [N, H, D].

    Rows with seq_lens <= 0 give zeros; lengths are clamped to the table width.
    """
    q = np.asarray(q, dtype=np.float64)
    k_cache = np.asarray(k_cache, dtype=np.float64)
    v_cache = np.asarray(v_cache, dtype=np.float64)
    N, H, D = q.shape
    bs = k_cache.shape[2]
    width = block_table.shape[1]
    out = np.zeros((N, H, D), dtype=np.float64)
    for r in range(N):
        L = min(int(seq_lens[r]), width * bs)
        if L <= 0:
            continue
        K = gather_context(k_cache, block_table[r], L)  # [H, L, D]
        V = gather_context(v_cache, block_table[r], L)
        s = np.einsum("hd,hld->hl", q[r], K) * scale
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[r] = np.einsum("hl,hld->hd", p, V)
    return out


def paged_attention_bruteforce(q, k_cache, v_cache, seq_lens, block_table, scale):
    """Pure-Python loops over tokens and dims; small inputs only."""
    import math

    N, H, D = q.shape
    bs = k_cache.shape[2]
    out = [[[0.0] * D for _ in range(H)] for _ in range(N)]
    for r in range(N):
        L = int(seq_lens[r])
        for h in range(H):
            scores = []
            for j in range(L):
                blk = int(block_table[r][j // bs])
                krow = k_cache[blk][h][j % bs]
                scores.append(scale * sum(float(q[r][h][d]) * float(krow[d]) for d in range(D)))
            if not scores:
                continue
            mx = max(scores)
            w = [math.exp(s - mx) for s in scores]
            tot = sum(w)
            for d in range(D):
                acc = 0.0
                for j in range(L):
                    blk = int(block_table[r][j // bs])
                    acc += w[j] * float(v_cache[blk][h][j % bs][d])
                out[r][h][d] = acc / tot
    return np.array(out, dtype=np.float64)


# ---------------------------------------------------------------------------
# C restatement (float32 accumulation, OpenMP)
# ---------------------------------------------------------------------------
_clib = None


def build_c(force: bool = False) -> str:
    """Compile oracle/paged_attention.c with oracle/Makefile."""
    import subprocess

    if force or not os.path.exists(LIB_PATH):
        cmd = ["make", "-C", HERE] + (["-B"] if force else [])
        subprocess.run(cmd, check=True, capture_output=True)
    return LIB_PATH


def clib() -> ctypes.CDLL:
    global _clib
    if _clib is None:
        if not os.path.exists(LIB_PATH):
            build_c()
        lib = ctypes.CDLL(LIB_PATH)
        vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        lib.oracle_reshape_and_cache.restype = None
        lib.oracle_reshape_and_cache.argtypes = [vp, vp, i64, i64, i64, i64, vp, vp, vp, i64, i32,
                                                 i32, i32, i64, i32]
        lib.oracle_copy_blocks.restype = i32
        lib.oracle_copy_blocks.argtypes = [vp, i32, vp, vp, i64, i64, i64]
        lib.oracle_paged_attention.restype = i32
        lib.oracle_paged_attention.argtypes = [vp, i64, i64, vp, vp, vp, vp, vp, i64, i32, i64, i32,
                                               i32, i32, i64, f32, i32, i32]
        _clib = lib
    return _clib


def _code(arr: np.ndarray, dtype_code: int | None) -> int:
    if dtype_code is not None:
        return dtype_code
    if arr.dtype == np.float32:
        return F32
    raise ValueError("pass dtype_code for 16-bit storage (BF16 or F16)")


def paged_attention_c(q, k_cache, v_cache, seq_lens, block_table, scale, dtype_code=None,
                      num_threads: int = 0) -> np.ndarray:
    """C restatement; arrays hold raw storage (float32, or uint16 bits with dtype_code).

    q may be a strided [N, H, D] view with a contiguous last dim; caches contiguous.
    Returns float32 [N, H, D].
    """
    code = _code(q, dtype_code)
    esz = q.itemsize
    assert q.strides[2] == esz
    k_cache = np.ascontiguousarray(k_cache)
    v_cache = np.ascontiguousarray(v_cache)
    seq_lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    block_table = np.ascontiguousarray(block_table, dtype=np.int32)
    N, H, D = q.shape
    nb, _, bs, _ = k_cache.shape
    out = np.zeros((N, H, D), dtype=np.float32)
    rc = clib().oracle_paged_attention(
        q.ctypes.data, q.strides[0] // esz, q.strides[1] // esz, k_cache.ctypes.data,
        v_cache.ctypes.data, out.ctypes.data, seq_lens.ctypes.data, block_table.ctypes.data,
        block_table.shape[1], block_table.shape[1], N, H, D, bs, nb, float(scale), code,
        int(num_threads),
    )
    if rc != 0:
        raise MemoryError("oracle_paged_attention: allocation failed")
    return out


def reshape_and_cache_c(key, value, k_cache, v_cache, slot_mapping) -> None:
    slot_mapping = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    esz = key.itemsize
    nb, H, bs, D = k_cache.shape
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    clib().oracle_reshape_and_cache(
        key.ctypes.data, value.ctypes.data, key.strides[0] // esz, key.strides[1] // esz,
        value.strides[0] // esz, value.strides[1] // esz, k_cache.ctypes.data,
        v_cache.ctypes.data, slot_mapping.ctypes.data, key.shape[0], H, D, bs, nb, esz,
    )


def copy_blocks_c(caches, pairs) -> None:
    if not pairs:
        return
    src = np.array([s for s, _ in pairs], dtype=np.int64)
    dst = np.array([d for _, d in pairs], dtype=np.int64)
    for c in caches:
        assert c.flags.c_contiguous
    ptrs = (ctypes.c_void_p * len(caches))(*[c.ctypes.data for c in caches])
    block_bytes = caches[0][0].nbytes
    rc = clib().oracle_copy_blocks(ptrs, len(caches), src.ctypes.data, dst.ctypes.data,
                                   len(pairs), block_bytes, caches[0].shape[0])
    if rc != 0:
        raise MemoryError("oracle_copy_blocks: allocation failed")
