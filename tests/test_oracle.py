"""Pins the CPU oracle before the HIP kernels are compared against it.

Each check is independent of the oracle's own formula: a library routine
(torch's scaled_dot_product_attention on densely gathered K/V), closed forms,
an invariance, pure-Python brute force, the reference's copy-on-write known answer,
and planted mistakes that must fail at least one check.
"""

import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def random_paged_case(rng, N=6, H=3, D=16, bs=4, pool=40, max_len=23, min_len=1):
    lens = rng.integers(min_len, max_len + 1, size=N)
    perm = rng.permutation(pool)
    width = int(max(-(-lens // bs)))
    table = np.zeros((N, width), dtype=np.int32)
    pos = 0
    for r, L in enumerate(lens):
        nb = -(-int(L) // bs)
        table[r, :nb] = perm[pos : pos + nb]
        pos += nb
    q = rng.standard_normal((N, H, D))
    kc = rng.standard_normal((pool, H, bs, D))
    vc = rng.standard_normal((pool, H, bs, D))
    return q, kc, vc, lens.astype(np.int32), table


def sdpa_reference(q, kc, vc, lens, table, scale):
    """Dense gather by hand, then torch's SDPA (a library routine), float64."""
    N, H, D = q.shape
    bs = kc.shape[2]
    out = np.zeros_like(q)
    for r in range(N):
        L = int(lens[r])
        toks = [(int(table[r][j // bs]), j % bs) for j in range(L)]
        K = np.stack([kc[b, :, o, :] for b, o in toks], axis=1)  # [H, L, D]
        V = np.stack([vc[b, :, o, :] for b, o in toks], axis=1)
        o = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[r][:, None, :]),
            torch.from_numpy(K),
            torch.from_numpy(V),
            scale=scale,
        )
        out[r] = o[:, 0, :].numpy()
    return out


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_numpy_oracle_matches_sdpa(seed):
    rng = np.random.default_rng(seed)
    q, kc, vc, lens, table = random_paged_case(rng)
    got = orc.paged_attention(q, kc, vc, lens, table, 0.25)
    want = sdpa_reference(q, kc, vc, lens, table, 0.25)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_one_token_context_returns_its_value():
    rng = np.random.default_rng(3)
    q, kc, vc, _, table = random_paged_case(rng)
    lens = np.ones(q.shape[0], dtype=np.int32)
    got = orc.paged_attention(q, kc, vc, lens, table, 0.125)
    want = vc[table[:, 0], :, 0, :]
    np.testing.assert_array_equal(got, want)


def test_equal_keys_give_mean_of_values():
    rng = np.random.default_rng(4)
    q, kc, vc, lens, table = random_paged_case(rng)
    kc[:] = 0.7
    got = orc.paged_attention(q, kc, vc, lens, table, 0.125)
    bs = kc.shape[2]
    for r, L in enumerate(lens):
        vals = np.stack([vc[table[r][j // bs], :, j % bs, :] for j in range(L)])
        np.testing.assert_allclose(got[r], vals.mean(axis=0), rtol=1e-12, atol=1e-13)


def test_block_permutation_invariance():
    rng = np.random.default_rng(5)
    q, kc, vc, lens, table = random_paged_case(rng)
    pool = kc.shape[0]
    sigma = rng.permutation(pool)  # physical block b moves to sigma[b]
    kc2, vc2 = np.empty_like(kc), np.empty_like(vc)
    kc2[sigma] = kc
    vc2[sigma] = vc
    table2 = sigma[table].astype(np.int32)
    a = orc.paged_attention(q, kc, vc, lens, table, 0.3)
    b = orc.paged_attention(q, kc2, vc2, lens, table2, 0.3)
    np.testing.assert_array_equal(a, b)


def test_bruteforce_tiny():
    rng = np.random.default_rng(6)
    q, kc, vc, lens, table = random_paged_case(rng, N=3, H=2, D=4, bs=2, pool=12, max_len=7)
    got = orc.paged_attention(q, kc, vc, lens, table, 0.5)
    want = orc.paged_attention_bruteforce(q, kc, vc, lens, table, 0.5)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_zero_length_rows_and_clamp():
    rng = np.random.default_rng(7)
    q, kc, vc, lens, table = random_paged_case(rng)
    lens = lens.copy()
    lens[0] = 0
    got = orc.paged_attention(q, kc, vc, lens, table, 0.3)
    assert not got[0].any()
    # A length past the table width attends to the whole table.
    bs, width = kc.shape[2], table.shape[1]
    lens2 = lens.copy()
    lens2[1] = width * bs + 100
    lens3 = lens.copy()
    lens3[1] = width * bs
    np.testing.assert_array_equal(
        orc.paged_attention(q, kc, vc, lens2, table, 0.3)[1],
        orc.paged_attention(q, kc, vc, lens3, table, 0.3)[1],
    )


# --- planted mistakes: each must be caught by the SDPA check --------------------
def _mut_no_scale(q, kc, vc, lens, table, scale):
    return orc.paged_attention(q, kc, vc, lens, table, 1.0)


def _mut_drop_last_token(q, kc, vc, lens, table, scale):
    return orc.paged_attention(q, kc, vc, np.maximum(lens - 1, 1), table, scale)


def _mut_swap_kv(q, kc, vc, lens, table, scale):
    return orc.paged_attention(q, vc, kc, lens, table, scale)


def _mut_transposed_block(q, kc, vc, lens, table, scale):
    # head and in-block token offset swapped in the gather (needs H == block_size)
    assert kc.shape[1] == kc.shape[2]
    return orc.paged_attention(q, kc.transpose(0, 2, 1, 3), vc.transpose(0, 2, 1, 3), lens, table,
                               scale)


@pytest.mark.parametrize("mutant", [_mut_no_scale, _mut_drop_last_token, _mut_swap_kv])
def test_planted_mistakes_are_caught(mutant):
    rng = np.random.default_rng(8)
    q, kc, vc, lens, table = random_paged_case(rng, min_len=2)
    want = sdpa_reference(q, kc, vc, lens, table, 0.25)
    got = mutant(q, kc, vc, lens, table, 0.25)
    assert not np.allclose(got, want, rtol=1e-6, atol=1e-6)


def test_planted_transposed_gather_is_caught():
    rng = np.random.default_rng(9)
    q, kc, vc, lens, table = random_paged_case(rng, H=4, bs=4, min_len=2)
    want = sdpa_reference(q, kc, vc, lens, table, 0.25)
    got = _mut_transposed_block(q, kc, vc, lens, table, 0.25)
    assert not np.allclose(got, want, rtol=1e-6, atol=1e-6)


# --- C restatement against the numpy one ------------------------------------------
@pytest.mark.parametrize("code", [orc.F32, orc.BF16, orc.F16])
def test_c_oracle_matches_numpy(code):
    rng = np.random.default_rng(10 + code)
    q, kc, vc, lens, table = random_paged_case(rng, N=9, H=4, D=64, bs=16, pool=64,
                                               max_len=150)
    if code == orc.F32:
        qs, ks, vs = (x.astype(np.float32) for x in (q, kc, vc))
        qv, kv, vv = qs, ks, vs
    elif code == orc.BF16:
        qs, ks, vs = (orc.f64_to_bf16_bits(x) for x in (q, kc, vc))
        qv, kv, vv = (orc.bf16_bits_to_f64(x) for x in (qs, ks, vs))
    else:
        qs, ks, vs = (x.astype(np.float16).view(np.uint16) for x in (q, kc, vc))
        qv, kv, vv = (x.view(np.float16).astype(np.float64) for x in (qs, ks, vs))
    want = orc.paged_attention(qv, kv, vv, lens, table, 0.125)
    got = orc.paged_attention_c(qs, ks, vs, lens, table, 0.125, dtype_code=code, num_threads=2)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_c_oracle_strided_query():
    rng = np.random.default_rng(20)
    q, kc, vc, lens, table = random_paged_case(rng, N=5, H=4, D=64, bs=16, pool=32, max_len=90)
    fused = np.zeros((5, 3 * 4 * 64), dtype=np.float32)
    fused[:, : 4 * 64] = q.reshape(5, -1)
    qview = fused[:, : 4 * 64].reshape(5, 4, 64)
    got = orc.paged_attention_c(qview, kc.astype(np.float32), vc.astype(np.float32), lens, table,
                                0.125)
    want = orc.paged_attention(q.astype(np.float32), kc.astype(np.float32), vc.astype(np.float32),
                               lens, table, 0.125)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


# --- KV slot write ----------------------------------------------------------------
@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_reshape_and_cache_closed_form(impl):
    rng = np.random.default_rng(30)
    T, H, D, bs, pool = 11, 3, 8, 4, 9
    fused = rng.integers(0, 2**16, size=(T, 3 * H * D), dtype=np.uint16)
    key = fused[:, H * D : 2 * H * D].reshape(T, H, D)
    value = fused[:, 2 * H * D :].reshape(T, H, D)
    kc = rng.integers(0, 2**16, size=(pool, H, bs, D), dtype=np.uint16)
    vc = rng.integers(0, 2**16, size=(pool, H, bs, D), dtype=np.uint16)
    k0, v0 = kc.copy(), vc.copy()
    slots = rng.choice(pool * bs, size=T, replace=False).astype(np.int64)
    slots[3] = -1  # padding token: skipped
    (orc.reshape_and_cache if impl == "numpy" else orc.reshape_and_cache_c)(
        key, value, kc, vc, slots)
    written = np.zeros((pool, bs), dtype=bool)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        np.testing.assert_array_equal(kc[s // bs, :, s % bs, :], key[t])
        np.testing.assert_array_equal(vc[s // bs, :, s % bs, :], value[t])
        written[s // bs, s % bs] = True
    untouched = ~written
    np.testing.assert_array_equal(kc.transpose(0, 2, 1, 3)[untouched], k0.transpose(0, 2, 1, 3)[untouched])
    np.testing.assert_array_equal(vc.transpose(0, 2, 1, 3)[untouched], v0.transpose(0, 2, 1, 3)[untouched])


def test_slot_formulas():
    table = [7, 2, 9]
    bs = 16
    assert orc.slot_for(table, 0, bs) == 7 * 16
    assert orc.slot_for(table, 17, bs) == 2 * 16 + 1
    assert orc.slot_for(table, 47, bs) == 9 * 16 + 15
    assert orc.context_len_for(47) == 48
    pages = np.array([[5, 1], [3, 8]], dtype=np.int32)
    np.testing.assert_array_equal(
        orc.cross_slots(pages, 18, bs),
        np.concatenate([5 * 16 + np.arange(16), 1 * 16 + np.arange(2),
                        3 * 16 + np.arange(16), 8 * 16 + np.arange(2)]),
    )


# --- copy-on-write ------------------------------------------------------------------
def load_kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_copy_blocks_reference_kat(impl):
    kat = load_kats()["copy_on_write"]
    caches = []
    for _ in range(kat["num_caches"]):
        c = np.zeros((kat["num_blocks"], 2, 4, 8), dtype=np.float32)
        for b in range(kat["num_blocks"]):
            c[b] = b
        caches.append(c)
    pairs = [tuple(p) for p in kat["pairs"]]
    (orc.copy_blocks if impl == "numpy" else orc.copy_blocks_c)(caches, pairs)
    for c in caches:
        assert [float(np.unique(c[b])[0]) for b in range(len(kat["expected_unique"]))] == \
            kat["expected_unique"]


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_copy_blocks_gathers_before_scattering(impl):
    c = np.stack([np.full((2, 4, 8), b, dtype=np.float32) for b in range(5)])
    (orc.copy_blocks if impl == "numpy" else orc.copy_blocks_c)([c], [(0, 1), (1, 2)])
    assert [float(c[b, 0, 0, 0]) for b in range(5)] == [0, 0, 1, 3, 4]


def test_bf16_conversion_round_trip():
    bits = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16)
    vals = orc.bf16_bits_to_f64(bits)
    finite = np.isfinite(vals)
    back = orc.f64_to_bf16_bits(vals[finite])
    np.testing.assert_array_equal(back, bits[finite])
    # torch's float -> bfloat16 rounding agrees on random floats
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32)
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.f64_to_bf16_bits(x), t)
