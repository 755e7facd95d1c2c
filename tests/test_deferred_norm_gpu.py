"""Deferred LayerNorm across the decoder's projections (vflorence_amd::linear_residual,
::linear_norm, ::layer_norm_apply): a sublayer's output projection stores the pre-norm
sum and its per-32-feature statistics, the projections that read the LayerNorm's output
fold it into their weights.  Checked against float64 torch references and against the
separate residual + LayerNorm kernel path on the same inputs."""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ops():
    from vflorence_amd import decoder_ops

    return decoder_ops


def ulp(t, dtype):
    """One unit in the last place of dtype at |t| (t float64)."""
    bits = 8 if dtype == torch.bfloat16 else 11
    e = torch.floor(torch.log2(t.abs().clamp_min(2.0**-60)))
    return torch.pow(2.0, e - bits + 1)


def tile_stats(v):
    """(mean, sum of squared deviations) of every 32-feature tile, float64."""
    t = v.double().view(v.shape[0], -1, 32)
    mean = t.mean(-1)
    return torch.stack([mean, ((t - mean[..., None]) ** 2).sum(-1)], -1)


def layer_norm64(v, gamma, beta, eps):
    return F.layer_norm(v.double(), (v.shape[-1],), gamma.double(), beta.double(), eps)


def unpack(packed, rows, cols):
    r = (rows + 31) // 32 * 32
    return packed.view(r // 16, cols // 32, 4, 16, 8).permute(0, 3, 1, 2, 4).reshape(r, cols)[:rows]


def rand(shape, g, dtype, scale=1.0, shift=0.0):
    return (torch.randn(*shape, device=DEV, generator=g) * scale + shift).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,d,inner", [(1, 1024, 1024), (7, 1024, 1024), (64, 768, 768),
                                          (256, 1024, 1024), (33, 512, 2048)])
def test_residual_plain_is_the_separate_projection_plus_rounded_add(dtype, rows, d, inner):
    """v = rnd(rnd(x W^T + b) + h) bit for bit (the projection's own rounding, then the
    residual add's), and every 32-feature tile's statistics of v."""
    g = torch.Generator(device=DEV).manual_seed(rows + d)
    x = rand((rows, inner), g, dtype)
    w = rand((d, inner), g, dtype, inner**-0.5)
    b = rand((d,), g, dtype)
    h = rand((rows, d), g, dtype, 2.0, 0.5)
    packed = ops().pack_linear_weight(w)
    print(f"[deferred] residual plain {dtype} rows {rows} d {d} in {inner}", flush=True)
    v, st = ops().linear_residual(x, packed, b, h, None, None, None, 0.0, d)
    y = ops().linear(x, packed, b, d)
    torch.cuda.synchronize()
    want = (y.float() + h.float()).to(dtype)
    assert torch.equal(v, want)
    ref = tile_stats(want)
    assert torch.allclose(st.double(), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [3, 64, 256])
def test_residual_deferred_normalizes_the_earlier_sum(dtype, rows):
    """The residual given as an earlier call's (v0, stats): v = rnd(y + rnd(LN(v0))), with
    LN from the tile statistics -- within one rounding of each step of the float64
    LayerNorm's value (the statistics are combined in a different order).  Also through
    a packed x (the feed-forward pair's second projection)."""
    d, inner = 1024, 4096
    g = torch.Generator(device=DEV).manual_seed(rows)
    x0 = rand((rows, d), g, dtype)
    w0 = rand((d, d), g, dtype, d**-0.5)
    h0 = rand((rows, d), g, dtype, 3.0, 1.0)
    v0, st0 = ops().linear_residual(x0, ops().pack_linear_weight(w0), None, h0, None, None, None,
                                    0.0, d)
    gamma = rand((d,), g, dtype, 0.2, 1.0)
    beta = rand((d,), g, dtype, 0.1)
    eps = 1e-5
    w1 = rand((inner, d), g, dtype, d**-0.5)
    w2 = rand((d, inner), g, dtype, inner**-0.5)
    b2 = rand((d,), g, dtype)
    mid = ops().linear(rand((rows, d), g, dtype), ops().pack_linear_weight(w1), None, inner,
                       flags=ops().LINEAR_GELU | ops().LINEAR_Y_PACKED)
    p2 = ops().pack_linear_weight(w2)
    print(f"[deferred] residual deferred {dtype} rows {rows}", flush=True)
    v, st = ops().linear_residual(mid, p2, b2, v0, st0, gamma, beta, eps, d, rows=rows,
                                  flags=ops().LINEAR_X_PACKED)
    y = ops().linear(mid, p2, b2, d, rows=rows, flags=ops().LINEAR_X_PACKED)
    torch.cuda.synchronize()
    hn = layer_norm64(v0, gamma, beta, eps)
    want = y.double() + hn
    err = (v.double() - want).abs()
    # rnd(LN) then rnd(sum): at most one unit of each rounding, plus the statistics' order
    bound = ulp(hn, dtype) + ulp(want, dtype) * 1.01
    assert (err <= bound).all(), float((err - bound).max())
    assert torch.allclose(st.double(), tile_stats(v), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,d,out,gelu", [(1, 1024, 1024, False), (256, 1024, 3072, False),
                                             (64, 768, 768, False), (256, 1024, 4096, True),
                                             (17, 768, 3072, True)])
def test_folded_projection_is_as_close_as_the_separate_layer_norm(dtype, rows, d, out, gelu):
    """linear_norm(v, stats) with the LayerNorm folded into the weight against the exact
    float64 projection of LN(v): no farther from it than the separate path (LayerNorm
    kernel, rounded, then the projection) -- folding rounds W diag(gamma) where the
    separate path rounds LN(v)."""
    g = torch.Generator(device=DEV).manual_seed(rows * 3 + out)
    v = rand((rows, d), g, dtype, 2.0, 0.7)
    gamma = rand((d,), g, dtype, 0.2, 1.0)
    beta = rand((d,), g, dtype, 0.1)
    eps = 1e-5
    w = rand((out, d), g, dtype, d**-0.5)
    b = rand((out,), g, dtype)
    st = tile_stats(v).float().contiguous()
    flags = (ops().LINEAR_GELU | ops().LINEAR_Y_PACKED) if gelu else 0
    packed, u, fb = ops().fold_layer_norm(w, b, gamma, beta)
    print(f"[deferred] folded {dtype} rows {rows} d {d} out {out} gelu {gelu}", flush=True)
    got = ops().linear_norm(v, st, eps, packed, u, fb, out, flags)
    sep = ops().linear(ops().add_layer_norm(v, torch.zeros_like(v), gamma, beta, eps),
                       ops().pack_linear_weight(w), b, out, flags=flags)
    torch.cuda.synchronize()
    exact = F.linear(layer_norm64(v, gamma, beta, eps), w.double(), b.double())
    if gelu:
        got, sep = unpack(got, rows, out), unpack(sep, rows, out)
        exact = F.gelu(exact)
    e_got = (got.double() - exact).abs()
    e_sep = (sep.double() - exact).abs()
    assert float(e_got.max()) <= 1.5 * float(e_sep.max()) + 1e-6, (float(e_got.max()),
                                                                   float(e_sep.max()))
    assert float(e_got.mean()) <= 1.25 * float(e_sep.mean()) + 1e-7


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,d", [(1, 1024), (255, 768), (256, 1024), (5, 96)])
def test_apply_is_layer_norm(dtype, rows, d):
    g = torch.Generator(device=DEV).manual_seed(d + rows)
    v = rand((rows, d), g, dtype, 4.0, -1.0)
    gamma = rand((d,), g, dtype, 0.3, 1.0)
    beta = rand((d,), g, dtype, 0.2)
    st = tile_stats(v).float().contiguous()
    got = ops().layer_norm_apply(v, st, gamma, beta, 1e-5)
    torch.cuda.synchronize()
    want = layer_norm64(v, gamma, beta, 1e-5)
    err = (got.double() - want).abs()
    bound = ulp(want, dtype) * 1.01 + 1e-6
    assert (err <= bound).all(), float((err - bound).max())


def test_deferred_entry_points_reject_bad_arguments():
    dt = torch.bfloat16
    x = torch.zeros(4, 256, dtype=dt, device=DEV)
    w = ops().pack_linear_weight(torch.zeros(256, 256, dtype=dt, device=DEV))
    h = torch.zeros(4, 256, dtype=dt, device=DEV)
    st = torch.zeros(4, 8, 2, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):  # 250 outputs: not whole statistics tiles
        ops().linear_residual(x, ops().pack_linear_weight(torch.zeros(250, 256, dtype=dt,
                                                                      device=DEV)),
                              None, torch.zeros(4, 250, dtype=dt, device=DEV), None, None,
                              None, 0.0, 250)
    with pytest.raises(ValueError):  # deferred residual without gamma / beta
        ops().linear_residual(x, w, None, h, st, None, None, 1e-5, 256)
    with pytest.raises(ValueError):  # GELU is not a residual epilogue
        ops().linear_residual(x, w, None, h, None, None, None, 0.0, 256,
                              flags=ops().LINEAR_GELU)
    u = torch.zeros(256, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):  # statistics of the wrong width
        ops().linear_norm(x, torch.zeros(4, 4, 2, device=DEV), 1e-5, w, u, u, 256)
    with pytest.raises(ValueError):  # a packed x has no row statistics
        ops().linear_norm(x, st, 1e-5, w, u, u, 256, flags=ops().LINEAR_X_PACKED)
    gam = torch.ones(256, dtype=dt, device=DEV)
    with pytest.raises(ValueError):  # LayerNorm weights of another dtype than the rows
        ops().linear_residual(x, w, None, h, st, gam.float(), gam, 1e-5, 256)
    with pytest.raises(ValueError):
        ops().layer_norm_apply(h, st, gam, gam.float(), 1e-5)
    with pytest.raises(RuntimeError):  # statistics left on the host
        ops().linear_residual(x, w, None, h, st.cpu(), gam, gam, 1e-5, 256)
    with pytest.raises(ValueError):  # a bias shorter than the outputs
        ops().linear_residual(x, w, gam[:128], h, None, None, None, 0.0, 256)
    with pytest.raises(RuntimeError):  # a bias left on the host
        ops().linear_residual(x, w, gam.cpu(), h, None, None, None, 0.0, 256)
    with pytest.raises(RuntimeError):  # y_stats aliasing r_stats is refused by the library
        from vflorence_amd._lib import check, lib

        check(lib.vfl_linear_residual(x.data_ptr(), 256, w.data_ptr(), None, h.data_ptr(), 256,
                                      st.data_ptr(), h.data_ptr(), h.data_ptr(), 1e-5,
                                      h.data_ptr(), 256, st.data_ptr(), 4, 256, 256, 0, 1, None))


class _FakeAttention:
    """Deterministic stand-ins for the two attention ops (the deferral is what is tested):
    self-attention mixes q and v, cross-attention scales q."""

    @staticmethod
    def self_attention(q, k, v, k_cache, v_cache, scale):
        return (q.float() * 0.5 + v.float() * 0.25 - k.float() * 0.125).to(q.dtype)

    @staticmethod
    def cross_attention(q, layer_idx, scale):
        return (torch.tanh(q.float()) * (1.0 + layer_idx)).to(q.dtype)


@pytest.mark.parametrize("rows", [96, 384, 512])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decoder_layers_with_deferred_norms_match_separate_layer_norms(monkeypatch, dtype, rows):
    """Three BART-large-width decoder layers with the attention ops replaced by fixed
    functions: the deferred path (6 projection launches per layer, one LayerNorm apply at
    the end) against the separate residual + LayerNorm kernels, within a few roundings,
    up to the projections' 512-row limit (past it the layers take the separate path)."""
    from transformers import BartConfig

    from vflorence_amd.layers import bart

    monkeypatch.setattr(bart, "decoder_self_attention", _FakeAttention.self_attention)
    monkeypatch.setattr(bart, "decoder_cross_attention", _FakeAttention.cross_attention)
    cfg = BartConfig(d_model=1024, decoder_layers=3, decoder_attention_heads=16,
                     decoder_ffn_dim=4096, encoder_layers=1, vocab_size=64)
    torch.manual_seed(0)
    dec = bart.BartDecoder(cfg).to(DEV, dtype)
    with torch.no_grad():
        for p in dec.parameters():
            p.normal_(0, 0.03)
        for m in dec.modules():
            if isinstance(m, torch.nn.LayerNorm):
                m.weight.normal_(1.0, 0.1)
                m.bias.normal_(0.0, 0.05)
    for m in dec.modules():
        if isinstance(m, bart.DecodeLinear):
            m.repack()
    ids = torch.randint(0, 64, (rows,), device=DEV)
    pos = torch.randint(0, 100, (rows,), device=DEV)
    with torch.no_grad():
        h0 = bart._residual_norm(dec.embed_tokens(ids), dec.embed_positions(pos),
                                 dec.layernorm_embedding)
        assert all(layer.deferred_ready(h0, rows) for layer in dec.layers)
        assert not any(layer.deferred_ready(h0, 513) for layer in dec.layers)
        dec.deferred_norms = True
        got = dec(ids, pos)
        dec.deferred_norms = False
        want = dec(ids, pos)
        torch.cuda.synchronize()
    assert got.shape == want.shape == (rows, 1024)
    diff = (got.float() - want.float()).abs()
    scale = want.float().abs().mean()
    tol = 0.02 if dtype == torch.bfloat16 else 0.004
    print(f"[deferred] decoder layers {dtype}: max |diff| {float(diff.max()):.4f}, mean "
          f"{float(diff.mean()):.5f}, mean |h| {float(scale):.3f}", flush=True)
    assert float(diff.mean()) < tol * float(scale)
    assert float(diff.max()) < 25 * tol * float(scale)
