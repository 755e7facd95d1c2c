"""The algebra of the deferred LayerNorm, in float64 on the CPU: the tile statistics
the output projections write combine to the row's mean and variance, and a projection
of LN(v) equals the folded form the reading projections compute.  Also how the decoder
wires each projection to the LayerNorm whose output it reads."""

import torch
import torch.nn.functional as F


def tile_stats(v):
    t = v.view(v.shape[0], -1, 32)
    mean = t.mean(-1)
    return mean, ((t - mean[..., None]) ** 2).sum(-1)


def combine(m_t, m2_t, eps):
    """The kernels' combination (Chan et al.: equal tile counts of 32)."""
    T = m_t.shape[1]
    mean = m_t.sum(1) / T
    m2 = m2_t.sum(1) + 32 * ((m_t - mean[:, None]) ** 2).sum(1)
    return mean, 1.0 / torch.sqrt(m2 / (32 * T) + eps)


def test_tile_statistics_combine_to_the_row_moments():
    g = torch.Generator().manual_seed(0)
    for d in (96, 768, 1024):
        v = torch.randn(37, d, generator=g, dtype=torch.float64) * 3 + 5
        mean, rstd = combine(*tile_stats(v), 1e-5)
        assert torch.allclose(mean, v.mean(1), rtol=1e-12, atol=1e-12)
        var = v.var(1, unbiased=False)
        assert torch.allclose(rstd, 1 / torch.sqrt(var + 1e-5), rtol=1e-12)


def test_folded_projection_equals_projection_of_layer_norm():
    """W LN(v) + b = rstd (W' v - mean u) + b' with W' = W diag(gamma), u = W' 1,
    b' = b + W beta (exact algebra; the kernels round W' to the element type)."""
    g = torch.Generator().manual_seed(1)
    d, out = 256, 96
    v = torch.randn(20, d, generator=g, dtype=torch.float64) * 2 + 0.5
    gamma = torch.randn(d, generator=g, dtype=torch.float64) * 0.2 + 1
    beta = torch.randn(d, generator=g, dtype=torch.float64) * 0.1
    w = torch.randn(out, d, generator=g, dtype=torch.float64)
    b = torch.randn(out, generator=g, dtype=torch.float64)
    want = F.linear(F.layer_norm(v, (d,), gamma, beta, 1e-5), w, b)
    wf = w * gamma
    u = wf.sum(1)
    fb = b + w @ beta
    mean, rstd = combine(*tile_stats(v), 1e-5)
    got = rstd[:, None] * (v @ wf.T - mean[:, None] * u) + fb
    assert torch.allclose(got, want, rtol=1e-10, atol=1e-10)


def test_decoder_projections_know_the_layer_norm_they_read():
    from transformers import BartConfig

    from vflorence_amd.layers import bart

    cfg = BartConfig(d_model=64, decoder_layers=3, decoder_attention_heads=2,
                     decoder_ffn_dim=128, encoder_layers=1, vocab_size=32)
    dec = bart.BartDecoder(cfg)
    assert dec.deferred_norms
    for i, layer in enumerate(dec.layers):
        qkv_in = layer.self_attn.qkv_proj._in_norm
        assert qkv_in == (() if i == 0 else (dec.layers[i - 1].final_layer_norm,))
        assert layer.encoder_attn.q_proj._in_norm == (layer.self_attn_layer_norm,)
        assert layer.fc1._in_norm == (layer.encoder_attn_layer_norm,)
        for lin in (layer.self_attn.out_proj, layer.encoder_attn.out_proj, layer.fc2):
            assert lin._in_norm == ()
    # references, not submodules: the state dict keeps the checkpoint's names only
    names = set(dec.state_dict())
    assert not any("_in_norm" in n for n in names)
    assert "layers.1.self_attn.qkv_proj.weight" in names
    # host tensors never take the deferred path (no folded operands without the GPU)
    assert dec.layers[1].self_attn.qkv_proj.folded_operands(4) is None
