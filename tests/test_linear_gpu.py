"""The decode-step linear kernel (vflorence_amd::linear over a weight re-laid out by
pack_linear_weight) against a float64 torch reference of nn.Linear on the same inputs,
and the decoder modules that use it."""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ops():
    from vflorence_amd import decoder_ops

    return decoder_ops


def reference(x, w, b):
    return F.linear(x.double(), w.double(), None if b is None else b.double())


def run(x, w, b):
    return ops().linear(x, ops().pack_linear_weight(w), b, w.shape[0])


def assert_one_rounding(got, want, dtype):
    """Within one rounding of the element type of the exact product (plus the fp32
    summation error, far below it at these sizes)."""
    ulp = 2**-8 if dtype == torch.bfloat16 else 2**-11
    err = (got.double() - want).abs()
    bound = want.abs() * ulp + 1e-4
    assert (err <= bound).all(), float((err - bound).max())


def test_packed_layout_is_the_documented_operand_order():
    """Block (r, c) holds row 16 r + l % 16, inputs 32 c + 8 (l / 16) .. +7 at element
    8 l; rows past out_features are zero (padding to a multiple of 32)."""
    out_f, in_f = 40, 512
    w = torch.arange(out_f * in_f, device=DEV, dtype=torch.float32).remainder(251)
    w = w.view(out_f, in_f).to(torch.bfloat16)
    packed = ops().pack_linear_weight(w).cpu()
    assert packed.numel() == 64 * in_f
    wp = torch.cat([w.cpu(), torch.zeros(64 - out_f, in_f, dtype=w.dtype)])
    want = wp.view(4, 16, in_f // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)
    assert torch.equal(packed, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,out_f,in_f", [
    (1, 1024, 1024), (7, 1024, 1024), (64, 768, 768), (256, 1024, 1024), (256, 3072, 1024),
    (100, 1000, 512), (33, 1021, 256), (300, 96, 256), (5, 64, 4096), (40, 512, 1280),
    (17, 256, 2560), (256, 1024, 4096), (384, 3072, 1024), (512, 1024, 4096),
    (448, 768, 768)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_linear_matches_float64(dtype, rows, out_f, in_f, with_bias):
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + out_f)
    x = torch.randn(rows, in_f, device=DEV, generator=g).to(dtype)
    w = (torch.randn(out_f, in_f, device=DEV, generator=g) / in_f**0.5).to(dtype)
    b = torch.randn(out_f, device=DEV, generator=g).to(dtype) if with_bias else None
    print(f"[linear] {dtype} rows {rows} out {out_f} in {in_f} bias {with_bias}", flush=True)
    got = run(x, w, b)
    torch.cuda.synchronize()
    assert got.shape == (rows, out_f) and got.dtype == dtype
    assert_one_rounding(got, reference(x, w, b), dtype)


def test_linear_takes_strided_and_batched_inputs():
    g = torch.Generator(device=DEV).manual_seed(5)
    big = torch.randn(40, 1024 + 512, device=DEV, generator=g).to(torch.bfloat16)
    x = big[:, 256:256 + 1024]  # row stride 1536 elements, 512-byte offset
    w = (torch.randn(1024, 1024, device=DEV, generator=g) / 32).to(torch.bfloat16)
    b = torch.randn(1024, device=DEV, generator=g).to(torch.bfloat16)
    got = run(x, w, b)
    assert_one_rounding(got, reference(x, w, b), torch.bfloat16)
    x3 = x.reshape(4, 10, 1024)  # leading dimensions are kept
    got3 = run(x3, w, b)
    assert got3.shape == (4, 10, 1024)
    assert torch.equal(got3.reshape(40, 1024), got)


def test_linear_rejects_bad_arguments():
    from vflorence_amd._lib import HipAttnError

    x = torch.zeros(4, 1024, device=DEV, dtype=torch.bfloat16)
    w = torch.zeros(64, 1024, device=DEV, dtype=torch.bfloat16)
    packed = ops().pack_linear_weight(w)
    with pytest.raises(ValueError, match="does not hold"):
        ops().linear(x, packed, None, 96)  # 64 x 1024 elements: not a padded 96-row weight
    with pytest.raises(ValueError, match="1024 features, the weight 512"):
        ops().linear(x, packed, None, 128)  # read as a 128 x 512 weight
    with pytest.raises(ValueError, match="one dtype"):
        ops().linear(x.half(), packed, None, 64)
    with pytest.raises(HipAttnError, match="multiple of 256"):
        ops().pack_linear_weight(torch.zeros(64, 1000, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(HipAttnError, match="bf16 and fp16"):
        ops().pack_linear_weight(torch.zeros(64, 1024, device=DEV))


def test_decoder_projections_use_the_kernel_where_it_fits():
    """DecodeLinear: decode-step rows on a 16-bit weight of up to 3072 x 4096 go through
    the kernel (identical to calling it directly, within one rounding of float64), and
    a changed weight is re-laid out; more rows, fp32 and other shapes take F.linear."""
    from vflorence_amd.layers.bart import DecodeLinear

    torch.manual_seed(0)
    lin = DecodeLinear(1024, 3072).to(DEV, torch.bfloat16)
    x = torch.randn(256, 1024, device=DEV).to(torch.bfloat16)
    got = lin(x)
    assert torch.equal(got, run(x, lin.weight, lin.bias))
    assert_one_rounding(got, reference(x, lin.weight, lin.bias), torch.bfloat16)
    with torch.no_grad():
        lin.weight.mul_(-1)
    assert torch.equal(lin(x), run(x, lin.weight, lin.bias))
    assert ops().linear_fits(512, lin.weight) and not ops().linear_fits(513, lin.weight)
    xm = torch.randn(300, 1024, device=DEV).to(torch.bfloat16)
    assert torch.equal(lin(xm), run(xm, lin.weight, lin.bias))
    xl = torch.randn(600, 1024, device=DEV).to(torch.bfloat16)
    assert torch.equal(lin(xl), F.linear(xl, lin.weight, lin.bias))
    wide = DecodeLinear(1024, 4096).to(DEV, torch.bfloat16)
    assert not ops().linear_fits(8, wide.weight)
    deep = DecodeLinear(4096, 1024).to(DEV, torch.bfloat16)
    xd = torch.randn(256, 4096, device=DEV).to(torch.bfloat16)
    assert ops().linear_fits(256, deep.weight)
    assert torch.equal(deep(xd), run(xd, deep.weight, deep.bias))
    assert not ops().linear_fits(8, torch.zeros(64, 8192, device=DEV, dtype=torch.bfloat16))
    lin32 = DecodeLinear(1024, 1024).to(DEV)
    x32 = torch.randn(8, 1024, device=DEV)
    assert torch.equal(lin32(x32), F.linear(x32, lin32.weight, lin32.bias))


def test_packed_weight_follows_in_place_updates_and_repack():
    """The packed copy is rewritten in place (captured graphs keep its address): an
    ordinary weight updated in place is re-laid out on the next eager call; an
    inference-mode weight, which has no version counter, after ``repack()``; a HIP graph
    captured before the update reads the new weight once ``repack()`` ran."""
    from vflorence_amd.layers.bart import DecodeLinear

    torch.manual_seed(1)
    lin = DecodeLinear(1024, 1024).to(DEV, torch.bfloat16)
    lin.repack()
    addr = lin.packed_weight().data_ptr()
    x = torch.randn(64, 1024, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.mul_(-1)
    assert torch.equal(lin(x), run(x, lin.weight, lin.bias))
    assert lin.packed_weight().data_ptr() == addr
    with torch.inference_mode():
        inf = DecodeLinear(1024, 1024).to(DEV, torch.bfloat16)
        assert inf.weight.is_inference()
        before = inf(x)
        inf.weight.mul_(0.5)
        inf.repack()
        after = inf(x)
    assert not torch.equal(before, after)
    assert torch.equal(after, run(x, inf.weight, inf.bias))
    # a graph captured over the packed copy sees a later update after repack()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lin(x)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = lin(x)
    with torch.no_grad():
        lin.weight.add_(0.01)
    lin.repack()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, run(x, lin.weight, lin.bias))


def unpack(packed, rows, cols):
    """The documented packed layout back to [rows, cols] (rows padded to 32 dropped)."""
    pr = (rows + 31) // 32 * 32
    t = packed.view(pr // 16, cols // 32, 4, 16, 8).permute(0, 3, 1, 2, 4)
    return t.reshape(pr, cols)[:rows]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 37, 256, 400, 512])
def test_feed_forward_pair_gelu_and_packed_activation(dtype, rows):
    """fc1 with VFL_LINEAR_GELU | VFL_LINEAR_Y_PACKED, then fc2 with VFL_LINEAR_X_PACKED:
    the packed activation holds exactly the unpacked call's rows, fc2 over it equals fc2
    over the unpacked rows bit for bit, and the pair is within rounding of float64."""
    d, ffn = 1024, 4096
    g = torch.Generator(device=DEV).manual_seed(rows)
    h = torch.randn(rows, d, device=DEV, generator=g).to(dtype)
    w1 = (torch.randn(ffn, d, device=DEV, generator=g) / d**0.5).to(dtype)
    b1 = (0.5 * torch.randn(ffn, device=DEV, generator=g)).to(dtype)
    w2 = (torch.randn(d, ffn, device=DEV, generator=g) / ffn**0.5).to(dtype)
    b2 = torch.randn(d, device=DEV, generator=g).to(dtype)
    o = ops()
    p1, p2 = o.pack_linear_weight(w1), o.pack_linear_weight(w2)
    mid = o.linear(h, p1, b1, ffn, flags=o.LINEAR_GELU)
    mid_packed = o.linear(h, p1, b1, ffn, flags=o.LINEAR_GELU | o.LINEAR_Y_PACKED)
    assert mid_packed.numel() == o.packed_elems(rows, ffn)
    assert torch.equal(unpack(mid_packed, rows, ffn), mid)
    out = o.linear(mid_packed, p2, b2, d, rows=rows, flags=o.LINEAR_X_PACKED)
    assert torch.equal(out, o.linear(mid, p2, b2, d))
    # GELU on the rounded pre-activation, as a separate activation kernel would see it
    pre = reference(h, w1, b1)
    want_mid = F.gelu(pre.to(dtype).double())
    ulp = 2**-8 if dtype == torch.bfloat16 else 2**-11
    err = (mid.double() - want_mid).abs()
    # a pre-activation one unit in the last place off (fp32 sums near a rounding
    # boundary), through GELU's slope (at most 1.13), plus the final rounding
    assert (err <= 2.5 * ulp * pre.abs() + ulp * want_mid.abs() + 1e-4).all()
    assert_one_rounding(out, reference(mid, w2, b2), dtype)


def test_decoder_feed_forward_matches_the_torch_ops():
    """BartDecoderLayer._feed_forward on a decode step's rows (the fused pair) against
    fc2(gelu(fc1(h))) through F.linear and torch's GELU, and the host path unchanged."""
    from transformers import BartConfig

    from vflorence_amd.layers.bart import BartDecoderLayer

    cfg = BartConfig(d_model=1024, decoder_ffn_dim=4096, decoder_attention_heads=16)
    torch.manual_seed(1)
    layer = BartDecoderLayer(cfg, 0).to(DEV, torch.bfloat16)
    h = torch.randn(200, 1024, device=DEV).to(torch.bfloat16)
    got = layer._feed_forward(h)
    want = F.linear(F.gelu(F.linear(h, layer.fc1.weight, layer.fc1.bias)), layer.fc2.weight,
                    layer.fc2.bias)
    torch.testing.assert_close(got.float(), want.float(), rtol=2e-2, atol=2e-2)
    # more rows than a decode step (over 512): the torch ops themselves
    hl = torch.randn(600, 1024, device=DEV).to(torch.bfloat16)
    wantl = F.linear(F.gelu(F.linear(hl, layer.fc1.weight, layer.fc1.bias)), layer.fc2.weight,
                     layer.fc2.bias)
    assert torch.equal(layer._feed_forward(hl), wantl)


def test_linear_rejects_bad_flags_and_packed_shapes():
    from vflorence_amd._lib import HipAttnError

    o = ops()
    w = torch.zeros(96, 256, device=DEV, dtype=torch.bfloat16)
    p = o.pack_linear_weight(w)
    x = torch.zeros(4, 256, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(HipAttnError, match="unknown flags"):
        o.linear(x, p, None, 96, flags=8)
    with pytest.raises(ValueError, match="not a packed"):
        o.linear(x.flatten(), p, None, 96, rows=4, flags=o.LINEAR_X_PACKED)
    w_odd = torch.zeros(100, 256, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(HipAttnError, match="packed output"):
        o.linear(x, o.pack_linear_weight(w_odd), None, 100, flags=o.LINEAR_Y_PACKED)


@pytest.mark.parametrize("vocab,tied", [(50265, False), (1000, True), (1024, False)])
def test_lm_head_runs_on_padded_operands(vocab, tied):
    """The LM head multiplies copies of its weight and the final logits bias padded with
    zero rows to a multiple of 256 outputs: the logits are the first ``vocab`` columns
    (row stride the padded width), within one rounding of the float64 product; the
    copies follow an in-place update on the next eager call, a tied head follows the
    shared embedding, and an inference-mode weight follows after ``repack_lm_head``."""
    from transformers import BartConfig

    from vflorence_amd.layers.bart import LM_HEAD_MULTIPLE, BartForConditionalGeneration

    cfg = BartConfig(vocab_size=vocab, d_model=256, encoder_layers=1, decoder_layers=1,
                     encoder_attention_heads=4, decoder_attention_heads=4, encoder_ffn_dim=256,
                     decoder_ffn_dim=256, max_position_embeddings=64, tie_word_embeddings=tied)
    with torch.device(DEV):
        model = BartForConditionalGeneration(cfg).to(torch.bfloat16)
    torch.manual_seed(3)
    with torch.no_grad():
        model.lm_head.weight.normal_(0, 0.05)
        model.final_logits_bias.normal_()
    model.repack_lm_head()
    padded = -(-vocab // LM_HEAD_MULTIPLE) * LM_HEAD_MULTIPLE
    h = torch.randn(37, 256, device=DEV).to(torch.bfloat16)
    got = model.logits(h)
    assert got.shape == (37, vocab) and got.stride(1) == 1
    if padded != vocab:
        assert got.stride(0) == padded and model._lm_padded[0].shape == (padded, 256)
        assert not model._lm_padded[0][vocab:].any() and not model._lm_padded[1][vocab:].any()
    else:
        assert model._lm_padded is None
    w, b = model.lm_head.weight, model.final_logits_bias[0]
    assert_one_rounding(got, reference(h, w, b), torch.bfloat16)
    with torch.no_grad():
        (model.model.shared.weight if tied else model.lm_head.weight).mul_(-1)
    assert_one_rounding(model.logits(h), reference(h, w, b), torch.bfloat16)
    with torch.inference_mode():
        with torch.device(DEV):
            inf = BartForConditionalGeneration(cfg).to(torch.bfloat16)
        inf.lm_head.weight.copy_(w)
        inf.final_logits_bias.copy_(model.final_logits_bias)
        inf.repack_lm_head()
        before = inf.logits(h).clone()
        inf.lm_head.weight.mul_(0.5)
        inf.repack_lm_head()
        after = inf.logits(h)
        assert not torch.equal(before, after)
        assert_one_rounding(after, reference(h, inf.lm_head.weight, inf.final_logits_bias[0]),
                            torch.bfloat16)
