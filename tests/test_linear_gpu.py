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
    (100, 1000, 512), (33, 1021, 256), (300, 96, 256), (5, 64, 4096)])
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
        ops().linear(x, packed, None, 128)
    with pytest.raises(ValueError, match="one dtype"):
        ops().linear(x.half(), packed, None, 64)
    with pytest.raises(HipAttnError, match="multiple of 256"):
        ops().pack_linear_weight(torch.zeros(64, 1000, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(HipAttnError, match="bf16 and fp16"):
        ops().pack_linear_weight(torch.zeros(64, 1024, device=DEV))


def test_decoder_projections_use_the_kernel_where_it_fits():
    """DecodeLinear: decode-step rows on a 16-bit weight of up to 3072 x 1024 go through
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
    assert ops().linear_fits(256, lin.weight) and not ops().linear_fits(257, lin.weight)
    xl = torch.randn(300, 1024, device=DEV).to(torch.bfloat16)
    assert torch.equal(lin(xl), F.linear(xl, lin.weight, lin.bias))
    wide = DecodeLinear(1024, 4096).to(DEV, torch.bfloat16)
    assert not ops().linear_fits(8, wide.weight)
    lin32 = DecodeLinear(1024, 1024).to(DEV)
    x32 = torch.randn(8, 1024, device=DEV)
    assert torch.equal(lin32(x32), F.linear(x32, lin32.weight, lin32.bias))
