"""The decode-step linear kernel (vflorence_amd::linear) against a float64 torch
reference of nn.Linear on the same inputs, and the decoder modules that use it."""

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


def assert_one_rounding(got, want, dtype):
    """Within one rounding of the element type of the exact product (plus the fp32
    summation error, far below it at these sizes)."""
    ulp = 2**-8 if dtype == torch.bfloat16 else 2**-11
    err = (got.double() - want).abs()
    bound = want.abs() * ulp + 1e-4
    assert (err <= bound).all(), float((err - bound).max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,out_f,in_f", [
    (1, 1024, 1024), (7, 1024, 1024), (64, 768, 768), (256, 1024, 1024), (100, 1000, 512),
    (33, 1021, 256), (300, 96, 256)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_linear_matches_float64(dtype, rows, out_f, in_f, with_bias):
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + out_f)
    x = torch.randn(rows, in_f, device=DEV, generator=g).to(dtype)
    w = (torch.randn(out_f, in_f, device=DEV, generator=g) / in_f**0.5).to(dtype)
    b = torch.randn(out_f, device=DEV, generator=g).to(dtype) if with_bias else None
    print(f"[linear] {dtype} rows {rows} out {out_f} in {in_f} bias {with_bias}", flush=True)
    got = ops().linear(x, w, b)
    torch.cuda.synchronize()
    assert got.shape == (rows, out_f) and got.dtype == dtype
    assert_one_rounding(got, reference(x, w, b), dtype)


def test_linear_takes_strided_and_batched_inputs():
    g = torch.Generator(device=DEV).manual_seed(5)
    big = torch.randn(40, 1024 + 512, device=DEV, generator=g).to(torch.bfloat16)
    x = big[:, 256:256 + 1024]  # row stride 1536 elements, 512-byte offset
    w = (torch.randn(1024, 1024, device=DEV, generator=g) / 32).to(torch.bfloat16)
    b = torch.randn(1024, device=DEV, generator=g).to(torch.bfloat16)
    got = ops().linear(x, w, b)
    assert_one_rounding(got, reference(x, w, b), torch.bfloat16)
    x3 = x.reshape(4, 10, 1024)  # leading dimensions are kept
    got3 = ops().linear(x3, w, b)
    assert got3.shape == (4, 10, 1024)
    assert torch.equal(got3.reshape(40, 1024), got)


def test_linear_rejects_bad_arguments():
    from vflorence_amd._lib import HipAttnError

    x = torch.zeros(4, 1024, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(HipAttnError, match="multiple of 256"):
        ops().linear(x[:, :1000], torch.zeros(64, 1000, device=DEV, dtype=torch.bfloat16), None)
    with pytest.raises(ValueError, match="one dtype"):
        ops().linear(x, torch.zeros(64, 1024, device=DEV, dtype=torch.float16), None)
    with pytest.raises(HipAttnError, match="bf16 and fp16"):
        ops().linear(x.float(), torch.zeros(64, 1024, device=DEV), None)


def test_decoder_projections_use_the_kernel_where_it_fits():
    """DecodeLinear: decode-step rows on a square 16-bit weight go through the kernel
    (results within one rounding of float64, identical to calling it directly); more
    rows, fp32 and other shapes take F.linear."""
    from vflorence_amd.layers.bart import DecodeLinear

    torch.manual_seed(0)
    lin = DecodeLinear(1024, 1024).to(DEV, torch.bfloat16)
    x = torch.randn(256, 1024, device=DEV).to(torch.bfloat16)
    got = lin(x)
    assert torch.equal(got, ops().linear(x, lin.weight, lin.bias))
    assert_one_rounding(got, reference(x, lin.weight, lin.bias), torch.bfloat16)
    assert ops().linear_fits(256, lin.weight) and not ops().linear_fits(257, lin.weight)
    xl = torch.randn(300, 1024, device=DEV).to(torch.bfloat16)
    assert torch.equal(lin(xl), F.linear(xl, lin.weight, lin.bias))
    lin32 = DecodeLinear(1024, 1024).to(DEV)
    x32 = torch.randn(8, 1024, device=DEV)
    assert torch.equal(lin32(x32), F.linear(x32, lin32.weight, lin32.bias))
