"""HIP VGG stem vs the oracle. conv2d_small_cin_quantize_int8 (FlashIM's contract tests/ops/test_ops_cuda.py:543-555):
the INT8 maps of the reference chain up to the FP32 summation order, at most one INT8 step on < 1e-4 of the elements;
the bound op (weights packed once) gives the same bytes. bias_relu_quantize_int8: byte-exact (no accumulation)."""

import pytest
import torch

from flashim_amd import ops
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _mismatch(a, b):
    return (a != b).float().mean().item()


@pytest.mark.parametrize("batch,height,width", [(1, 17, 50), (2, 40, 129), (1, 224, 300)])
@pytest.mark.parametrize("cout", [64, 32])
def test_conv2d_small_cin_quantize_int8(batch, height, width, cout):
    torch.manual_seed(0)
    x = torch.randn(batch, 3, height, width).bfloat16()
    weight = (torch.randn(cout, 3, 3, 3) * 0.3).bfloat16()
    bias = torch.randn(cout).bfloat16()
    scale = torch.tensor(0.04)
    xs, ws, bs, ss = x.to(DEV), weight.to(DEV), bias.to(DEV), scale.to(DEV)
    fast = ops.conv2d_small_cin_quantize_int8.get("hip")(xs, ss, ws, bs)
    want = ref.conv2d_small_cin_quantize_int8(x, scale, weight, bias)
    got = fast.values.cpu()
    assert got.shape == (batch, height, width, cout) and fast.scale is ss
    assert (got.int() - want.int()).abs().max() <= 1 and _mismatch(got, want) < 1e-4
    bound = ops.conv2d_small_cin_quantize_int8.bind(ws, bs)
    assert torch.equal(bound(xs, ss).values, fast.values)


@pytest.mark.parametrize("cin,cout", [(1, 16), (2, 128), (4, 64), (8, 32), (8, 128)])
@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32])
def test_conv2d_small_cin_shapes(cin, cout, bias_dtype):
    """Other Cin (K = 9 Cin padded to 32 or 96), Cout 16-128, an FP32 bias (the sum is not rounded to BF16), widths
    that are not multiples of the 64-pixel segment."""
    torch.manual_seed(cin * 100 + cout)
    x = torch.randn(2, cin, 19, 70).bfloat16()
    weight = (torch.randn(cout, cin, 3, 3) * 0.3).bfloat16()
    bias = torch.randn(cout).to(bias_dtype)
    scale = torch.tensor(0.05)
    got = ops.conv2d_small_cin_quantize_int8.get("hip")(x.to(DEV), scale.to(DEV), weight.to(DEV), bias.to(DEV)).values.cpu()
    want = ref.conv2d_small_cin_quantize_int8(x, scale, weight, bias)
    assert got.shape == want.shape
    assert (got.int() - want.int()).abs().max() <= 1 and _mismatch(got, want) < 1e-3


def test_conv2d_small_cin_rejects():
    """Outside the kernel's shapes the HIP impl does not apply (a 5x5 weight, Cout not a power of two)."""
    x = torch.randn(1, 3, 8, 8).bfloat16().to(DEV)
    scale = torch.tensor(0.05).to(DEV)
    for w, b in ((torch.randn(64, 3, 5, 5), torch.randn(64)), (torch.randn(48, 3, 3, 3), torch.randn(48))):
        report = ops.conv2d_small_cin_quantize_int8.explain(x, scale, w.bfloat16().to(DEV), b.bfloat16().to(DEV))
        assert "accepts" in report["hip"], report


@pytest.mark.parametrize("shape", [(2, 64, 17, 50), (1, 100, 9, 33), (3, 3, 5, 7), (1, 256, 32, 32)])
@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32])
def test_bias_relu_quantize_int8(shape, bias_dtype):
    torch.manual_seed(sum(shape))
    raw = (torch.randn(*shape) * 3).bfloat16()
    bias = torch.randn(shape[1]).to(bias_dtype)
    scale = torch.tensor(0.03)
    got = ops.bias_relu_quantize_int8.get("hip")(raw.to(DEV), bias.to(DEV), scale.to(DEV))
    want = ref.bias_relu_quantize_int8(raw, bias, scale)
    assert got.values.shape == want.shape and torch.equal(got.values.cpu(), want)
