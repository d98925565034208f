"""HIP quantizers vs the oracle: byte-exact (FlashIM's contracts tests/ops/test_ops_cuda.py:419-445 and
tests/quant/test_int8.py:26-29, with the torch reference's IEEE division for INT8)."""

import pytest
import torch

from flashim_amd import ops, quant
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("shape", [(300, 96), (2, 17, 19, 64), (1, 128, 128, 64), (7, 5, 1000), (3, 40)])
def test_quantize_mxfp8_bytes(shape, dtype):
    torch.manual_seed(0)
    x = (torch.randn(shape) * 5).to(dtype)
    exponent = ref.calibrate_block32_exponent(x.float())
    got = ops.quantize_mxfp8.get("hip")(x.to(DEV), exponent.to(DEV))
    want = ref.quantize_mxfp8(x, exponent)
    assert got.values.shape == want.shape and got.logical_shape == tuple(shape)
    assert torch.equal(got.values.cpu().view(torch.uint8), want.view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(300, 96), (2, 17, 19, 64), (1, 128, 128, 64), (5, 1000), (3, 7)])
def test_quantize_int8_bytes(shape, dtype):
    torch.manual_seed(0)
    x = (torch.randn(shape) * 3).to(dtype)
    scale = torch.tensor(x.float().abs().max().item() / 127)
    got = ops.quantize_int8.get("hip")(x.to(DEV), scale.to(DEV))
    assert got.values.dtype == torch.int8 and got.values.is_contiguous()
    assert torch.equal(got.values.cpu(), ref.quantize_int8(x, scale))


def test_quantize_int8_known_answer_and_channel_scale():
    x = torch.tensor([[0.5, 1.5, 2.5, -0.5, 1000.0, -1000.0, 0.0]])
    got = ops.quantize_int8.get("hip")(x.to(DEV), torch.tensor(1.0, device=DEV))
    assert got.values.cpu().tolist() == [[0, 2, 2, 0, 127, -127, 0]]  # tests/quant/test_int8.py:26-29
    torch.manual_seed(1)
    y = torch.randn(33, 48).bfloat16()
    cs = torch.rand(48) + 0.5
    s = torch.tensor(0.02)
    got = ops.quantize_int8.get("hip")(y.to(DEV), s.to(DEV), channel_scale=cs.to(DEV))
    assert torch.equal(got.values.cpu(), ref.quantize_int8(y, s, cs))


@pytest.mark.parametrize("channels", [16, 48, 96, 257])
@pytest.mark.parametrize("fmt", ["int8", "mxfp8"])
def test_quantize_channels_first_view(channels, fmt):
    """The NHWC view of NCHW memory is read in place: the bytes of the packed copy and of the oracle
    (tests/ops/test_ops_cuda.py:427-445)."""
    torch.manual_seed(0)
    x = torch.randn(2, channels, 17, 19, dtype=torch.bfloat16) * 5
    view = x.to(DEV).permute(0, 2, 3, 1)
    assert not view.is_contiguous()
    if fmt == "int8":
        op, scale = ops.quantize_int8, torch.tensor(0.04)
        want = ref.quantize_int8(x.permute(0, 2, 3, 1), scale)
    else:
        op, scale = ops.quantize_mxfp8, ref.calibrate_block32_exponent(x.permute(0, 2, 3, 1).reshape(-1, channels).float())
        want = ref.quantize_mxfp8(x.permute(0, 2, 3, 1), scale)
    fast = op.get("hip")(view, scale.to(DEV))
    packed = op.get("hip")(view.contiguous(), scale.to(DEV))
    assert fast.values.is_contiguous()
    assert torch.equal(fast.values.cpu().view(torch.uint8), packed.values.cpu().view(torch.uint8))
    assert torch.equal(fast.values.cpu().view(torch.uint8), want.view(torch.uint8))


@pytest.mark.parametrize("rows,k", [(1, 32), (333, 128), (4099, 512), (130, 96)])
def test_quantize_dynamic_2d_and_swizzle(rows, k):
    torch.manual_seed(3)
    x = torch.randn(rows, k).relu() * torch.rand(rows, 1) * 8
    x[rows // 2, :32] = 0  # an all-zero block: exponent -127
    values, exponent = quant.quantize_dynamic_2d(x.to(DEV))
    want_v, want_e = ref.quantize_dynamic_2d(x)
    assert torch.equal(exponent.cpu(), want_e)
    assert torch.equal(values.cpu().view(torch.uint8), want_v.view(torch.uint8))
    v2, swz = quant.quantize_dynamic_swizzled(x.to(DEV))
    assert torch.equal(v2.cpu().view(torch.uint8), want_v.view(torch.uint8))
    assert torch.equal(swz.cpu().view(torch.uint8), ref.swizzle_scales(want_e))
    assert torch.equal(quant.swizzle_scales(exponent).cpu().view(torch.uint8), ref.swizzle_scales(want_e))
    assert torch.equal(quant.unswizzle_scales(swz, rows, k // 32).cpu(), want_e)


@pytest.mark.parametrize("n,k", [(100, 70), (512, 512), (128, 1152), (64, 64)])
def test_weight_packing(n, k):
    torch.manual_seed(4)
    w = torch.randn(n, k) * 0.05
    qw = quant.QuantizedWeight.from_float(w.to(DEV))
    want_v, want_e = ref.quantized_weight_from_float(w)
    assert torch.equal(qw.scale_exponent.cpu(), want_e)
    assert torch.equal(qw.values.cpu().view(torch.uint8), want_v.view(torch.uint8))
    q8, s8 = quant.weight_scales_and_values(w.to(DEV))
    want_s = ref.weight_scales(w)
    assert torch.equal(s8.cpu(), want_s)
    assert torch.equal(q8.cpu(), ref.quantize_symmetric(w, want_s[:, None]))


@pytest.mark.parametrize("shape", [(7, 5, 32), (7, 5, 1000), (20000, 512), (2, 17, 1024)])
def test_calibrate_block32(shape):
    torch.manual_seed(5)
    x = torch.randn(shape) * 10 * torch.rand(shape[-1])
    got = quant.calibrate_block32_exponent(x.to(DEV))
    assert torch.equal(got.cpu(), ref.calibrate_block32_exponent(x))
