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


def test_quantize_int8_channel_scale_multiplies():
    """ops/quantize.py:91-97: value * channel_scale, then / scale (dividing by the channel scale gives [2, 12])."""
    x = torch.tensor([[3.0, 3.0], [-3.0, 100.0]], device=DEV)
    cs = torch.tensor([2.0, 0.25], device=DEV)
    got = ops.quantize_int8.get("hip")(x, torch.tensor(1.0, device=DEV), channel_scale=cs)
    assert got.values.cpu().tolist() == [[6, 1], [-6, 25]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("rows,k", [(5376, 1024), (777, 4096), (300, 1000), (5, 64), (3, 7)])
def test_quantize_int8_rows_bytes(rows, k, dtype):
    """Per-row dynamic INT8 (ops/quantize.py:148-154): codes and scales bit-identical to the oracle, with an outlier
    row and an all-zero row (FlashIM's contract, tests/ops/test_ops_cuda.py:967-979)."""
    torch.manual_seed(0)
    x = (torch.randn(rows, k) * 3).to(dtype)
    x[rows // 2] *= 300
    x[-1] = 0
    got_q, got_s = ops.quantize_int8_rows.get("hip")(x.to(DEV))
    want_q, want_s = ref.quantize_int8_rows(x)
    assert got_s.shape == (rows, 1) and got_s.dtype == torch.float32
    assert torch.equal(got_s.cpu(), want_s) and torch.equal(got_q.cpu(), want_q)


def test_quantize_int8_rows_reciprocal_scale_known_answer():
    """amax = 5.798794: amax * float32(1/127) and amax / 127 differ by one ulp, and 0.068489686 rounds to 2 only under
    the reciprocal product, which the reference specifies."""
    x = torch.tensor([[5.798794, 0.068489686, -0.068489686, 0.0]], device=DEV)
    q, s = ops.quantize_int8_rows.get("hip")(x)
    assert q.cpu().tolist() == [[127, 2, -2, 0]]
    want_q, want_s = ref.quantize_int8_rows(x.cpu())
    assert torch.equal(s.cpu(), want_s)
    q3, s3 = ops.quantize_int8_rows.get("hip")(torch.randn(2, 3, 64, device=DEV, dtype=torch.bfloat16))
    assert q3.shape == (2, 3, 64) and s3.shape == (2, 3, 1)


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
