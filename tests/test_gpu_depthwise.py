"""HIP depthwise 5x5 producers vs the oracle (FlashIM's contracts tests/ops/test_ops_cuda.py:56-69 and
tests/quant/test_int8.py:93-107): MXFP8 scales byte-exact with < 1e-3 code mismatch, INT8 within one code with < 5e-3
mismatch (FP32 tap order differs from torch's CPU conv), all-zero rows encode exponent -127 and zero codes."""

import pytest
import torch

from flashim_amd import ops, quant
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(batch, channels, hw, seed=1):
    torch.manual_seed(seed)
    x = (torch.randn(batch, channels, *hw) * 2).to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
    w = (torch.randn(25, channels) * 0.3).to(torch.bfloat16)
    b = torch.randn(channels)
    return x, w, b


def _mismatch(a, b):
    return (a.view(torch.uint8) != b.view(torch.uint8)).float().mean().item()


SHAPES = [(2, 32, (7, 9)), (2, 128, (50, 50)), (2, 512, (7, 9)), (1, 64, (1, 1)), (3, 96, (33, 17)), (1, 64, (5, 130))]


@pytest.mark.parametrize("batch,channels,hw", SHAPES)
def test_depthwise_relu_mxfp8(batch, channels, hw):
    x, w, b = _inputs(batch, channels, hw)
    q, s = ops.depthwise5x5_relu_mxfp8.get("hip")(x.to(DEV), w.to(DEV), b.to(DEV))
    wq, ws = ref.depthwise5x5_relu_mxfp8(x, w, b)
    assert q.shape == wq.shape and q.dtype == torch.float8_e4m3fn
    assert torch.equal(s.cpu().view(torch.uint8), ws)
    assert _mismatch(q.cpu(), wq) < 1e-3
    z, zs = ops.depthwise5x5_relu_mxfp8.get("hip")(x.to(DEV), w.to(DEV), torch.full_like(b, -1e4).to(DEV))
    assert torch.equal(z.cpu().float(), torch.zeros(z.shape))
    rows = batch * hw[0] * hw[1]
    assert (quant.unswizzle_scales(zs, rows, channels // 32) == -127).all()


@pytest.mark.parametrize("batch,channels,hw", SHAPES)
def test_depthwise_relu_int8(batch, channels, hw):
    x, w, b = _inputs(batch, channels, hw)
    scale = torch.tensor(0.03)
    got = ops.depthwise5x5_relu_int8.get("hip")(x.to(DEV), w.to(DEV), b.to(DEV), scale.to(DEV)).cpu()
    want = ref.depthwise5x5_relu_int8(x, w, b, scale)
    assert got.dtype == torch.int8 and got.shape == want.shape
    assert (got.int() - want.int()).abs().max() <= 1 and (got != want).float().mean() < 5e-3


@pytest.mark.parametrize("mode", ["bf16", "int8", "mxfp8", "mxfp8_tiny_scale"])
@pytest.mark.parametrize("batch,channels,hw", [(2, 64, (40, 37)), (1, 256, (9, 20)), (2, 32, (3, 3))])
def test_depthwise_gelu(batch, channels, hw, mode):
    x, w, b = _inputs(batch, channels, hw, seed=2)
    kwargs = {}
    if mode == "int8":
        kwargs["scale"] = torch.tensor(0.02)
    elif mode == "mxfp8":
        kwargs["exponent"] = torch.full((channels // 32,), -5, dtype=torch.int8)
    elif mode == "mxfp8_tiny_scale":  # a bound of 448 * 2^-13 < 0.17: GELU's negative values saturate too (the kernel's two-sided clamp)
        kwargs["exponent"] = torch.full((channels // 32,), -13, dtype=torch.int8)
    got = ops.depthwise5x5_gelu.get("hip")(x.to(DEV), w.to(DEV), b.to(DEV),
                                            **{k: v.to(DEV) for k, v in kwargs.items()}).cpu()
    want = ref.depthwise5x5_gelu(x, w, b, **kwargs)
    assert got.shape == want.shape and got.dtype == want.dtype
    if mode == "bf16":
        diff = (got.float() - want.float()).abs()
        # GELU's tail (x < -3) is tiny and computed through erfc here, through 1 + erf (cancelling) in torch:
        # an absolute floor of 2^-12 covers it, everything else is within one BF16 rounding. The FP32 sum of the
        # 25 taps and the bias runs in another order than torch's CPU conv, so a pre-activation value within an FP32
        # ulp or two of a BF16 rounding boundary can round to the neighbouring BF16 input, which GELU (slope <= 1.13)
        # carries to at most two output steps: allowed for 1e-4 of the elements.
        one_step = diff <= want.float().abs() * 2**-7 + 2**-12
        assert (diff <= want.float().abs() * 2**-6 + 2**-12).all()
        assert (~one_step).float().mean() <= 1e-4
    elif mode == "int8":
        assert (got.int() - want.int()).abs().max() <= 1 and (got != want).float().mean() < 5e-3
    else:
        assert _mismatch(got, want) < 5e-3
        assert (got.float() - want.float()).abs().max() <= want.float().abs().max() * 0.07
