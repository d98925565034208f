"""The GELU -> quantize producers (``ops.gelu_quantize`` with and without ``input_bias``, ``ops.gelu_quantize_int8``:
flashim/ops/quantize.py:63-74, 128-131), ``ops.int8_linear_quantize`` into a strided buffer
(flashim/ops/gemm.py:104-116) and the conv weight packers (flashim_amd.packing; quant/methods/conv2d.py:92-100,
194-205) vs the oracle.

Bars: the packers and ``int8_linear_quantize`` are byte-exact. The GELU producers evaluate erf with this library's own
fit, which agrees with torch's libm GELU within one BF16 rounding (about 1% of BF16 inputs land one step apart, and
torch's FP32 ``1 + erf`` cancels below |GELU| ~ 4e-3): codes are compared after dequantizing, each within one code step
of the oracle's value or an absolute 2^-12 (in the unscaled domain), and at most 0.5% of the codes may differ. The tanh
form is x / (1 + e^(-2y)), which avoids torch's 1 + tanh cancellation in the negative tail; same bars."""

import pytest
import torch
import torch.nn.functional as F

from flashim_amd import ops, packing, quant
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _e4m3_step(v: torch.Tensor) -> torch.Tensor:
    """Spacing of E4M3 codes at |v| (subnormal spacing 2^-9 below 2^-6)."""
    mag = v.abs().clamp_min(2.0**-6)
    return torch.exp2(torch.floor(torch.log2(mag)) - 3)


def _assert_mx_codes_close(got_codes, want_codes, exponent):
    scale = torch.exp2(exponent.float()).repeat_interleave(32)[: got_codes.shape[-1]]
    g = got_codes.float() * scale
    w = want_codes.float() * scale
    step = _e4m3_step(want_codes.float()) * scale
    assert ((g - w).abs() <= torch.maximum(step, torch.full_like(step, 2.0**-12)) * 1.0001).all()
    frac = (got_codes.view(torch.uint8) != want_codes.view(torch.uint8)).float().mean().item()
    assert frac <= 5e-3, frac


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("shape", [(2, 17, 19, 64), (300, 96), (4, 9, 70)])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_gelu_quantize(shape, dtype, with_bias, approximate):
    torch.manual_seed(0)
    x = (torch.randn(shape) * 3).to(dtype)
    bias = torch.randn(shape[-1]) * 0.5 if with_bias else None
    activated = F.gelu(x.float() + (bias if with_bias else 0), approximate=approximate).to(dtype)
    exponent = ref.calibrate_block32_exponent(activated.float())
    got = ops.gelu_quantize.get("hip")(x.to(DEV), exponent.to(DEV), approximate,
                                       input_bias=None if bias is None else bias.to(DEV))
    want = ref.gelu_quantize(x, exponent, approximate, input_bias=bias)
    assert got.values.shape == want.shape and got.logical_shape == tuple(shape)
    _assert_mx_codes_close(got.values.cpu(), want, exponent)


def test_gelu_quantize_channels_first_view_and_forms():
    torch.manual_seed(1)
    x = torch.randn(2, 64, 9, 11, dtype=torch.bfloat16) * 2
    view = x.to(DEV).permute(0, 2, 3, 1)
    exponent = torch.tensor([-6, -5], dtype=torch.int8)
    got = ops.gelu_quantize.get("hip")(view, exponent.to(DEV))
    packed = ops.gelu_quantize.get("hip")(view.contiguous(), exponent.to(DEV))
    assert torch.equal(got.values.view(torch.uint8), packed.values.view(torch.uint8))
    _assert_mx_codes_close(got.values.cpu(), ref.gelu_quantize(x.permute(0, 2, 3, 1), exponent), exponent)
    tanh = ops.gelu_quantize.get("hip")(view, exponent.to(DEV), "tanh")
    _assert_mx_codes_close(tanh.values.cpu(), ref.gelu_quantize(x.permute(0, 2, 3, 1), exponent, "tanh"), exponent)
    assert not ops.gelu_quantize.supports(view, exponent.to(DEV), "sigmoid")
    # the forms part in the negative tail: GELU(-2.5) = -0.015084 (tanh) / -0.015524 (erf), INT8 codes -15 / -16 at 1e-3
    tail = torch.full((1, 64), -2.5, device=DEV)
    s = torch.tensor(1e-3, device=DEV)
    assert ops.gelu_quantize_int8.get("hip")(tail, s, "tanh").values[0, 0].item() == -15
    assert ops.gelu_quantize_int8.get("hip")(tail, s).values[0, 0].item() == -16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_gelu_quantize_int8(dtype, approximate):
    torch.manual_seed(2)
    x = (torch.randn(3, 33, 40, 48) * 2).to(dtype)
    scale = torch.tensor(0.021)
    got = ops.gelu_quantize_int8.get("hip")(x.to(DEV), scale.to(DEV), approximate).values.cpu()
    want = ref.gelu_quantize_int8(x, scale, approximate)
    assert (got.int() - want.int()).abs().max() <= 1
    assert (got != want).float().mean() <= 5e-3


@pytest.mark.parametrize("m,k,n", [(300, 128, 96), (1000, 256, 256), (77, 40, 24), (20000, 512, 64)])
@pytest.mark.parametrize("per_row", [False, True])
def test_int8_linear_quantize_into_strided_out(m, k, n, per_row):
    g = torch.Generator().manual_seed(m)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
    w_scale = torch.rand(n, generator=g) * 0.01 + 0.001
    a_scale = (torch.rand(m, 1, generator=g) * 0.05 + 0.001) if per_row else torch.tensor(0.017)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    out_scale = torch.tensor(0.9)
    cat = torch.full((m, 2 * n + 16), 55, dtype=torch.int8, device=DEV)  # the right half of a cat buffer
    target = cat[:, n + 16:]
    got = ops.int8_linear_quantize.get("hip")(a.to(DEV), w.to(DEV), a_scale.to(DEV), w_scale.to(DEV), bias.to(DEV),
                                              out_scale.to(DEV), target)
    assert got is target
    want = ref.int8_linear_quantize(a, w, a_scale, w_scale, bias, out_scale)
    assert torch.equal(target.cpu(), want)
    assert (cat[:, : n + 16] == 55).all()  # nothing outside the view is written


@pytest.mark.parametrize("cout,cin,k", [(64, 64, 3), (48, 40, 3), (32, 3, 7), (128, 96, 1)])
def test_conv_weight_packers_bit_exact(cout, cin, k):
    torch.manual_seed(cout + cin)
    w = torch.randn(cout, cin, k, k) * 0.1
    q, s = packing.pack_int8_conv(w.to(DEV))
    flat = w.permute(0, 2, 3, 1).reshape(cout, -1)
    want_s = ref.weight_scales(flat)
    assert torch.equal(s.cpu(), want_s) and torch.equal(q.cpu(), ref.quantize_symmetric(flat, want_s[:, None]))
    qw = packing.pack_mxfp8_conv(w.to(DEV))
    cp = ref.padded_channels(cin)
    padded = F.pad(w.permute(0, 2, 3, 1), (0, cp - cin)).reshape(cout, -1)
    wv, we = ref.quantized_weight_from_float(padded)
    assert torch.equal(qw.values.cpu().view(torch.uint8), wv.view(torch.uint8)) and torch.equal(
        qw.scale_exponent.cpu(), we)


def test_packed_conv_matches_nn_conv_geometry():
    """conv_geometry + pack_int8_conv feed ops.int8_conv2d; 'same' padding resolves as the conv pads."""
    torch.manual_seed(9)
    conv = torch.nn.Conv2d(32, 48, 3, padding="same", dilation=2)
    geo = packing.conv_geometry(conv)
    assert geo == (3, 3, 1, 1, 2, 2, 2, 2)
    q, s = packing.pack_int8_conv(conv.weight.to(DEV))
    x = torch.randint(-127, 127, (1, 12, 13, 32), dtype=torch.int8)
    a_s = torch.tensor(0.02)
    got = ops.int8_conv2d(x.to(DEV), q, a_s.to(DEV), s, None, *geo).cpu()
    want = ref.int8_conv2d(x, q.cpu(), a_s, s.cpu(), None, *geo)
    assert got.shape == (1, 12, 13, 48) and torch.equal(got, want)
    with pytest.raises(ValueError):
        packing.conv_geometry(torch.nn.Conv2d(4, 4, 3, groups=2))
