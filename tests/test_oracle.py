"""Pins the CPU oracle (oracle/reference.py) before it is trusted as the checker: known answers from FlashIM's own
tests, closed forms, and brute force on small inputs -- each chosen so a plausible slip (wrong rounding mode, dropped
term, transposed operand, wrong tap order) fails."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reference as ref


# -- MX format -------------------------------------------------------------------------------------------------


def test_exponent_rule_known_answers():
    # tests/quant/test_mx_format.py:13-17
    e = ref.scale_exponent_from_amax(torch.tensor([0.0, 448.0, 449.0, 1.0, 1e-30]))
    assert e.dtype == torch.int8 and e.tolist() == [-127, 0, 1, -8, -108]


def test_exponent_rule_is_smallest_power_fitting_448():
    amax = torch.rand(10000) * torch.exp2(torch.randint(-60, 60, (10000,)).float()) + 1e-30
    e = ref.scale_exponent_from_amax(amax).double()
    scaled = amax.double() / torch.exp2(e)
    assert (scaled <= 448 * (1 + 2**-20)).all()  # fits (up to log2's FP32 rounding at a power of two)
    assert (amax.double() / torch.exp2(e - 1) > 448 * (1 - 2**-20)).all()  # one smaller power would not


@pytest.mark.parametrize("channels", [32, 1000, 1024])
def test_static_quantize_roundtrip_and_saturation(channels):
    # tests/quant/test_mx_format.py:21-34
    torch.manual_seed(0)
    x = torch.randn(7, 5, channels) * 10
    exponent = ref.calibrate_block32_exponent(x)
    q = ref.quantize_static(x, exponent)
    assert q.shape == (7, 5, ref.padded_channels(channels))
    scale = torch.exp2(exponent.float()).repeat_interleave(32)
    back = (q.float() * scale)[..., :channels]
    s = scale[:channels]
    assert ((back - x).abs() <= x.abs() * 2**-4 + s * 2**-10 + 1e-12).all()
    big = (ref.quantize_static(x * 1000, exponent).float() * scale)[..., :channels]
    assert torch.isfinite(big).all() and (big.abs() <= 448 * s + 1e-3).all()
    assert (q.float()[..., channels:] == 0).all()  # padding channels are zero codes


def test_e4m3_is_round_to_nearest_even():
    # midpoints between adjacent E4M3 codes round to the even code; E4M3 RNE is the library routine torch.to()
    codes = torch.arange(0, 126, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = (codes[:-1] + codes[1:]) / 2
    got = mids.to(torch.float8_e4m3fn).view(torch.uint8).int()
    lo = torch.arange(0, 125)
    assert ((got == lo) | (got == lo + 1)).all() and (got % 2 == 0).all()


def test_weight_quantization_padding():
    # tests/quant/test_mx_format.py:37-42
    torch.manual_seed(0)
    w = torch.randn(100, 70)
    values, exponent = ref.quantized_weight_from_float(w)
    assert values.shape == (128, 96) and exponent.shape == (128, 3)
    scale = torch.exp2(exponent.float()).repeat_interleave(32, dim=1)
    deq = (values.float() * scale)[:100, :70]
    assert ((deq - w).abs() <= w.abs() * 2**-4 + scale[:100, :70] * 2**-10 + 1e-12).all()


def _swizzle_offset(r, g, groups):
    # closed form of the cuBLAS 128x4 layout (flashim/backends/triton/conv.py:118-124)
    tiles_k = (groups + 3) // 4
    rt = r % 128
    return ((r // 128) * tiles_k + g // 4) * 512 + (rt % 32) * 16 + (rt // 32) * 4 + g % 4


@pytest.mark.parametrize("rows,groups", [(1, 1), (300, 32), (128, 4), (5000, 24), (130, 5)])
def test_swizzle_closed_form_and_invertible(rows, groups):
    torch.manual_seed(1)
    exponent = torch.randint(-20, 10, (rows, groups), dtype=torch.int8)
    sw = ref.swizzle_scales(exponent)
    r = torch.arange(rows)[:, None].expand(rows, groups)
    g = torch.arange(groups)[None, :].expand(rows, groups)
    off = _swizzle_offset(r, g, groups)
    assert torch.equal(sw[off], (exponent.to(torch.int16) + 127).to(torch.uint8))
    # tests/quant/test_mx_format.py:45-51
    values = torch.randn(rows, groups * 32).clamp(-448, 448).to(torch.float8_e4m3fn)
    dense = ref.dequantize_swizzled(values, sw)
    assert torch.equal(dense, values.float() * torch.exp2(exponent.float()).repeat_interleave(32, dim=1))


def test_dynamic_quantize_matches_per_block_rule():
    torch.manual_seed(2)
    x = torch.randn(33, 96) * torch.rand(33, 1) * 50
    x[3, :32] = 0
    q, e = ref.quantize_dynamic_2d(x)
    amax = x.reshape(33, 3, 32).abs().amax(-1)
    assert torch.equal(e, ref.scale_exponent_from_amax(amax))
    assert e[3, 0] == -127 and (q[3, :32].float() == 0).all()
    want = (x.reshape(33, 3, 32) / torch.exp2(e.float())[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert torch.equal(q.view(torch.uint8), want.reshape(33, 96).view(torch.uint8))


# -- INT8 format ---------------------------------------------------------------------------------------------


def test_int8_round_half_even_and_saturation():
    # tests/quant/test_int8.py:26-29
    x = torch.tensor([[0.5, 1.5, 2.5, -0.5, 1000.0, -1000.0, 0.0]])
    assert ref.quantize_int8_static(x, torch.tensor(1.0)).tolist() == [[0, 2, 2, 0, 127, -127, 0]]


def test_int8_quantize_is_one_ieee_division():
    # 3.375 / 0.03 = 112.5000... in exact arithmetic rounds differently from 3.375 * (1 / 0.03)
    # (tests/ops/test_depthwise_cuda.py:61-68): the reference divides
    x, s = torch.tensor([3.375]), torch.tensor(0.03)
    q = ref.quantize_int8_static(x, s)
    exact = np.float32(3.375) / np.float32(0.03)
    assert q.item() == int(np.rint(exact))


def test_weight_scales_per_channel():
    # tests/quant/test_int8.py:14-21
    torch.manual_seed(0)
    w = torch.randn(16, 64) * torch.rand(16, 1) * 5
    s = ref.weight_scales(w)
    q = ref.quantize_symmetric(w, s[:, None])
    assert q.abs().amax(dim=1).eq(127).all()
    assert ((q.float() * s[:, None] - w).abs() <= s[:, None] / 2 + 1e-6).all()
    assert torch.equal(ref.weight_scales(torch.zeros(2, 8)), torch.full((2,), torch.finfo(torch.float32).eps))


# -- im2col and the convs ------------------------------------------------------------------------------------


@pytest.mark.parametrize("k,s,p,d", [(3, 1, 1, 1), (3, 2, 1, 1), (3, 1, 2, 2), (1, 1, 0, 1), (5, 1, 2, 1), (7, 2, 3, 1)])
def test_im2col_matches_unfold(k, s, p, d):
    # tests/quant/test_conv2d.py:23-28: (ky, kx, c) order
    torch.manual_seed(0)
    x = torch.randint(-127, 127, (2, 11, 13, 6), dtype=torch.int8)
    cols = ref.im2col_gather(x, k, k, s, s, p, p, d, d)
    unf = F.unfold(x.permute(0, 3, 1, 2).float(), k, dilation=d, padding=p, stride=s)  # [B, C*k*k, L], (c, ky, kx)
    unf = unf.reshape(2, 6, k * k, -1).permute(0, 3, 2, 1).reshape(-1, k * k * 6)
    assert torch.equal(cols.float(), unf)


@pytest.mark.parametrize("cin,cout,k,s,p,d", [(64, 64, 3, 1, 1, 1), (48, 40, 3, 2, 1, 1), (8, 16, 7, 2, 3, 1),
                                              (32, 32, 3, 1, 2, 2)])
def test_int8_conv_accumulators_brute_force(cin, cout, k, s, p, d):
    torch.manual_seed(0)
    x = torch.randint(-127, 127, (2, 9, 11, cin), dtype=torch.int8)
    w = torch.randint(-127, 127, (cout, k * k * cin), dtype=torch.int8)
    acc = ref.int8_conv2d_accumulators(x, w, k, k, s, s, p, p, d, d)
    exact = F.conv2d(x.permute(0, 3, 1, 2).double(), w.reshape(cout, k, k, cin).permute(0, 3, 1, 2).double(),
                     stride=s, padding=p, dilation=d).permute(0, 2, 3, 1)
    assert torch.equal(acc.double(), exact)


def test_int8_conv_epilogue_rounding_points():
    """acc * (a_scale * w_scale) then + bias as two FP32 roundings, then BF16 (ops/gemm.py:88-93); relu commutes."""
    torch.manual_seed(3)
    x = torch.randint(-127, 127, (1, 5, 6, 16), dtype=torch.int8)
    w = torch.randint(-127, 127, (24, 9 * 16), dtype=torch.int8)
    a_scale, w_scale = torch.tensor(0.017), torch.rand(24) * 0.01 + 0.001
    bias = torch.randn(24).to(torch.bfloat16)
    geo = (3, 3, 1, 1, 1, 1, 1, 1)
    out = ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo)
    acc = ref.int8_conv2d_accumulators(x, w, *geo).numpy().astype(np.float32)
    sc = (np.float32(a_scale.item()) * w_scale.numpy()).astype(np.float32)
    manual = (acc * sc).astype(np.float32) + bias.float().numpy()
    assert torch.equal(out, torch.from_numpy(manual.astype(np.float32)).to(torch.bfloat16))
    assert torch.equal(ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo, relu=True), F.relu(out))


def test_mxfp8_conv_matches_float64_conv_of_dequantized_operands():
    torch.manual_seed(4)
    x = (torch.randn(2, 7, 9, 64) * 3).to(torch.float8_e4m3fn)
    ce = torch.randint(-6, 3, (2,), dtype=torch.int8)
    w = (torch.randn(40, 9 * 64) * 2).to(torch.float8_e4m3fn)
    we = torch.randint(-9, -3, (40, 18), dtype=torch.int8)
    bias = torch.randn(40).to(torch.bfloat16)
    out = ref.mxfp8_conv2d(x, ce, w, we, bias, 3, 3, 1, 1, 1, 1, 1, 1).double()
    xd = x.double() * torch.exp2(ce.double()).repeat_interleave(32)
    wd = (w.double() * torch.exp2(we.double()).repeat_interleave(32, dim=1)).reshape(40, 3, 3, 64).permute(0, 3, 1, 2)
    exact = F.conv2d(xd.permute(0, 3, 1, 2), wd, bias.double(), padding=1).permute(0, 2, 3, 1)
    mag = F.conv2d(xd.abs().permute(0, 3, 1, 2), wd.abs(), bias.double().abs(), padding=1).permute(0, 2, 3, 1)
    assert ((out - exact).abs() <= exact.abs() * 2**-8 + mag * 2**-18).all()


def test_mxfp8_1x1_conv_is_the_linear():
    torch.manual_seed(5)
    x = (torch.randn(1, 3, 4, 64) * 3).to(torch.float8_e4m3fn)
    ce = torch.tensor([-2, 1], dtype=torch.int8)
    w = (torch.randn(32, 64)).to(torch.float8_e4m3fn)
    we = torch.randint(-5, 0, (32, 2), dtype=torch.int8)
    conv = ref.mxfp8_conv2d(x, ce, w, we, None, 1, 1, 1, 1, 0, 0, 1, 1)
    lin = ref.mxfp8_linear(x.reshape(12, 64), ce, None, w, we)
    assert torch.equal(conv.reshape(12, 32), lin)


# -- depthwise ---------------------------------------------------------------------------------------------------


def test_depthwise_oracle_against_float64():
    torch.manual_seed(6)
    x = torch.randn(2, 64, 9, 11)
    w = (torch.randn(25, 64) * 0.3).to(torch.bfloat16)
    b = torch.randn(64)
    scale = torch.tensor(0.03)
    q = ref.depthwise5x5_relu_int8(x, w, b, scale)
    exact = F.relu(F.conv2d(x.to(torch.bfloat16).double(), w.double().t().reshape(64, 1, 5, 5), b.double(),
                            padding=2, groups=64))
    want = (exact.to(torch.bfloat16).float() / 0.03).round().clamp(-127, 127).permute(0, 2, 3, 1).reshape(-1, 64)
    assert (q.float() - want).abs().max() <= 1 and (q.float() != want).float().mean() < 1e-3
    # all-zero rows (ReLU of large negative) -> exponent -127, zero codes (tests/ops/test_ops_cuda.py:67-69)
    z, zs = ref.depthwise5x5_relu_mxfp8(x, w, torch.full_like(b, -1e4))
    assert (z.float() == 0).all() and (zs[: 2 * 9 * 11 * 2] == 0).all()  # E8M0 0 = 2^-127


# -- the VGG stem: bias_relu_quantize_int8 / conv2d_small_cin_quantize_int8 -------------------------------------


def test_bias_relu_quantize_known_answers():
    """Hand-derived codes: ReLU, torch's round-half-even, saturation; and the dtype promotion of the bias add
    (ops/quantize.py:134-142): raw 1.0 + bias 2^-7 + 2^-10 is 1 + 2^-7 in BF16 (the 2^-10 is under half a BF16 step)
    -> 64.5 steps of 1/64 -> code 64 (tie to even), but 1.0087890625 in FP32 -> 64.5625 -> code 65."""
    raw = torch.tensor([-1.0, 0.0, 0.5, 1.5, 2.5, 200.0]).to(torch.bfloat16).view(1, 6, 1, 1)
    got = ref.bias_relu_quantize_int8(raw, torch.zeros(6, dtype=torch.bfloat16), torch.tensor(1.0))
    assert got.shape == (1, 1, 1, 6) and got.flatten().tolist() == [0, 0, 0, 2, 2, 127]
    one = torch.ones(1, 1, 1, 1, dtype=torch.bfloat16)
    b = 2.0**-7 + 2.0**-10
    assert ref.bias_relu_quantize_int8(one, torch.tensor([b], dtype=torch.bfloat16), torch.tensor(1 / 64)).item() == 64
    assert ref.bias_relu_quantize_int8(one, torch.tensor([b], dtype=torch.float32), torch.tensor(1 / 64)).item() == 65


def test_small_cin_oracle_against_float64():
    """torch's CPU BF16 conv is one BF16 rounding of the FP32-accumulated sum: against float64 of the same BF16
    operands rounded once to BF16 it differs by at most one BF16 step on a tiny fraction (accumulation order), and the
    INT8 codes by at most one step (FlashIM's own contract for this op, tests/ops/test_ops_cuda.py:543-555)."""
    torch.manual_seed(12)
    x = torch.randn(2, 3, 23, 37).to(torch.bfloat16)
    w = (torch.randn(32, 3, 3, 3) * 0.3).to(torch.bfloat16)
    bias = torch.randn(32).to(torch.bfloat16)
    scale = torch.tensor(0.04)
    conv = F.conv2d(x, w, None, padding=1)
    exact = F.conv2d(x.double(), w.double(), None, padding=1).to(torch.bfloat16)
    step = exact.float().abs().clamp_min(2.0**-126) * 2.0**-7
    assert ((conv.float() - exact.float()).abs() <= step).all() and (conv != exact).float().mean() < 1e-3
    got = ref.conv2d_small_cin_quantize_int8(x, scale, w, bias)
    want = ((F.relu(exact + bias.view(1, -1, 1, 1)).float() / 0.04).round().clamp(-127, 127)).permute(0, 2, 3, 1)
    assert got.shape == (2, 23, 37, 32) and got.dtype == torch.int8
    assert (got.float() - want).abs().max() <= 1 and (got.float() != want).float().mean() < 1e-3


# -- golden fixtures ---------------------------------------------------------------------------------------------


def test_golden_fixtures():
    """The committed fixtures (tests/golden/make_golden.py) still equal the oracle: catches a torch upgrade that
    changes any of the reference arithmetic."""
    from tests.golden import make_golden

    data = np.load(make_golden.PATH, allow_pickle=False)
    fresh = make_golden.compute()
    assert set(data.files) == set(fresh)
    for key in data.files:
        assert np.array_equal(data[key], fresh[key]), key
