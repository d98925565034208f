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
    g = torch.Generator().manual_seed(0)
    amax = torch.rand(10000, generator=g) * torch.exp2(torch.randint(-60, 60, (10000,), generator=g).float()) + 1e-30
    e = ref.scale_exponent_from_amax(amax).double()
    scaled = amax.double() / torch.exp2(e)
    # fits, up to FP32 log2's rounding just above a power of two: log2(2^k (1 + d)) rounds to k when d is under about
    # half an ulp of k (2^-17 relative for |k| < 64)
    assert (scaled <= 448 * (1 + 2**-17)).all()
    assert (amax.double() / torch.exp2(e - 1) > 448 * (1 - 2**-17)).all()  # one smaller power would not


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


def test_int8_channel_scale_multiplies_before_the_division():
    # ops/quantize.py:91-97: value * channel_scale (SmoothQuant's 1 / s), then round(. / scale). Dividing by the channel
    # scale instead would give [2, 12]; applying it after the rounding would give [6, 0] (round(3) * 0.25 -> 1 -> ...).
    x = torch.tensor([[3.0, 3.0], [-3.0, 100.0]])
    q = ref.quantize_int8(x, torch.tensor(1.0), torch.tensor([2.0, 0.25]))
    assert q.tolist() == [[6, 1], [-6, 25]]
    # scale and channel scale compose as (x * cs) / s: 10 * 0.5 / 0.25 = 20 (x / (cs * s) would give 80)
    assert ref.quantize_int8(torch.tensor([10.0]), torch.tensor(0.25), torch.tensor([0.5])).tolist() == [20]
    # saturation applies after the channel scale
    assert ref.quantize_int8(torch.tensor([100.0]), torch.tensor(1.0), torch.tensor([3.0])).tolist() == [127]


def test_quantize_int8_rows_reciprocal_scale():
    # ops/quantize.py:148-154: scale = amax * float32(1 / 127), not amax / 127. For amax = 5.798794 the two differ by
    # one FP32 ulp (0.04565979 against 0.045659795), and x = 0.068489686 then rounds to 2 under the reciprocal-product
    # scale but to 1 under the divided one.
    amax, x = np.float32("5.798794"), np.float32("0.068489686")
    recip = np.float32(amax * np.float32(np.float32(1) / np.float32(127)))
    divided = np.float32(amax / np.float32(127))
    assert recip != divided and np.rint(x / recip) == 2 and np.rint(x / divided) == 1
    rows = torch.tensor([[float(amax), float(x), -float(x), 0.0], [0.0, 0.0, 0.0, 0.0], [-1000.0, 2.0, 0.5, 1e-9]])
    q, s = ref.quantize_int8_rows(rows)
    assert s.shape == (3, 1) and s.dtype == torch.float32
    assert s[0, 0].item() == float(recip)
    assert q[0].tolist() == [127, 2, -2, 0]
    # all-zero row: safe_scale -> FP32 eps, codes 0 (tests/ops/test_ops_cuda.py:967-979 zeroes the last row)
    assert s[1, 0].item() == torch.finfo(torch.float32).eps and q[1].abs().sum() == 0
    # the row's amax element saturates to exactly -127/127 and every code is within half a step of the value
    assert q[2, 0].item() == -127
    assert ((q[2].double() * s[2, 0].double() - rows[2].double()).abs() <= s[2, 0].double() / 2).all()
    # per row: each row is scaled by its own amax (a transposed reduction would mix rows 0 and 2)
    torch.manual_seed(0)
    m = torch.randn(64, 96) * 3
    m[5] *= 300
    q, s = ref.quantize_int8_rows(m)
    assert torch.equal(q.abs().amax(1), torch.full((64,), 127, dtype=torch.int8))
    assert ((q.double() * s.double() - m.double()).abs() <= s.double() / 2 + 1e-12).all()


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


# -- pins of the remaining checker functions --------------------------------------------------------------------


def _bf16_np(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even of float32 values to BF16 by bit manipulation (independent of torch's conversion)."""
    bits = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return rounded.astype(np.uint32).view(np.float32)


def _gelu64(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + erf(x / sqrt 2)) in float64 (math.erf), the exact-erf GELU."""
    erf = np.vectorize(math.erf)
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def _mx_operand(rows, k, seed):
    g = torch.Generator().manual_seed(seed)
    values = (torch.randn(rows, k, generator=g) * 4).to(torch.float8_e4m3fn)
    exponent = torch.randint(-9, 4, (rows, k // 32), dtype=torch.int8, generator=g)
    dense = values.double() * torch.exp2(exponent.double()).repeat_interleave(32, dim=1)
    return values, exponent, dense


def test_mxfp8_scaled_mm_against_float64_of_dequantized_operands():
    """ops/gemm.py:21-52: a [M, K] with per-(row, 32) swizzled scales times b_t [K, N] (K != N, so a transposed b_t or
    swapped scale operands cannot pass) + bias, one BF16 rounding."""
    a, ae, ad = _mx_operand(150, 96, 0)
    b, be, bd = _mx_operand(40, 96, 1)  # b = b_t^T [N, K]
    bias = torch.randn(40).to(torch.bfloat16)
    out = ref.mxfp8_scaled_mm(a, b.t(), ref.swizzle_scales(ae), ref.swizzle_scales(be), bias)
    exact = ad @ bd.t() + bias.double()
    mag = ad.abs() @ bd.abs().t() + bias.double().abs()
    assert out.shape == (150, 40) and out.dtype == torch.bfloat16
    assert ((out.double() - exact).abs() <= exact.abs() * 2**-8 + mag * 2**-20).all()
    swapped = ref.mxfp8_scaled_mm(a, b.t(), ref.swizzle_scales(ae), ref.swizzle_scales(torch.roll(be, 1, 0)), bias)
    assert not torch.equal(swapped, out)


def test_mxfp8_gelu_mlp_against_explicit_step_chain():
    """ops/gemm.py:146-157 restated step by step in float64 / numpy: hidden = bf16(x W1^T); bf16(gelu(hidden + b1));
    static E4M3 with the hidden exponents; bf16(. W2^T). b1 enters before the GELU: adding it after fails the bar."""
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(64, 64, generator=g) * 4).to(torch.float8_e4m3fn)
    xe = torch.tensor([-3, -2], dtype=torch.int8)  # one static exponent per 32 channels, shared by the rows
    xd = x.double() * torch.exp2(xe.double()).repeat_interleave(32)
    w1, w1e, w1d = _mx_operand(256, 64, 3)
    w2, w2e, w2d = _mx_operand(64, 256, 4)
    w1e, w2e = w1e.clamp(-7, -5), w2e.clamp(-7, -5)
    w1d = w1.double() * torch.exp2(w1e.double()).repeat_interleave(32, dim=1)
    w2d = w2.double() * torch.exp2(w2e.double()).repeat_interleave(32, dim=1)
    b1 = torch.randn(256, generator=g)
    he = torch.full((8,), -6, dtype=torch.int8)
    got = ref.mxfp8_gelu_mlp(x, xe, w1, w1e, b1, he, w2, w2e).double()

    def chain(bias_first: bool) -> torch.Tensor:
        hidden = _bf16_np((xd @ w1d.t()).numpy().astype(np.float32)).astype(np.float64)
        act = _gelu64(hidden + b1.double().numpy()) if bias_first else _gelu64(hidden) + b1.double().numpy()
        act = _bf16_np(act.astype(np.float32))
        q = torch.from_numpy((act * 64).clip(-448, 448).astype(np.float32)).to(torch.float8_e4m3fn).double() / 64
        return torch.from_numpy(_bf16_np((q @ w2d.t()).numpy().astype(np.float32))).double()

    want = chain(True)
    assert (got - want).norm() / want.norm() < 2e-3
    wrong = chain(False)
    assert (wrong - want).norm() / want.norm() > 5e-2


@pytest.mark.parametrize("h,w", [(8, 10), (7, 9)])
def test_int8_conv2d_maxpool_against_brute_force_window_max(h, w):
    """ops/conv.py:209-222: the pooled codes are quantize(max over each 2x2 window of the BF16 conv output), odd
    trailing rows and columns dropped."""
    torch.manual_seed(7)
    x = torch.randint(-127, 127, (2, h, w, 16), dtype=torch.int8)
    wt = torch.randint(-127, 127, (24, 9 * 16), dtype=torch.int8)
    args = (x, wt, torch.tensor(0.02), torch.rand(24) * 0.01, torch.randn(24), 3, 3, 1, 1, 1, 1, 1, 1)
    out, pooled = ref.int8_conv2d_maxpool(*args, relu=True, out_scale=torch.tensor(0.05))
    assert torch.equal(out, ref.int8_conv2d(*args, relu=True))
    o = out.float().numpy()
    want = np.empty((2, h // 2, w // 2, 24), np.float32)
    for y2 in range(h // 2):
        for x2 in range(w // 2):
            want[:, y2, x2] = o[:, 2 * y2: 2 * y2 + 2, 2 * x2: 2 * x2 + 2].max(axis=(1, 2))
    codes = np.clip(np.rint(want / np.float32(0.05)), -127, 127)
    assert pooled.shape == want.shape and np.array_equal(pooled.numpy(), codes.astype(np.int8))


def test_depthwise5x5_gelu_against_float64():
    """The producer: BF16 depthwise conv (FP32 accumulate) + bias -> BF16 -> GELU in BF16 (-> the consumer's quantize),
    against a float64 tap loop, float64 GELU, and BF16 roundings by bit manipulation."""
    torch.manual_seed(8)
    x = torch.randn(1, 32, 9, 12) * 2
    wt = (torch.randn(25, 32) * 0.3).to(torch.bfloat16)
    b = torch.randn(32)
    xb = x.to(torch.bfloat16).double().numpy()[0]  # [C, H, W]
    pad = np.pad(xb, ((0, 0), (2, 2), (2, 2)))
    conv = np.zeros_like(xb)
    wn = wt.double().numpy()
    for ky in range(5):
        for kx in range(5):
            conv += wn[ky * 5 + kx][:, None, None] * pad[:, ky: ky + 9, kx: kx + 12]
    conv += b.double().numpy()[:, None, None]
    pre = _bf16_np(conv.astype(np.float32))
    want = _bf16_np(_gelu64(pre.astype(np.float64)).astype(np.float32)).transpose(1, 2, 0).reshape(-1, 32)
    got = ref.depthwise5x5_gelu(x, wt, b).float().numpy()
    step = np.maximum(np.abs(want), 2.0**-126) * 2.0**-7
    # torch's CPU GELU of a BF16 tensor uses a vectorized erf: one BF16 step apart on a few percent of the values
    assert (np.abs(got - want) <= step + 2.0**-14).all() and (got != want).mean() < 0.1
    q = ref.depthwise5x5_gelu(x, wt, b, scale=torch.tensor(0.02)).numpy()
    assert np.abs(q - np.clip(np.rint(want / np.float32(0.02)), -127, 127)).max() <= 1


def test_add_residual_against_numpy_including_narrow_residual():
    """ops/conv.py:198-203: out + residual in FP32 over the residual's channels (a narrower residual leaves the other
    channels unchanged), optional ReLU over all channels, then one BF16 rounding."""
    torch.manual_seed(9)
    out = torch.randn(2, 3, 4, 48).to(torch.bfloat16)
    res = torch.randn(2, 3, 4, 40).to(torch.bfloat16)
    for relu in (False, True):
        got = ref.add_residual(out, res, relu).float().numpy()
        s = out.float().numpy().copy()
        s[..., :40] = s[..., :40] + res.float().numpy()
        if relu:
            s = np.maximum(s, 0)
        assert np.array_equal(got, _bf16_np(s.astype(np.float32)))


def test_int8_linear_epilogue_order_relu_gelu_residual():
    """ops/gemm.py:88-98: FP32 dequant + bias, ReLU, BF16, GELU in BF16, then residual + out in BF16 (residual after
    GELU: adding it first gives different bits)."""
    torch.manual_seed(10)
    a = torch.randint(-127, 127, (33, 64), dtype=torch.int8)
    w = torch.randint(-127, 127, (24, 64), dtype=torch.int8)
    a_s, w_s, bias = torch.tensor(0.004), torch.rand(24) * 0.01, torch.randn(24)
    res = torch.randn(33, 24).to(torch.bfloat16)
    got = ref.int8_linear(a, w, a_s, w_s, bias, relu=True, gelu=True, residual=res).float().numpy()
    acc = (a.long() @ w.long().t()).numpy().astype(np.float32)
    y = (acc * (np.float32(a_s.item()) * w_s.numpy()).astype(np.float32)).astype(np.float32) + bias.numpy()
    y = _bf16_np(np.maximum(y, 0).astype(np.float32))
    y = _bf16_np(_gelu64(y.astype(np.float64)).astype(np.float32))
    want = _bf16_np((y + res.float().numpy()).astype(np.float32))
    assert np.abs(got - want).max() <= np.abs(want).max() * 2**-7 and (got != want).mean() < 2e-2
    wrong = _bf16_np(_gelu64((y + res.float().numpy()).astype(np.float64)).astype(np.float32))
    assert (np.abs(wrong - want) > 0.05).mean() > 0.2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gelu_quantize_producers_against_float64(dtype):
    """ops/quantize.py:63-74, 128-131: GELU in the value's dtype (with input_bias: FP32 GELU of the sum, rounded back)
    then the pinned static quantizers."""
    torch.manual_seed(11)
    x = (torch.randn(40, 64) * 3).to(dtype)
    bias = torch.randn(64)
    e = torch.tensor([-6, -6], dtype=torch.int8)
    for input_bias in (None, bias):
        v = x.double().numpy() + (0 if input_bias is None else bias.double().numpy())
        g = _gelu64(v).astype(np.float32)
        if dtype == torch.bfloat16:
            g = _bf16_np(g)
        want = ref.quantize_static(torch.from_numpy(g).to(dtype), e).view(torch.uint8)
        got = ref.gelu_quantize(x, e, input_bias=input_bias).view(torch.uint8)
        assert (got != want).float().mean() < 1e-2
        step = torch.from_numpy(g).abs().double() * 2**-3 * 64 + 2**-9
        diff = (got.view(torch.float8_e4m3fn).double() - want.view(torch.float8_e4m3fn).double()).abs()
        assert (diff <= step).all()
    gi = ref.gelu_quantize_int8(x, torch.tensor(0.05)).numpy()
    g = _gelu64(x.double().numpy()).astype(np.float32)
    g = _bf16_np(g) if dtype == torch.bfloat16 else g
    assert np.abs(gi - np.clip(np.rint(g / np.float32(0.05)), -127, 127)).max() <= 1


def _gelu_tanh64(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3))) in float64."""
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x**3)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gelu_quantize_tanh_form_against_float64(dtype):
    """approximate="tanh" reaches F.gelu's tanh form (ops/quantize.py:63-74, 128-131), not the erf form: at x = 1 the
    two differ by 1.5e-4 (0.841192 against 0.841345)."""
    assert abs(_gelu_tanh64(np.array([1.0]))[0] - 0.8411919906082768) < 1e-15
    x = torch.linspace(-6, 6, 4800).reshape(75, 64).to(dtype)
    s = torch.tensor(0.05)
    g = _gelu_tanh64(x.double().numpy()).astype(np.float32)
    g = _bf16_np(g) if dtype == torch.bfloat16 else g
    gi = ref.gelu_quantize_int8(x, s, approximate="tanh").numpy()
    want = np.clip(np.rint(g / np.float32(0.05)), -127, 127)
    assert np.abs(gi - want).max() <= 1 and (gi != want).mean() < 1e-2
    e = torch.tensor([-6, -6], dtype=torch.int8)
    got = ref.gelu_quantize(x, e, approximate="tanh").view(torch.float8_e4m3fn).double() * 2**-6
    exact = torch.from_numpy(g).double()
    assert ((got - exact).abs() <= exact.abs() * 2**-4 + 2**-6 * 2**-9).all()
    # the forms part in the negative tail: GELU(-2.5) is -0.015084 (tanh) against -0.015524 (erf), codes -15 / -16
    # at scale 1e-3
    tail = torch.full((1, 64), -2.5)
    assert ref.gelu_quantize_int8(tail, torch.tensor(1e-3), approximate="tanh")[0, 0].item() == -15
    assert ref.gelu_quantize_int8(tail, torch.tensor(1e-3))[0, 0].item() == -16


def test_int8_linear_quantize_is_the_requantized_linear():
    """ops/gemm.py:104-116: round_half_even(int8_linear(...) / out_scale) saturated, computed here in numpy."""
    torch.manual_seed(12)
    a = torch.randint(-127, 127, (50, 32), dtype=torch.int8)
    w = torch.randint(-127, 127, (16, 32), dtype=torch.int8)
    args = (a, w, torch.tensor(0.01), torch.rand(16) * 0.01, torch.randn(16).to(torch.bfloat16))
    got = ref.int8_linear_quantize(*args, torch.tensor(0.3)).numpy()
    lin = ref.int8_linear(*args).float().numpy()
    assert np.array_equal(got, np.clip(np.rint(lin / np.float32(0.3)), -127, 127).astype(np.int8))


def test_pointwise_composites_against_float64_on_the_producer_codes():
    """ops/conv.py:93-138: each block is its producer's codes through the pinned GEMM; recomputed in float64 from the
    dequantized codes (MXFP8) and exactly in int64 (INT8)."""
    torch.manual_seed(13)
    x = torch.randn(1, 64, 6, 7)
    dw_w, dw_b = (torch.randn(25, 64) * 0.3).to(torch.bfloat16), torch.randn(64)
    pw, pe, pwd = _mx_operand(64, 64, 14)
    pb = torch.randn(64)
    out = ref.depthwise5x5_relu_pointwise_mxfp8(x, dw_w, dw_b, pw, ref.swizzle_scales(pe), ref.exponent_to_e8m0(pe),
                                                pb)
    codes, swz = ref.depthwise5x5_relu_mxfp8(x, dw_w, dw_b)
    deq = ref.dequantize_swizzled(codes, swz).double()
    exact = (deq @ pwd.t() + pb.double()).reshape(1, 6, 7, 64).permute(0, 3, 1, 2)
    mag = (deq.abs() @ pwd.abs().t() + pb.double().abs()).reshape(1, 6, 7, 64).permute(0, 3, 1, 2)
    assert ((out.double() - exact).abs() <= exact.abs() * 2**-8 + mag * 2**-20).all()
    w8 = torch.randint(-127, 127, (64, 64), dtype=torch.int8)
    ws, s = torch.rand(64) * 0.01, torch.tensor(0.05)
    out8 = ref.depthwise5x5_relu_pointwise_int8(x, dw_w, dw_b, w8, ws, pb, s).permute(0, 2, 3, 1).reshape(-1, 64)
    q = ref.depthwise5x5_relu_int8(x, dw_w, dw_b, s)
    acc = (q.long() @ w8.long().t()).numpy().astype(np.float32)
    y = (acc * (np.float32(0.05) * ws.numpy()).astype(np.float32)).astype(np.float32) + pb.numpy()
    assert np.array_equal(out8.float().numpy(), _bf16_np(y.astype(np.float32)))


def test_bf16_pointwise_block_against_shifted_window_float64():
    """ops/conv.py:67-81: the depthwise window as 25 shifted slices of the zero-padded image in float64 (no F.conv2d),
    ReLU, BF16, then a float64 GEMM with C_out != C (a transposed weight cannot even multiply), bias, BF16. The oracle
    accumulates in FP32, so the bar is one BF16 step of the result plus the FP32 error of the sums."""
    torch.manual_seed(21)
    b, c, h, w, n = 2, 32, 7, 9, 48
    x = torch.randn(b, c, h, w).to(torch.bfloat16)
    dw_w, dw_b = (torch.randn(25, c) * 0.3).to(torch.bfloat16), torch.randn(c).to(torch.bfloat16)
    pw, pb = (torch.randn(n, c) * 0.2).to(torch.bfloat16), torch.randn(n).to(torch.bfloat16)
    out = ref.depthwise5x5_relu_pointwise(x, dw_w, dw_b, pw, pb)
    assert out.shape == (b, n, h, w) and out.is_contiguous(memory_format=torch.channels_last)
    xp = F.pad(x.double(), (2, 2, 2, 2))
    hidden = dw_b.double().view(1, c, 1, 1).expand(b, c, h, w).clone()
    for ky in range(5):
        for kx in range(5):
            hidden += xp[:, :, ky:ky + h, kx:kx + w] * dw_w[ky * 5 + kx].double().view(1, c, 1, 1)
    hidden = hidden.clamp_min(0).to(torch.bfloat16).double()
    rows = hidden.permute(0, 2, 3, 1).reshape(-1, c)
    exact = rows @ pw.double().t() + pb.double()
    mag = rows.abs() @ pw.double().abs().t() + pb.double().abs()
    got = out.permute(0, 2, 3, 1).reshape(-1, n).double()
    assert ((got - exact).abs() <= exact.abs() * 2**-8 + mag * 2**-18).all()


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
