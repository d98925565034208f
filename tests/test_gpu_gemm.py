"""HIP GEMM-shaped ops vs the oracle: ``int8_linear`` bit-exact (FlashIM's INT8 contract tests/ops/test_ops_cuda.py:
470-501 applied to the GEMM, per-tensor and per-row activation scales, every epilogue), ``mxfp8_linear`` and
``mxfp8_scaled_mm`` within the MXFP8 tolerance (rel-L2 <= 1e-3, tests/ops/test_ops_cuda.py:608-637), ``im2col_gather``
byte-exact (its oracle pinned to F.unfold in the CPU tests), and the two depthwise-then-pointwise composites
(ops/conv.py:93-138)."""

import pytest
import torch
import torch.nn.functional as F

from flashim_amd import _lib, library, ops, quant
from flashim_amd.backends.hip import conv as hip_conv
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _assert_mx_close(fast, want):
    """Relative L2 <= 1e-3; per element |diff| <= max(1e-2 x output RMS, 2^-7 |want|): one BF16 rounding step of the
    reference value covers a final rounding flipped by the other FP32 accumulation order."""
    fast, want = fast.float(), want.float()
    rms = want.pow(2).mean().sqrt()
    rel = (fast - want).norm() / want.norm()
    assert rel <= 1e-3, rel
    assert ((fast - want).abs() <= torch.maximum(1e-2 * rms, want.abs() * 2**-7)).all()


def _gelu_close(got, want):
    """The kernel's erf is a Chebyshev fit, torch's is libm: within one BF16 rounding plus an absolute 2^-12 floor
    for GELU's tail."""
    diff = (got.float() - want.float()).abs()
    assert (diff <= want.float().abs() * 2**-7 + 2**-12).all()


def _int8_linear_inputs(m, k, n, seed=0):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
    w_scale = torch.rand(n, generator=g) * 0.01 + 0.001
    return a, w, w_scale, g


INT8_SHAPES = [(1, 16, 8), (300, 128, 96), (777, 256, 256), (64, 40, 24), (129, 7, 200), (2000, 512, 64)]


@pytest.mark.parametrize("m,k,n", INT8_SHAPES)
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("bias_dtype", [None, torch.bfloat16, torch.float32])
def test_int8_linear_bit_exact(m, k, n, per_row, bias_dtype):
    a, w, w_scale, g = _int8_linear_inputs(m, k, n)
    a_scale = (torch.rand(m, 1, generator=g) * 0.05 + 0.001) if per_row else torch.tensor(0.017)
    bias = None if bias_dtype is None else torch.randn(n, generator=g).to(bias_dtype)
    hip = ops.int8_linear.get("hip")
    d = [t.to(DEV) if t is not None else None for t in (a, w, a_scale, w_scale, bias)]
    got = hip(*d).cpu()
    want = ref.int8_linear(a, w, a_scale, w_scale, bias)
    assert got.dtype == torch.bfloat16 and got.shape == (m, n)
    assert torch.equal(got, want)
    assert torch.equal(hip(*d, relu=True).cpu(), ref.int8_linear(a, w, a_scale, w_scale, bias, relu=True))
    residual = torch.randn(m, n, generator=g).to(torch.bfloat16)
    got = hip(*d, relu=True, residual=residual.to(DEV)).cpu()
    assert torch.equal(got, ref.int8_linear(a, w, a_scale, w_scale, bias, relu=True, residual=residual))


@pytest.mark.parametrize("m,k,n", [(300, 128, 96), (1000, 64, 256)])
def test_int8_linear_gelu(m, k, n):
    a, w, w_scale, g = _int8_linear_inputs(m, k, n, seed=3)
    a_scale = torch.tensor(0.01)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    residual = torch.randn(m, n, generator=g).to(torch.bfloat16)
    d = [t.to(DEV) for t in (a, w, a_scale, w_scale, bias)]
    got = ops.int8_linear.get("hip")(*d, gelu=True).cpu()
    _gelu_close(got, ref.int8_linear(a, w, a_scale, w_scale, bias, gelu=True))
    # the residual add is one more BF16 rounding of (gelu + residual): within one step of the reference sum
    got = ops.int8_linear.get("hip")(*d, gelu=True, residual=residual.to(DEV)).cpu().float()
    want = ref.int8_linear(a, w, a_scale, w_scale, bias, gelu=True, residual=residual).float()
    assert ((got - want).abs() <= want.abs() * 2**-7 + 2**-11).all()


def test_int8_linear_accumulators_are_exact():
    """Unit scales and no bias: the outputs are the int32 accumulators rounded to BF16."""
    a, w, _, _ = _int8_linear_inputs(513, 1024, 128, seed=5)
    got = ops.int8_linear.get("hip")(a.to(DEV), w.to(DEV), torch.tensor(1.0, device=DEV),
                                     torch.ones(128, device=DEV), None).cpu()
    assert torch.equal(got, ref.int8_accumulators(a, w).float().to(torch.bfloat16))


def _mx_activation(rows, channels, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, channels, generator=g) * torch.exp(torch.empty(channels).uniform_(-2, 2, generator=g))
    exponent = ref.calibrate_block32_exponent(x)
    return ref.quantize_static(x, exponent), exponent, g


@pytest.mark.parametrize("rows,k,n", [(1, 32, 32), (300, 256, 96), (2048, 512, 512), (77, 1152, 128)])
@pytest.mark.parametrize("has_bias", [False, True])
def test_mxfp8_linear(rows, k, n, has_bias):
    values, exponent, g = _mx_activation(rows, k, rows + k)
    w_values, w_exponent = ref.quantized_weight_from_float(torch.randn(n, k, generator=g) * 0.05)
    bias = torch.randn(n, generator=g).to(torch.bfloat16) if has_bias else None
    act = quant.QuantizedTensor(values.to(DEV), exponent.to(DEV), (rows, k))
    weight = quant.QuantizedWeight(w_values.to(DEV), w_exponent.to(DEV), (n, k))
    got = ops.mxfp8_linear.get("hip")(act, None if bias is None else bias.to(DEV), weight).cpu()
    want = ref.mxfp8_linear(values, exponent, bias, w_values, w_exponent)
    assert got.shape == want.shape and got.dtype == torch.bfloat16
    _assert_mx_close(got, want)


# the last four have at least two 256-row tiles per CU (256 CUs) and run the register-operand pointwise kernel with
# per-row swizzled scales (K = 1024: two load phases of 4 K steps, a partial last tile); the others the one-round
# kernels
@pytest.mark.parametrize("m,k,n", [(1, 32, 32), (300, 256, 96), (4096, 128, 128), (1000, 512, 320),
                                   (140000, 128, 128), (70000, 256, 256), (40001, 512, 512), (65600, 1024, 256)])
@pytest.mark.parametrize("has_bias", [False, True])
def test_mxfp8_scaled_mm(m, k, n, has_bias):
    g = torch.Generator().manual_seed(m + n)
    a, a_exp = ref.quantize_dynamic_2d(torch.randn(m, k, generator=g) * 3)
    b, b_exp = ref.quantized_weight_from_float(torch.randn(n, k, generator=g) * 0.05)
    a_scale, b_scale = ref.swizzle_scales(a_exp), ref.swizzle_scales(b_exp)
    bias = torch.randn(n, generator=g) if has_bias else None
    b_t = b.t()
    got = ops.mxfp8_scaled_mm.get("hip")(a.to(DEV), b.to(DEV).t(), a_scale.to(DEV), b_scale.to(DEV),
                                         None if bias is None else bias.to(DEV)).cpu()
    want = ref.mxfp8_scaled_mm(a, b_t, a_scale, b_scale, bias)
    assert got.shape == (m, n) and got.dtype == torch.bfloat16
    _assert_mx_close(got, want)
    # the weight scales as E8M0 bytes (the refiner-block ops' pw_scale_u8) give the same bits on every kernel
    b_e8m0 = ref.exponent_to_e8m0(b_exp).view(torch.int8)
    args = (a.view(torch.uint8).to(DEV), a_scale.view(torch.uint8).to(DEV), b.view(torch.uint8).to(DEV))
    bias_d = None if bias is None else bias.to(DEV)
    signed = library.mxfp8_scaled_mm(*args, b_exp.to(torch.int8).to(DEV), bias_d)
    biased = library.mxfp8_scaled_mm(*args, b_e8m0.to(DEV), bias_d, True)
    assert torch.equal(signed.view(torch.int16), biased.view(torch.int16))
    assert torch.equal(signed.cpu().view(torch.int16), got.view(torch.int16))


IM2COL = [
    ((2, 17, 19, 64), (3, 3, 1, 1, 1, 1, 1, 1)),
    ((1, 9, 11, 6), (3, 3, 2, 2, 1, 1, 1, 1)),
    ((2, 16, 16, 32), (3, 3, 1, 1, 2, 2, 2, 2)),
    ((1, 20, 13, 8), (7, 7, 2, 2, 3, 3, 1, 1)),
    ((3, 5, 5, 48), (1, 1, 1, 1, 0, 0, 1, 1)),
    ((1, 12, 12, 128), (5, 5, 1, 1, 0, 0, 1, 1)),
]


@pytest.mark.parametrize("shape,geo", IM2COL)
@pytest.mark.parametrize("dtype", [torch.int8, torch.float8_e4m3fn])
def test_im2col_gather_byte_exact(shape, geo, dtype):
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randint(-128, 128, shape, dtype=torch.int8, generator=g)
    if dtype == torch.float8_e4m3fn:
        x = x.view(torch.uint8).clamp(max=0x7E).view(torch.float8_e4m3fn)  # no NaN codes
    got = ops.im2col_gather.get("hip")(x.to(DEV), *geo).cpu()
    want = ref.im2col_gather(x, *geo)
    assert got.dtype == dtype and got.shape == want.shape
    assert torch.equal(got.view(torch.uint8), want.view(torch.uint8))


def _block_inputs(batch, channels, hw, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(batch, channels, *hw, generator=g) * 2).to(torch.bfloat16)
    x = x.contiguous(memory_format=torch.channels_last)
    dw_w = (torch.randn(25, channels, generator=g) * 0.3).to(torch.bfloat16)
    dw_b = torch.randn(channels, generator=g)
    pw_b = torch.randn(channels, generator=g)
    return x, dw_w, dw_b, pw_b, g


# (1, 128, (256, 256)): 256 tiles of the one-kernel block, inside its band on 256 CUs (the op takes the one kernel)
@pytest.mark.parametrize("batch,channels,hw", [(2, 64, (20, 30)), (1, 128, (33, 17)), (2, 32, (5, 7)), (1, 128, (256, 256))])
def test_depthwise_pointwise_int8(batch, channels, hw):
    x, dw_w, dw_b, pw_b, g = _block_inputs(batch, channels, hw, seed=channels)
    pw_w = torch.randint(-127, 128, (channels, channels), dtype=torch.int8, generator=g)
    pw_s = torch.rand(channels, generator=g) * 0.01 + 0.001
    scale = torch.tensor(0.03)
    args = (x, dw_w, dw_b, pw_w, pw_s, pw_b, scale)
    got = ops.depthwise5x5_relu_pointwise_int8.get("hip")(*[t.to(DEV) for t in args])
    assert got.shape == (batch, channels, *hw) and got.is_contiguous(memory_format=torch.channels_last)
    # exact against the oracle GEMM on the producer's own codes (the producer is within one code of the oracle's)
    codes = ops.depthwise5x5_relu_int8.get("hip")(*[t.to(DEV) for t in (x, dw_w, dw_b, scale)]).cpu()
    want = ref.int8_linear(codes, pw_w, scale, pw_s, pw_b).reshape(batch, *hw, channels).permute(0, 3, 1, 2)
    assert torch.equal(got.cpu(), want)
    end_to_end = ref.depthwise5x5_relu_pointwise_int8(*args).float()
    rel = (got.cpu().float() - end_to_end).norm() / end_to_end.norm()
    assert rel < 1e-2


# (1, 128, (256, 256)): 256 tiles of the one-kernel block, inside its band on 256 CUs (the op takes the one kernel)
@pytest.mark.parametrize("batch,channels,hw", [(2, 64, (20, 30)), (1, 128, (33, 17)), (2, 32, (5, 7)), (1, 128, (256, 256))])
def test_depthwise_pointwise_mxfp8(batch, channels, hw):
    x, dw_w, dw_b, pw_b, g = _block_inputs(batch, channels, hw, seed=channels + 1)
    pw_w, pw_e = ref.quantized_weight_from_float(torch.randn(channels, channels, generator=g) * 0.1)
    pw_sw, pw_u8 = ref.swizzle_scales(pw_e), ref.exponent_to_e8m0(pw_e)
    args = (x, dw_w, dw_b, pw_w, pw_sw, pw_u8, pw_b)
    got = ops.depthwise5x5_relu_pointwise_mxfp8.get("hip")(*[t.to(DEV) for t in args])
    assert got.shape == (batch, channels, *hw) and got.is_contiguous(memory_format=torch.channels_last)
    q, s = ops.depthwise5x5_relu_mxfp8.get("hip")(*[t.to(DEV) for t in (x, dw_w, dw_b)])
    want = ref.mxfp8_scaled_mm(q.cpu(), pw_w.t(), s.cpu(), pw_sw, pw_b)
    _assert_mx_close(got.cpu().permute(0, 2, 3, 1).reshape(-1, channels), want)
    end_to_end = ref.depthwise5x5_relu_pointwise_mxfp8(*args).float()
    rel = (got.cpu().float() - end_to_end).norm() / end_to_end.norm()
    assert rel < 1e-2


# the reference's BF16 block cases (tests/ops/test_ops_cuda.py:230-243; its 16-channel case needs C % 32 == 0 here and
# takes FlashIM's own path), plus a C_out != C weight and a ragged last pixel block
BF16_BLOCK = [(32, 32, (37, 53)), (32, 32, (256, 256)), (64, 64, (40, 48)), (64, 64, (130, 97)), (128, 128, (45, 67)),
              (64, 48, (9, 11)), (96, 128, (3, 5))]


@pytest.mark.parametrize("channels,cout,hw", BF16_BLOCK)
def test_depthwise_relu_pointwise_bf16(channels, cout, hw):
    """The reference's contract (tests/ops/test_ops_cuda.py:230-243): FP32 reduction order may differ, at most one
    BF16 step (|d| <= |ref| 2^-7 + 1e-6). The GEMM half meets it everywhere on this producer's own hidden tensor. The
    hidden tensor is the depthwise sum rounded to BF16, where a different FP32 order flips a rounding for about 1 in
    10^5 values (one BF16 step, the depthwise producer's contract); the few outputs downstream of such a flip are
    bounded by one hidden step times the weight row's magnitude, and their fraction is held below 10^-5."""
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, channels, *hw, generator=g).contiguous(memory_format=torch.channels_last)
    dw = (torch.randn(25, channels, generator=g) * 0.2).to(torch.bfloat16)
    dwb = torch.randn(channels, generator=g).to(torch.bfloat16)
    pw = (torch.randn(cout, channels, generator=g) * 0.2).to(torch.bfloat16).contiguous()
    pwb = torch.randn(cout, generator=g).to(torch.bfloat16)
    args = (x, dw, dwb, pw, pwb)
    assert ops.depthwise5x5_relu_pointwise.supports(*[t.to(DEV) for t in args])
    got = ops.depthwise5x5_relu_pointwise(*[t.to(DEV) for t in args])
    assert got.shape == (2, cout, *hw) and got.is_contiguous(memory_format=torch.channels_last)
    want = ref.depthwise5x5_relu_pointwise(*args).float()
    hidden = library.depthwise5x5(hip_conv._nhwc_bf16(x.to(DEV)), dw.to(DEV), dwb.float().to(DEV), 0,
                                  library.DW_BF16, None, None).cpu().float()
    gemm = (hidden @ pw.float().t() + pwb.float()).to(torch.bfloat16).float()
    flat = got.cpu().permute(0, 2, 3, 1).reshape(-1, cout).float()
    assert ((flat - gemm).abs() <= gemm.abs() * 2**-7 + 1e-6).all()
    kernel = dw.float().t().reshape(channels, 1, 5, 5)
    hid_ref = F.relu(F.conv2d(x.to(torch.bfloat16).float(), kernel, dwb.float(), padding=2, groups=channels))
    hid_ref = hid_ref.to(torch.bfloat16).float().permute(0, 2, 3, 1).reshape(-1, channels)
    flips = hidden != hid_ref
    assert flips.float().mean() < 1e-4
    # one BF16 step at most, or (a sum within FP32 error of 0 on either side of the ReLU) the sum's FP32 error
    mag = F.conv2d(x.to(torch.bfloat16).float().abs(), kernel.abs(), dwb.float().abs(), padding=2, groups=channels)
    mag = mag.permute(0, 2, 3, 1).reshape(-1, channels)
    assert ((hidden - hid_ref).abs() <= torch.maximum(hidden.abs(), hid_ref.abs()) * 2**-7 + mag * 2**-20).all()
    got = got.cpu().float()
    strict = (got - want).abs() <= want.abs() * 2**-7 + 1e-6
    step = (hidden - hid_ref).abs() @ pw.float().abs().t()  # the hidden differences through the weights
    loose = (got - want).abs().permute(0, 2, 3, 1).reshape(-1, cout) <= \
        want.abs().permute(0, 2, 3, 1).reshape(-1, cout) * 2**-7 + step * 1.01 + 1e-6
    assert loose.all() and (~strict).float().mean() < 1e-5


def test_pointwise_bf16_rejects_unsupported_shapes():
    x = torch.zeros(16, 48, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(_lib.UnsupportedShape):
        library.pointwise_bf16(x, torch.zeros(32, 48, device=DEV, dtype=torch.bfloat16), None)
    y = library.pointwise_bf16(x[:, :32].contiguous(), torch.zeros(32, 32, device=DEV, dtype=torch.bfloat16), None)
    assert y.shape == (16, 32) and not y.float().abs().any()


# the last two have more tiles than the persistent grid's workgroups (512 on 256 CUs): each workgroup runs several
# tiles, prefetching the next tile's first window during the pointwise of the current one
FUSED_BLOCK = [(1, (8, 32)), (2, (19, 45)), (1, (3, 5)), (2, (40, 70)), (1, (1, 1)), (2, (203, 331)), (1, (400, 400))]


@pytest.mark.parametrize("batch,hw", FUSED_BLOCK)
@pytest.mark.parametrize("bias", ["fp32", "bf16", "none"])
def test_fused_depthwise_pointwise_matches_composite(batch, hw, bias):
    """C = 128 with a 128 x 128 pointwise weight runs as one kernel (flashim/backends/triton/conv.py:310-508's
    shapes, MXFP8): bit for bit the two-launch composite it replaces (same producer arithmetic, same MFMA per output
    block); tiles cut by the image edges, images smaller than the halo, every bias form."""
    channels = 128
    x, dw_w, dw_b, pw_b, g = _block_inputs(batch, channels, hw, seed=sum(hw) + batch)
    pw_b = {"fp32": pw_b, "bf16": pw_b.to(torch.bfloat16), "none": None}[bias]
    dev = lambda ts: [t.to(DEV) if t is not None else None for t in ts]  # noqa: E731
    pw_w, pw_e = ref.quantized_weight_from_float(torch.randn(channels, channels, generator=g) * 0.1)
    args = dev((x, dw_w, dw_b, pw_w, ref.swizzle_scales(pw_e), ref.exponent_to_e8m0(pw_e), pw_b))
    fused = hip_conv.pointwise_mxfp8_fused(*args)
    composite = hip_conv.pointwise_mxfp8_composite(*args)
    assert fused.shape == composite.shape == (batch, channels, *hw)
    assert torch.equal(fused.view(torch.int16), composite.view(torch.int16))


@pytest.mark.parametrize("batch,hw", FUSED_BLOCK)
@pytest.mark.parametrize("bias", ["fp32", "bf16", "none"])
def test_fused_depthwise_pointwise_int8_matches_composite(batch, hw, bias):
    """The INT8 block as one kernel (flashim/backends/triton/conv.py:417-475, registered for C = 128 at :585-599):
    bit for bit the composite (the INT8 depthwise producer, then int8_linear; exact int32 sums, the same FP32
    epilogue), and the composite within the oracle's bar; a scale small enough that many codes saturate at 127."""
    channels = 128
    x, dw_w, dw_b, pw_b, g = _block_inputs(batch, channels, hw, seed=3 * sum(hw) + batch)
    pw_b = {"fp32": pw_b, "bf16": pw_b.to(torch.bfloat16), "none": None}[bias]
    dev = lambda ts: [t.to(DEV) if t is not None else None for t in ts]  # noqa: E731
    pw_w = torch.randint(-127, 128, (channels, channels), dtype=torch.int8, generator=g)
    pw_s = torch.rand(channels, generator=g) * 0.01 + 0.001
    for scale in (torch.tensor(0.03), torch.tensor(0.004)):
        args = dev((x, dw_w, dw_b, pw_w, pw_s, pw_b, scale))
        fused = hip_conv.pointwise_int8_fused(*args)
        composite = hip_conv.pointwise_int8_composite(*args)
        assert fused.shape == composite.shape == (batch, channels, *hw)
        assert torch.equal(fused.view(torch.int16), composite.view(torch.int16))
        assert torch.equal(ops.depthwise5x5_relu_pointwise_int8.get("hip")(*args).view(torch.int16),
                           composite.view(torch.int16))
