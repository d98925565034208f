"""HIP implicit-GEMM convs vs the oracle.

INT8 (FlashIM's contract tests/ops/test_ops_cuda.py:470-501): the BF16 output is bit-identical to the reference, and so
are the int32 accumulators (checked through a unit-scale, no-bias run whose outputs are the accumulators rounded to
BF16, and exactly through the INT8 quant-out path with out_scale chosen so each code is one accumulator step).
MXFP8 (tests/ops/test_ops_cuda.py:608-637): relative L2 <= 1e-3 and max abs <= 1e-2 x output RMS vs the reference
(same E4M3 operands and scales, FP32 accumulation in another order)."""

import pytest
import torch
import torch.nn.functional as F

from flashim_amd import ops
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"

GEOMETRIES = [
    (64, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    (48, 40, 3, 3, 1, 1, 1, 1, 1, 1),  # Cin not a multiple of 32
    (16, 24, 3, 3, 1, 1, 1, 1, 1, 1),  # Cin < 32
    (64, 64, 1, 1, 1, 1, 0, 0, 1, 1),  # 1x1
    (32, 32, 3, 3, 2, 2, 1, 1, 1, 1),  # stride 2
    (32, 32, 3, 3, 1, 1, 2, 2, 2, 2),  # dilation 2
    (8, 16, 7, 7, 2, 2, 3, 3, 1, 1),  # 7x7 stride 2, Cin < 32
    (196, 128, 3, 3, 1, 1, 1, 1, 1, 1),  # Cin > 128, ragged chunk
    (512, 64, 3, 3, 1, 1, 1, 1, 1, 1),  # four 128-channel chunks per tap
    (96, 64, 5, 5, 1, 1, 2, 2, 1, 1),  # 5x5
    (6, 200, 3, 3, 1, 1, 1, 1, 1, 1),  # Cin % 4 != 0 (byte loads), Cout > 128
]


def _int8_inputs(cin, cout, kh, kw, has_bias, shape=(2, 17, 19)):
    torch.manual_seed(0)
    x = torch.randint(-127, 127, (*shape, cin), dtype=torch.int8)
    weight = torch.randint(-127, 127, (cout, kh * kw * cin), dtype=torch.int8)
    a_scale = torch.tensor(0.017)
    w_scale = torch.rand(cout) * 0.01 + 0.001
    bias = torch.randn(cout).to(torch.bfloat16) if has_bias else None
    return x, weight, a_scale, w_scale, bias


def _dev(*ts):
    return [t.to(DEV) if isinstance(t, torch.Tensor) else t for t in ts]


@pytest.mark.parametrize("cin,cout,kh,kw,sh,sw,ph,pw,dh,dw", GEOMETRIES)
@pytest.mark.parametrize("has_bias", [True, False])
def test_int8_conv2d_bit_exact(cin, cout, kh, kw, sh, sw, ph, pw, dh, dw, has_bias):
    x, weight, a_scale, w_scale, bias = _int8_inputs(cin, cout, kh, kw, has_bias)
    geo = (kh, kw, sh, sw, ph, pw, dh, dw)
    fast = ops.int8_conv2d.get("hip")(*_dev(x, weight, a_scale, w_scale, bias), *geo).cpu()
    want = ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo)
    assert fast.shape == want.shape and fast.dtype == torch.bfloat16
    assert torch.equal(fast, want)
    fused = ops.int8_conv2d.get("hip")(*_dev(x, weight, a_scale, w_scale, bias), *geo, relu=True).cpu()
    assert torch.equal(fused, F.relu(fast))


@pytest.mark.parametrize("cin,cout,kh,kw,sh,sw,ph,pw,dh,dw", GEOMETRIES[:6])
def test_int8_conv2d_accumulators_exact(cin, cout, kh, kw, sh, sw, ph, pw, dh, dw):
    """Unit scales and no bias make the INT8 quant-out code equal to the accumulator wherever |acc| <= 127: the
    device's int32 accumulators equal the oracle's int64 ones there; the oracle's equal F.conv2d in float64 everywhere."""
    torch.manual_seed(1)
    x = torch.randint(-8, 8, (2, 17, 19, cin), dtype=torch.int8)
    weight = torch.randint(-8, 8, (cout, kh * kw * cin), dtype=torch.int8)
    one, ones = torch.tensor(1.0), torch.ones(cout)
    geo = (kh, kw, sh, sw, ph, pw, dh, dw)
    acc = ref.int8_conv2d_accumulators(x, weight, *geo)
    got = ops.int8_conv2d.get("hip")(*_dev(x, weight, one, ones, None), *geo, out_scale=torch.tensor(1.0, device=DEV))
    small = acc.abs() <= 127
    want = ref.int8_conv2d(x, weight, one, ones, None, *geo, out_scale=torch.tensor(1.0))
    assert torch.equal(got.cpu(), want)
    assert torch.equal(got.cpu().long()[small], acc[small])
    # and the full-range accumulators through F.conv2d in float64 (exact for |acc| < 2^53)
    exact = F.conv2d(
        x.permute(0, 3, 1, 2).double(), weight.reshape(cout, kh, kw, cin).permute(0, 3, 1, 2).double(),
        stride=(sh, sw), padding=(ph, pw), dilation=(dh, dw),
    ).permute(0, 2, 3, 1).long()
    assert torch.equal(acc, exact)


def test_int8_conv2d_config1():
    """Config 1: N=1, 128x128, 64 -> 64, 3x3 pad 1; per-tensor activation scale, per-channel weights, fp32 bias."""
    torch.manual_seed(0)
    act = torch.randn(1, 64, 128, 128)
    a_scale = act.abs().amax() / 127
    x = ref.quantize_int8(act.permute(0, 2, 3, 1), a_scale)
    w = torch.randn(64, 64, 3, 3) * 0.05
    wm = w.permute(0, 2, 3, 1).reshape(64, -1)
    w_scale = ref.weight_scales(wm)
    wq = ref.quantize_symmetric(wm, w_scale[:, None])
    bias = torch.randn(64)
    geo = (3, 3, 1, 1, 1, 1, 1, 1)
    got = ops.int8_conv2d.get("hip")(*_dev(x, wq, a_scale, w_scale, bias), *geo).cpu()
    assert torch.equal(got, ref.int8_conv2d(x, wq, a_scale, w_scale, bias, *geo))


# small 3x3 stride-1 convs with Cin = 64 and an output width that is a multiple of 64 run on the one-load-phase
# row-segment kernel: images at the top and bottom and both side edges, two images, two to four N tiles of 32
# channels; the shapes stay below one 128-row tile per CU (256 CUs)
ROW3_CASES = [((1, 7, 64), 64), ((2, 5, 128), 64), ((1, 9, 192), 128), ((1, 128, 128), 64), ((1, 6, 64), 96)]


@pytest.mark.parametrize("case", range(len(ROW3_CASES)))
def test_int8_conv2d_row_segment_kernel(case):
    """Bit-exact BF16 out (bias, ReLU), with a residual, and INT8 out, against the oracle."""
    shape, cout = ROW3_CASES[case]
    geo = (3, 3, 1, 1, 1, 1, 1, 1)
    x, weight, a_scale, w_scale, bias = _int8_inputs(64, cout, 3, 3, True, shape=shape)
    args = _dev(x, weight, a_scale, w_scale, bias)
    hip = ops.int8_conv2d.get("hip")
    for relu in (False, True):
        got = hip(*args, *geo, relu=relu).cpu()
        assert torch.equal(got, ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, relu=relu)), (case, relu)
    res = (torch.randn(*shape, cout) * 4).to(torch.bfloat16)
    got_r = hip(*args, *geo, relu=True, residual=res.to(DEV)).cpu()
    assert torch.equal(got_r, ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, relu=True, residual=res)), case
    out_scale = torch.tensor(0.09)
    got_q = hip(*args, *geo, out_scale=out_scale.to(DEV)).cpu()
    assert torch.equal(got_q, ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, out_scale=out_scale)), case


@pytest.mark.parametrize("relu", [False, True])
@pytest.mark.parametrize("gelu", [False, True])
def test_int8_conv2d_epilogues(relu, gelu):
    x, weight, a_scale, w_scale, bias = _int8_inputs(64, 96, 3, 3, True)
    geo = (3, 3, 1, 1, 1, 1, 1, 1)
    residual = torch.randn(2, 17, 19, 80).to(torch.bfloat16)  # fewer channels than Cout
    out_scale = torch.tensor(0.05)
    for kwargs in ({}, {"residual": residual}, {"out_scale": out_scale}, {"residual": residual, "out_scale": out_scale}):
        got = ops.int8_conv2d.get("hip")(*_dev(x, weight, a_scale, w_scale, bias), *geo, relu=relu, gelu=gelu,
                                          **{k: v.to(DEV) for k, v in kwargs.items()}).cpu()
        want = ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, relu=relu, gelu=gelu, **kwargs)
        if gelu:  # GELU within one BF16 rounding (or 2^-12 in torch's cancelling tail); INT8 codes within one step
            diff = (got.float() - want.float()).abs()
            if got.dtype == torch.int8:
                assert diff.max() <= 1 and (got != want).float().mean() < 1e-3
            else:
                assert (diff <= want.float().abs() * 2**-7 + 2**-12).all()
        else:
            assert torch.equal(got, want), kwargs.keys()


def _mx_inputs(cin, cout, kh, kw, has_bias, seed=0):
    torch.manual_seed(seed)
    x = (torch.randn(2, 17, 19, cin) * 3).to(torch.float8_e4m3fn)
    channel_exponent = torch.randint(-6, 3, (cin // 32,), dtype=torch.int8)
    weight = (torch.randn(cout, kh * kw * cin) * 2).to(torch.float8_e4m3fn)
    weight_exponent = torch.randint(-9, -3, (cout, kh * kw * cin // 32), dtype=torch.int8)
    bias = torch.randn(cout).to(torch.bfloat16) if has_bias else None
    return x, channel_exponent, weight, weight_exponent, bias


def _assert_mx_close(fast, want):
    """Relative L2 <= 1e-3; per element |diff| <= max(1e-2 x output RMS, 2^-7 |want|). The second term is one BF16
    rounding step of the reference value: two FP32 accumulation orders flip the final BF16 rounding of some outputs,
    and at |y| > 2.56 x RMS that single flip alone exceeds 1e-2 x RMS."""
    fast, want = fast.float(), want.float()
    rms = want.pow(2).mean().sqrt()
    rel = (fast - want).norm() / want.norm()
    assert rel <= 1e-3, rel
    assert ((fast - want).abs() <= torch.maximum(1e-2 * rms, want.abs() * 2**-7)).all()


MX_GEOMETRIES = [
    (64, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    (224, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    (512, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    (96, 64, 5, 5, 1, 1, 2, 2, 1, 1),
    (64, 196, 3, 3, 2, 2, 1, 1, 1, 1),
    (32, 32, 3, 3, 1, 1, 2, 2, 2, 2),
    (128, 128, 1, 1, 1, 1, 0, 0, 1, 1),
]


@pytest.mark.parametrize("cin,cout,kh,kw,sh,sw,ph,pw,dh,dw", MX_GEOMETRIES)
@pytest.mark.parametrize("has_bias", [True, False])
def test_mxfp8_conv2d(cin, cout, kh, kw, sh, sw, ph, pw, dh, dw, has_bias):
    args = _mx_inputs(cin, cout, kh, kw, has_bias)
    geo = (kh, kw, sh, sw, ph, pw, dh, dw)
    fast = ops.mxfp8_conv2d.get("hip")(*_dev(*args), *geo).cpu()
    want = ref.mxfp8_conv2d(*args, *geo)
    assert fast.shape == want.shape and fast.dtype == torch.bfloat16
    _assert_mx_close(fast, want)
    fused = ops.mxfp8_conv2d.get("hip")(*_dev(*args), *geo, relu=True).cpu()
    assert torch.equal(fused, F.relu(fast))


def test_mxfp8_conv2d_matches_float64_conv():
    """Independent of the oracle: dequantized operands through F.conv2d in float64."""
    x, ce, w, we, bias = _mx_inputs(64, 96, 3, 3, True, seed=7)
    geo = (3, 3, 1, 1, 1, 1, 1, 1)
    fast = ops.mxfp8_conv2d.get("hip")(*_dev(x, ce, w, we, bias), *geo).cpu().double()
    xd = x.double() * torch.exp2(ce.double()).repeat_interleave(32)
    wd = (w.double() * torch.exp2(we.double()).repeat_interleave(32, dim=1)).reshape(96, 3, 3, 64).permute(0, 3, 1, 2)
    exact = F.conv2d(xd.permute(0, 3, 1, 2), wd, bias.double(), padding=1).permute(0, 2, 3, 1)
    magnitude = F.conv2d(xd.abs().permute(0, 3, 1, 2), wd.abs(), bias.double().abs(), padding=1).permute(0, 2, 3, 1)
    # one BF16 rounding of the exact value plus FP32 accumulation error (K = 576 terms)
    assert ((fast - exact).abs() <= exact.abs() * 2**-8 + magnitude * 2**-14).all()


@pytest.mark.parametrize("relu", [False, True])
@pytest.mark.parametrize("gelu", [False, True])
def test_mxfp8_conv2d_epilogues(relu, gelu):
    x, ce, w, we, bias = _mx_inputs(64, 96, 3, 3, True, seed=3)
    geo = (3, 3, 1, 1, 1, 1, 1, 1)
    residual = torch.randn(2, 17, 19, 80).to(torch.bfloat16)
    out_exponent = torch.tensor([-4, -3, -2], dtype=torch.int8)
    for kwargs in ({}, {"residual": residual}):
        got = ops.mxfp8_conv2d.get("hip")(*_dev(x, ce, w, we, bias), *geo, relu=relu, gelu=gelu,
                                           **{k: v.to(DEV) for k, v in kwargs.items()}).cpu()
        want = ref.mxfp8_conv2d(x, ce, w, we, bias, *geo, relu=relu, gelu=gelu, **kwargs)
        _assert_mx_close(got, want)
    # quant-out: the E4M3 codes of the BF16 result quantized with out_exponent (chained = separate quantize)
    got_bf16 = ops.mxfp8_conv2d.get("hip")(*_dev(x, ce, w, we, bias), *geo, relu=relu, gelu=gelu).cpu()
    got_q = ops.mxfp8_conv2d.get("hip")(*_dev(x, ce, w, we, bias), *geo, relu=relu, gelu=gelu,
                                         out_exponent=out_exponent.to(DEV)).cpu()
    assert torch.equal(got_q.view(torch.uint8), ref.quantize_static(got_bf16, out_exponent).view(torch.uint8))


def test_repeated_launches_identical():
    """Race guard (tests/ops/test_ops_cuda.py:81-97 style): repeated launches give the same bytes."""
    args = _dev(*_mx_inputs(128, 128, 3, 3, True))
    geo = (3, 3, 1, 1, 1, 1, 1, 1)
    first = ops.mxfp8_conv2d.get("hip")(*args, *geo)
    for _ in range(10):
        assert torch.equal(ops.mxfp8_conv2d.get("hip")(*args, *geo), first)
    iargs = _dev(*_int8_inputs(96, 200, 3, 3, True))
    ifirst = ops.int8_conv2d.get("hip")(*iargs, *geo)
    for _ in range(10):
        assert torch.equal(ops.int8_conv2d.get("hip")(*iargs, *geo), ifirst)


MAXPOOL = [
    ((2, 16, 20), 64, 64, (3, 3, 1, 1, 1, 1, 1, 1)),   # even Ho, Wo: pooled in the epilogue
    ((1, 34, 18), 48, 40, (3, 3, 1, 1, 1, 1, 1, 1)),   # Cout % 4 == 0 but not 64-aligned, Cin % 16 != 0
    ((2, 17, 19), 32, 96, (3, 3, 1, 1, 1, 1, 1, 1)),   # odd Ho, Wo: separate pool pass
    ((1, 40, 40), 16, 130, (3, 3, 2, 2, 1, 1, 1, 1)),  # stride 2, Cout > 128 and % 4 != 0
    ((3, 6, 10), 128, 64, (1, 1, 1, 1, 0, 0, 1, 1)),   # 1x1
]


@pytest.mark.parametrize("shape,cin,cout,geo", MAXPOOL)
@pytest.mark.parametrize("relu", [False, True])
def test_int8_conv2d_maxpool_bit_exact(shape, cin, cout, geo, relu):
    """ops/conv.py:209-222: the BF16 output equals int8_conv2d's and the pooled INT8 codes equal quantize_int8 of
    F.max_pool2d of it, bit for bit."""
    x, weight, a_scale, w_scale, bias = _int8_inputs(cin, cout, geo[0], geo[1], True, shape=shape)
    out_scale = torch.tensor(0.05)
    out, pooled = ops.int8_conv2d_maxpool.get("hip")(*_dev(x, weight, a_scale, w_scale, bias), *geo, relu=relu,
                                                     out_scale=out_scale.to(DEV))
    want_out, want_pooled = ref.int8_conv2d_maxpool(x, weight, a_scale, w_scale, bias, *geo, relu=relu,
                                                    out_scale=out_scale)
    assert out.shape == want_out.shape and pooled.shape == want_pooled.shape and pooled.dtype == torch.int8
    assert torch.equal(out.cpu(), want_out)
    assert torch.equal(pooled.cpu(), want_pooled)


@pytest.mark.parametrize("kind", ["int8", "mxfp8"])
def test_split_launch_tail(kind):
    """More tiles than two rounds of resident workgroups, the last round mostly empty: 1x1, 64 -> 192 channels on
    1 x 260 x 256 pixels = 520 M tiles x 2 N tiles = 1040 tiles on 512 slots (2 per CU on 256 CUs), so rows from 65536
    on run as a second launch of 64 x 64 tiles (3 N tiles). A 1x1 conv's rows are independent: every row must equal,
    bit for bit, the same rows from launches on 4-row slices of the image (too small to split; the same MFMA per
    16 x 16 block and the same epilogue). Plus the oracle bar (INT8 bit-exact; MXFP8 with GELU: relative L2)."""
    torch.manual_seed(11)
    geo = (1, 1, 1, 1, 0, 0, 1, 1)
    if kind == "int8":
        x = torch.randint(-127, 127, (1, 260, 256, 64), dtype=torch.int8)
        w = torch.randint(-127, 127, (192, 64), dtype=torch.int8)
        a_scale, w_scale = torch.tensor(0.013), torch.rand(192) * 0.01 + 0.001
        bias = torch.randn(192).to(torch.bfloat16)
        run = lambda xs: ops.int8_conv2d.get("hip")(*_dev(xs, w, a_scale, w_scale, bias), *geo, relu=True).cpu()  # noqa: E731
        got = run(x)
        assert torch.equal(got, ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo, relu=True))
    else:
        x = (torch.randn(1, 260, 256, 64) * 3).to(torch.float8_e4m3fn)
        ce = torch.randint(-6, 3, (2,), dtype=torch.int8)
        w = (torch.randn(192, 64) * 2).to(torch.float8_e4m3fn)
        we = torch.randint(-9, -3, (192, 2), dtype=torch.int8)
        bias = torch.randn(192).to(torch.bfloat16)
        run = lambda xs: ops.mxfp8_conv2d.get("hip")(*_dev(xs, ce, w, we, bias), *geo, gelu=True).cpu()  # noqa: E731
        got = run(x)
        want = ref.mxfp8_conv2d(x, ce, w, we, bias, *geo, gelu=True).float()
        assert (got.float() - want).norm() / want.norm() <= 1e-3
    for r0 in (0, 128, 254, 256):  # slices in the first launch, across the boundary row 65536 = 256 x 256, the tail
        sl = run(x[:, r0:r0 + 4].contiguous())
        assert torch.equal(got[:, r0:r0 + 4].view(torch.int16), sl.view(torch.int16)), r0


def _wide_cases():
    """Shapes whose tiles fill one round of one wide (8-wavefront) workgroup per CU, so launch_conv picks the wide
    kernel: 160 x 256 tiles for Cout 512 and 200 (the wavefront grid that pads Cout the least), 320 x 128 for
    Cout 128. M is not a multiple of the tile height; Cin 32 leaves 96 of each 128-byte K step empty; Cout 200 runs
    the general epilogue (Cout % 16 != 0) with a residual and quantized outputs, N tile 256 past Cout."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return [
        # (name, image (B, H, W), Cin, Cout, geometry, per-case kwargs)
        ("1x1_c512", (1, 64, (cus // 2) * 160 // 64 - 1), 256, 512, (1, 1, 1, 1, 0, 0, 1, 1), {}),
        ("3x3_c128", (1, 160, 2 * cus - 3), 32, 128, (3, 3, 1, 1, 1, 1, 1, 1), {}),
        ("3x3_c200_res", (1, 128, cus * 160 // 128 - 1), 64, 200, (3, 3, 1, 1, 2, 2, 2, 2), {"residual": True}),
    ]


@pytest.mark.parametrize("case", range(3))
def test_int8_conv2d_wide_tiles(case):
    """INT8 through the wide kernel: bit-exact with the oracle (BF16 out, then INT8 out for the residual case)."""
    name, shape, cin, cout, geo, kw = _wide_cases()[case]
    x, weight, a_scale, w_scale, bias = _int8_inputs(cin, cout, geo[0], geo[1], True, shape=shape)
    extra = {}
    if kw.get("residual"):
        extra["residual"] = (torch.randn(*shape[:3], cout) * 4).to(torch.bfloat16)
    args = _dev(x, weight, a_scale, w_scale, bias)
    got = ops.int8_conv2d.get("hip")(*args, *geo, relu=True, **{k: v.to(DEV) for k, v in extra.items()}).cpu()
    assert torch.equal(got, ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, relu=True, **extra)), name
    if extra:
        out_scale = torch.tensor(0.07)
        got_q = ops.int8_conv2d.get("hip")(*args, *geo, relu=True, residual=extra["residual"].to(DEV),
                                           out_scale=out_scale.to(DEV)).cpu()
        want_q = ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, relu=True, out_scale=out_scale, **extra)
        assert torch.equal(got_q, want_q), name


@pytest.mark.parametrize("case", range(3))
def test_mxfp8_conv2d_wide_tiles(case):
    """MXFP8 through the wide kernel, at sizes where one pre-activation BF16 flip (FP32 accumulation order) turns into
    two BF16 steps after GELU's slope, so the activation is checked on its own: the plain conv meets the oracle bar;
    GELU of it is torch's BF16 GELU of the same values within one BF16 step (2^-12 absolute in the cancelling tail);
    + residual is that GELU output plus the residual rounded once, bit for bit; the 1x1 case's rows equal, bit for bit,
    the same rows from small launches (4-row slices: another kernel, the same MFMA per 16 x 16 block and K step);
    E4M3 output equals the BF16 output quantized separately."""
    name, shape, cin, cout, geo, kw = _wide_cases()[case]
    torch.manual_seed(case + 20)
    x = (torch.randn(*shape, cin) * 3).to(torch.float8_e4m3fn)
    ce = torch.randint(-6, 3, (cin // 32,), dtype=torch.int8)
    w = (torch.randn(cout, geo[0] * geo[1] * cin) * 2).to(torch.float8_e4m3fn)
    we = torch.randint(-9, -3, (cout, geo[0] * geo[1] * cin // 32), dtype=torch.int8)
    bias = torch.randn(cout).to(torch.bfloat16)
    run = lambda xs, **k: ops.mxfp8_conv2d.get("hip")(*_dev(xs, ce, w, we, bias), *geo, **k).cpu()  # noqa: E731
    plain = run(x)
    _assert_mx_close(plain, ref.mxfp8_conv2d(x, ce, w, we, bias, *geo))
    got = run(x, gelu=True)
    want = F.gelu(plain).float()
    assert ((got.float() - want).abs() <= torch.clamp(want.abs() * 2**-7, min=2**-12)).all(), name
    if kw.get("residual"):
        r = torch.randn(*shape[:3], cout).to(torch.bfloat16)
        got_r = run(x, gelu=True, residual=r.to(DEV))
        assert torch.equal(got_r.view(torch.int16), (got.float() + r.float()).bfloat16().view(torch.int16)), name
        got = got_r
        extra = {"residual": r.to(DEV)}
    else:
        extra = {}
    if geo[0] == 1:
        for r0 in (0, 31, 60):
            sl = run(x[:, r0:r0 + 4].contiguous(), gelu=True)
            assert torch.equal(got[:, r0:r0 + 4].view(torch.int16), sl.view(torch.int16)), (name, r0)
    if cout % 32 == 0:  # E4M3 outputs take whole 32-channel scale blocks
        out_exponent = torch.randint(-3, 2, (cout // 32,), dtype=torch.int8)
        got_q = run(x, gelu=True, out_exponent=out_exponent.to(DEV), **extra)
        assert torch.equal(got_q.view(torch.uint8), ref.quantize_static(got, out_exponent).view(torch.uint8)), name


@pytest.mark.parametrize("kind", ["int8", "mxfp8"])
@pytest.mark.parametrize("gelu", [False, True])
@pytest.mark.parametrize("wide", [False, True])
def test_dense_residual_fast_epilogue(kind, gelu, wide):
    """A residual laid out as the output ([B, Ho, Wo, Cout] BF16, Cout % 16 == 0: the refiner blocks' contract convs)
    runs on the fast epilogue: INT8 without GELU bit-exact with the oracle (BF16 and INT8 out); otherwise bit-exact
    with relu(y + r) rounded once, y the same conv's output without the residual, y at the oracle bar (GELU: within one
    BF16 step). 128-row tiles, and a one-round launch of the wide kernel."""
    torch.manual_seed(31 + 2 * gelu + wide)
    if wide:
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        shape, cin, cout, geo = (1, 64, (cus // 2) * 160 // 64 - 1), 128, 512, (1, 1, 1, 1, 0, 0, 1, 1)
    else:
        shape, cin, cout, geo = (2, 17, 19), 64, 96, (3, 3, 1, 1, 1, 1, 1, 1)
    r = (torch.randn(*shape, cout) * 2).to(torch.bfloat16)
    if kind == "int8":
        x, w, a_scale, w_scale, bias = _int8_inputs(cin, cout, geo[0], geo[1], True, shape=shape)
        args = _dev(x, w, a_scale, w_scale, bias)
        run = lambda **k: ops.int8_conv2d.get("hip")(*args, *geo, gelu=gelu, **k).cpu()  # noqa: E731
        got = run(relu=True, residual=r.to(DEV))
        out_scale = torch.tensor(0.05)
        got_q = run(relu=True, residual=r.to(DEV), out_scale=out_scale.to(DEV))
        if not gelu:
            assert torch.equal(got, ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo, relu=True, residual=r))
            assert torch.equal(got_q, ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo, relu=True, residual=r,
                                                      out_scale=out_scale))
        else:  # this GELU is within one BF16 step of torch's: pin y there, the residual add by the exact identity
            y = run()
            want_y = ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo, gelu=True)
            assert ((y.float() - want_y.float()).abs() <= want_y.float().abs() * 2**-7 + 2**-12).all()
            assert torch.equal(got.view(torch.int16), torch.relu(y.float() + r.float()).bfloat16().view(torch.int16))
            assert torch.equal(got_q, ref.quantize_int8_static(got, out_scale))
    else:
        x = (torch.randn(*shape, cin) * 3).to(torch.float8_e4m3fn)
        ce = torch.randint(-6, 3, (cin // 32,), dtype=torch.int8)
        w = (torch.randn(cout, geo[0] * geo[1] * cin) * 2).to(torch.float8_e4m3fn)
        we = torch.randint(-9, -3, (cout, geo[0] * geo[1] * cin // 32), dtype=torch.int8)
        bias = torch.randn(cout).to(torch.bfloat16)
        run = lambda **k: ops.mxfp8_conv2d.get("hip")(*_dev(x, ce, w, we, bias), *geo, gelu=gelu, **k).cpu()  # noqa: E731
        plain = run()
        got = run(relu=True, residual=r.to(DEV))
        want = torch.relu(plain.float() + r.float()).bfloat16()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        if not gelu:  # y itself at the oracle bar (a cancelling residual would turn one FP32-order flip of y into
            # more than the bar's relative term of the small sum: the identity above pins the residual add)
            _assert_mx_close(plain, ref.mxfp8_conv2d(x, ce, w, we, bias, *geo))
        out_exponent = torch.randint(-3, 2, (cout // 32,), dtype=torch.int8)
        got_q = run(relu=True, residual=r.to(DEV), out_exponent=out_exponent.to(DEV))
        assert torch.equal(got_q.view(torch.uint8), ref.quantize_static(got, out_exponent).view(torch.uint8))


@pytest.mark.parametrize("kind", ["int8", "mxfp8"])
def test_single_k_step_kernel_quantized_outputs(kind):
    """1x1 convs with K = 128 over many rounds run the single-K-step 128-row kernel (one LDS stage, three workgroups
    per CU): INT8 bit-exact with the oracle (BF16 and INT8 out), MXFP8 at the oracle bar and its E4M3 output equal to
    the BF16 output quantized separately."""
    torch.manual_seed(41)
    shape, geo = (1, 300, 256), (1, 1, 1, 1, 0, 0, 1, 1)
    if kind == "int8":
        x, w, a_scale, w_scale, bias = _int8_inputs(128, 128, 1, 1, True, shape=shape)
        args = _dev(x, w, a_scale, w_scale, bias)
        out_scale = torch.tensor(0.04)
        got = ops.int8_conv2d.get("hip")(*args, *geo, relu=True).cpu()
        assert torch.equal(got, ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo, relu=True))
        got_q = ops.int8_conv2d.get("hip")(*args, *geo, relu=True, out_scale=out_scale.to(DEV)).cpu()
        assert torch.equal(got_q, ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo, relu=True, out_scale=out_scale))
    else:
        x = (torch.randn(*shape, 128) * 3).to(torch.float8_e4m3fn)
        ce = torch.randint(-6, 3, (4,), dtype=torch.int8)
        w = (torch.randn(128, 128) * 2).to(torch.float8_e4m3fn)
        we = torch.randint(-9, -3, (128, 4), dtype=torch.int8)
        bias = torch.randn(128).to(torch.bfloat16)
        run = lambda **k: ops.mxfp8_conv2d.get("hip")(*_dev(x, ce, w, we, bias), *geo, relu=True, **k).cpu()  # noqa: E731
        got = run()
        _assert_mx_close(got, ref.mxfp8_conv2d(x, ce, w, we, bias, *geo, relu=True))
        out_exponent = torch.tensor([-2, -1, 0, 1], dtype=torch.int8)
        got_q = run(out_exponent=out_exponent.to(DEV))
        assert torch.equal(got_q.view(torch.uint8), ref.quantize_static(got, out_exponent).view(torch.uint8))


# (name, image (B, H, W), Cin, Cout, geometry): shapes the patch-tile kernel takes (3 x 3, stride 1, dilation 1,
# Cin == 128): partial tiles at the image edges, a partial channel block, several channel blocks and images (the
# workgroups walk several tiles each), padding 0 and 2
PATCH_CASES = [
    ("3x3_edges", (1, 37, 45), 128, 128, (3, 3, 1, 1, 1, 1, 1, 1)),
    ("3x3_n96_b2", (2, 19, 50), 128, 96, (3, 3, 1, 1, 1, 1, 1, 1)),
    ("3x3_pad0", (1, 33, 41), 128, 48, (3, 3, 1, 1, 0, 0, 1, 1)),
    ("3x3_n256_many_tiles", (3, 64, 120), 128, 256, (3, 3, 1, 1, 1, 1, 1, 1)),
    ("3x3_pad2", (1, 20, 30), 128, 64, (3, 3, 1, 1, 2, 2, 1, 1)),
    # larger images: several tiles per workgroup and group (partial tiles at both image edges, a partial channel
    # block, padding 0)
    ("3x3_wg_tiles", (2, 150, 170), 128, 128, (3, 3, 1, 1, 1, 1, 1, 1)),
    ("3x3_wg_tiles_n96", (3, 120, 130), 128, 96, (3, 3, 1, 1, 1, 1, 1, 1)),
    ("3x3_wg_tiles_pad0", (3, 130, 140), 128, 128, (3, 3, 1, 1, 0, 0, 1, 1)),
]


@pytest.mark.parametrize("case", range(len(PATCH_CASES)))
def test_int8_conv2d_patch_tiles(case):
    """INT8 through the patch-tile kernel: bit-exact BF16 out (bias + ReLU), with a dense residual, and INT8 out."""
    name, shape, cin, cout, geo = PATCH_CASES[case]
    x, weight, a_scale, w_scale, bias = _int8_inputs(cin, cout, geo[0], geo[1], True, shape=shape)
    args = _dev(x, weight, a_scale, w_scale, bias)
    hip = ops.int8_conv2d.get("hip")
    got = hip(*args, *geo, relu=True).cpu()
    want = ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, relu=True)
    assert torch.equal(got, want), name
    res = (torch.randn(*want.shape) * 4).to(torch.bfloat16)
    got_r = hip(*args, *geo, relu=True, residual=res.to(DEV)).cpu()
    assert torch.equal(got_r, ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, relu=True, residual=res)), name
    out_scale = torch.tensor(0.09)
    got_q = hip(*args, *geo, out_scale=out_scale.to(DEV)).cpu()
    assert torch.equal(got_q, ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *geo, out_scale=out_scale)), name


@pytest.mark.parametrize("case", range(len(PATCH_CASES)))
def test_mxfp8_conv2d_patch_tiles(case):
    """MXFP8 through the patch-tile kernel: the oracle bar (plain, GELU within one BF16 step), and the E4M3 output
    byte-identical to quantizing the kernel's own BF16 output."""
    name, shape, cin, cout, geo = PATCH_CASES[case]
    torch.manual_seed(case)
    x = (torch.randn(*shape, cin) * 3).to(torch.float8_e4m3fn)
    ce = torch.randint(-6, 3, (cin // 32,), dtype=torch.int8)
    w = (torch.randn(cout, geo[0] * geo[1] * cin) * 2).to(torch.float8_e4m3fn)
    we = torch.randint(-10, -4, (cout, geo[0] * geo[1] * cin // 32), dtype=torch.int8)
    bias = torch.randn(cout).to(torch.bfloat16)
    hip = ops.mxfp8_conv2d.get("hip")
    args = _dev(x, ce, w, we, bias)
    got = hip(*args, *geo).cpu()
    want = ref.mxfp8_conv2d(x, ce, w, we, bias, *geo)
    _assert_mx_close(got, want)
    got_g = hip(*args, *geo, gelu=True).cpu().float()
    want_g = ref.mxfp8_conv2d(x, ce, w, we, bias, *geo, gelu=True).float()
    assert (got_g - want_g).norm() / want_g.norm() <= 1e-3, name
    if cout % 32 == 0:
        oe = torch.full((cout // 32,), -1, dtype=torch.int8)
        got_q = hip(*args, *geo, out_exponent=oe.to(DEV))
        assert torch.equal(got_q.view(torch.uint8), ops.quantize_mxfp8(hip(*args, *geo), oe.to(DEV)).values
                           .view(torch.uint8)), name


# (name, image (B, H, W), Cin, Cout): pointwise shapes (1 x 1, stride 1, Cin a multiple of 128 up to 512 or 1024,
# Cout >= 128): 1 to 4 and 8 K steps, a partial last tile of pixels, a partial channel block; the large ones run the
# register-operand pointwise kernel (at 8 K steps in two load phases, its output staged in 64-channel half rows), the
# "resident" ones (one to two 160-pixel tiles per CU on 256 CUs) the whole-K kernel, the small ones the one-round
# kernels
ROW_CASES = [
    ("k1_n128_resident", (2, 150, 151), 128, 128),
    ("k2_n144_resident", (2, 110, 111), 256, 144),
    ("k3_n256_resident", (1, 150, 151), 384, 256),
    ("k4_n512_resident", (2, 100, 101), 512, 512),
    # a resident-sized shape whose Cout % 16 != 0 needs the general epilogue: it takes the other kernels
    ("k2_n136_resident_size_general", (2, 110, 111), 256, 136),
    ("k1_partial_tile", (1, 7, 13), 128, 128),
    ("k2_n144", (2, 9, 11), 256, 144),
    ("k3_n256", (1, 30, 31), 384, 256),
    ("k4_n512_many", (2, 60, 70), 512, 512),
    # at least two 256-pixel tiles per CU (the kernel's condition on 256 CUs)
    ("k1_n128_big", (2, 256, 257), 128, 128),
    ("k2_n144_big", (1, 256, 257), 256, 144),
    ("k3_n256_big", (2, 160, 210), 384, 256),
    ("k4_n512_big", (2, 128, 129), 512, 512),
    # the refiner stack's s = 4 contract (1024 -> 256), and a partial channel block at 8 K steps
    ("k8_n256_big", (2, 200, 200), 1024, 256),
    ("k8_n144_big", (1, 256, 257), 1024, 144),
    ("k8_n256", (1, 30, 31), 1024, 256),
]
PW_GEO = (1, 1, 1, 1, 0, 0, 1, 1)


@pytest.mark.parametrize("case", range(len(ROW_CASES)))
def test_int8_conv2d_pointwise_tiles(case):
    """INT8 through the pointwise kernel: bit-exact BF16 out (bias + ReLU), with a dense residual, and INT8 out."""
    name, shape, cin, cout = ROW_CASES[case]
    x, weight, a_scale, w_scale, bias = _int8_inputs(cin, cout, 1, 1, True, shape=shape)
    args = _dev(x, weight, a_scale, w_scale, bias)
    hip = ops.int8_conv2d.get("hip")
    got = hip(*args, *PW_GEO, relu=True).cpu()
    want = ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *PW_GEO, relu=True)
    assert torch.equal(got, want), name
    res = (torch.randn(*want.shape) * 4).to(torch.bfloat16)
    got_r = hip(*args, *PW_GEO, relu=True, residual=res.to(DEV)).cpu()
    assert torch.equal(got_r, ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *PW_GEO, relu=True, residual=res)), name
    out_scale = torch.tensor(0.09)
    got_q = hip(*args, *PW_GEO, out_scale=out_scale.to(DEV)).cpu()
    assert torch.equal(got_q, ref.int8_conv2d(x, weight, a_scale, w_scale, bias, *PW_GEO, out_scale=out_scale)), name


@pytest.mark.parametrize("case", range(len(ROW_CASES)))
def test_mxfp8_conv2d_pointwise_tiles(case):
    """MXFP8 through the pointwise kernel: the oracle bar (plain; GELU; GELU with a residual), and the E4M3 output
    byte-identical to quantizing the kernel's own BF16 output."""
    name, shape, cin, cout = ROW_CASES[case]
    torch.manual_seed(100 + case)
    x = (torch.randn(*shape, cin) * 3).to(torch.float8_e4m3fn)
    ce = torch.randint(-6, 3, (cin // 32,), dtype=torch.int8)
    w = (torch.randn(cout, cin) * 2).to(torch.float8_e4m3fn)
    we = torch.randint(-10, -4, (cout, cin // 32), dtype=torch.int8)
    bias = torch.randn(cout).to(torch.bfloat16)
    hip = ops.mxfp8_conv2d.get("hip")
    args = _dev(x, ce, w, we, bias)
    got = hip(*args, *PW_GEO).cpu()
    want = ref.mxfp8_conv2d(x, ce, w, we, bias, *PW_GEO)
    _assert_mx_close(got, want)
    got_g = hip(*args, *PW_GEO, gelu=True).cpu().float()
    want_g = ref.mxfp8_conv2d(x, ce, w, we, bias, *PW_GEO, gelu=True).float()
    assert (got_g - want_g).norm() / want_g.norm() <= 1e-3, name
    res = (torch.randn(*want.shape) * 2).to(torch.bfloat16)
    got_r = hip(*args, *PW_GEO, gelu=True, residual=res.to(DEV)).cpu().float()
    want_r = ref.mxfp8_conv2d(x, ce, w, we, bias, *PW_GEO, gelu=True, residual=res).float()
    assert (got_r - want_r).norm() / want_r.norm() <= 1e-3, name
    if cout % 32 == 0:
        oe = torch.full((cout // 32,), -1, dtype=torch.int8)
        got_q = hip(*args, *PW_GEO, out_exponent=oe.to(DEV))
        assert torch.equal(got_q.view(torch.uint8), ops.quantize_mxfp8(hip(*args, *PW_GEO), oe.to(DEV)).values
                           .view(torch.uint8)), name
