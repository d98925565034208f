"""Every BASELINE config at its full workload, on the inputs ``bench.py`` times, against the oracle.

* config 1 (INT8 3x3, 1x128x128, 64 -> 64): bit-exact BF16 output.
* config 2 (MXFP8 1x1, 2x100x100, 512 -> 512, outlier channels, bias + GELU): the plain conv at the MXFP8 bar (relative
  L2 <= 1e-3; per element within max(1e-2 x output RMS, one BF16 rounding of the reference)), then the GELU output within
  that bar plus GELU's own one-BF16-step agreement (2^-7 |ref| + 2^-12). Also the same layer at Cin 640 (five 128-byte K
  steps: the wide kernel's three-stage ring wraps and ends on a partial tail) and INT8 bit-exact at Cin 512 / 640.
* config 3 (MXFP8 3x3, 2x200x200, 128 -> 128, folded BN + ReLU): the conv at the MXFP8 bar; its quantizer byte-exact.
* config 4 (refiner block, 2x400x400, C = 64), both presets, stage by stage on the GPU's own intermediate codes:
  depthwise + GELU codes within one code step (at most 0.5% differ), the expand conv's quantized hidden codes the same
  way, the contract conv + residual at the MXFP8 bar (INT8: bit-exact), the fused MLP launch bit-identical to the two
  conv launches, and the block end to end within relative L2 1e-2 (MXFP8) / 2e-2 (INT8): three quantization steps
  compound there, which the per-stage bars bound one at a time.
* config 5 (refiner stack): one block per stack scale at its true width and pixel count (512 @ 52768, 256 @ 211072,
  128 @ 844288, 64 @ 3377152 pixels), both presets, end to end within the config-4 bars; and the first two blocks of
  the coarsest scale chained.

The oracle runs on the host CPU (torch, at most 16 threads) on the same seeded inputs."""

import os

import pytest
import torch
import torch.nn.functional as F

import bench
from flashim_amd import blocks, ops, quant
from flashim_amd.backends.hip import gemm as hip_gemm
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
ONE = (1, 1, 1, 1, 0, 0, 1, 1)


@pytest.fixture(scope="module", autouse=True)
def _cpu_threads():
    before = torch.get_num_threads()
    torch.set_num_threads(min(os.cpu_count() or 1, 16))
    yield
    torch.set_num_threads(before)


def _cpu(args):
    return [a.cpu() if isinstance(a, torch.Tensor) else a for a in args]


def _assert_mx_close(got, want, pre=None):
    """The MXFP8 bar. With a residual, ``pre`` is the oracle's conv output before the residual add: a different FP32
    accumulation order may flip that value's BF16 rounding, and the one-step change can then flip the rounding of the
    sum too (one BF16 step of the output)."""
    got, want = got.float(), want.float()
    rms = want.pow(2).mean().sqrt()
    rel = ((got - want).norm() / want.norm()).item()
    assert rel <= 1e-3, rel
    if pre is None:
        bound = torch.maximum(1e-2 * rms, want.abs() * 2**-7)
    else:
        bound = torch.maximum(1e-2 * rms, pre.float().abs() * 2**-7) + want.abs() * 2**-7
    worst = ((got - want).abs() - bound).max().item()
    assert worst <= 0, worst


def _e4m3_step(v):
    return torch.exp2(torch.floor(torch.log2(v.abs().clamp_min(2.0**-6))) - 3)


def _assert_codes_close(got, want, scale, frac=5e-3):
    """Dequantized codes within one code step (or 2^-12 unscaled), at most ``frac`` of them different."""
    if got.dtype == torch.int8:
        assert (got.int() - want.int()).abs().max() <= 1
    else:
        g, w = got.float(), want.float()
        assert ((g - w).abs() * scale <= torch.maximum(_e4m3_step(w) * scale, torch.full_like(w, 2.0**-12))).all()
    mism = (got.view(torch.uint8) != want.view(torch.uint8)).float().mean().item()
    assert mism <= frac, mism


def test_config1_full_size_bit_exact():
    fn, _, args = bench.cfg1()
    got = fn().cpu()
    assert torch.equal(got, ref.int8_conv2d(*_cpu(args)))


def test_config2_full_size():
    fn, _, args = bench.cfg2()
    cargs = _cpu(args)
    plain = ops.mxfp8_conv2d(*args).cpu()
    want_plain = ref.mxfp8_conv2d(*cargs)
    assert plain.shape == (2, 100, 100, 512)
    _assert_mx_close(plain, want_plain)
    got = fn().cpu()
    want = ref.mxfp8_conv2d(*cargs, gelu=True)
    rel = ((got.float() - want.float()).norm() / want.float().norm()).item()
    assert rel <= 1e-3, rel
    rms = want.float().pow(2).mean().sqrt()
    bound = torch.maximum(1e-2 * rms, want.float().abs() * 2**-7) + want.float().abs() * 2**-7 + 2**-12
    assert ((got.float() - want.float()).abs() <= bound).all()


@pytest.mark.parametrize("cin", [512, 640])
def test_config2_layer_four_and_five_k_steps(cin):
    """The config-2 layer shape with four 128-byte K steps (the whole-K pointwise kernel) and five (the wide
    three-stage kernel, its ring of stages wrapping with a partial tail)."""
    g = torch.Generator().manual_seed(cin)
    x_bf16 = (torch.randn(2, 100, 100, cin, generator=g) * 2).to(torch.bfloat16)
    e = ref.calibrate_block32_exponent(x_bf16.float())
    xq = ref.quantize_mxfp8(x_bf16, e)
    wv, we = ref.quantized_weight_from_float(torch.randn(512, cin, generator=g) * 0.05)
    bias = (torch.randn(512, generator=g) * 0.1).to(torch.bfloat16)
    got = ops.mxfp8_conv2d(xq.to(DEV), e.to(DEV), wv.to(DEV), we.to(DEV), bias.to(DEV), *ONE).cpu()
    _assert_mx_close(got, ref.mxfp8_conv2d(xq, e, wv, we, bias, *ONE))
    x8 = torch.randint(-127, 128, (2, 100, 100, cin), dtype=torch.int8, generator=g)
    w8 = torch.randint(-127, 128, (512, cin), dtype=torch.int8, generator=g)
    a_s, w_s = torch.tensor(0.011), torch.rand(512, generator=g) * 0.01
    got8 = ops.int8_conv2d(x8.to(DEV), w8.to(DEV), a_s.to(DEV), w_s.to(DEV), bias.to(DEV), *ONE, gelu=True).cpu()
    want8 = ref.int8_conv2d(x8, w8, a_s, w_s, bias, *ONE, gelu=True)
    plain8 = ops.int8_conv2d(x8.to(DEV), w8.to(DEV), a_s.to(DEV), w_s.to(DEV), bias.to(DEV), *ONE).cpu()
    assert torch.equal(plain8, ref.int8_conv2d(x8, w8, a_s, w_s, bias, *ONE))
    diff = (got8.float() - want8.float()).abs()
    assert (diff <= want8.float().abs() * 2**-7 + 2**-12).all()


def test_config3_full_size():
    (conv, _, args), (qfn, _, (x_bf16, exponent)) = bench.cfg3()
    q = qfn()
    assert torch.equal(q.values.cpu().view(torch.uint8),
                       ref.quantize_mxfp8(x_bf16.cpu(), exponent.cpu()).view(torch.uint8))
    got = conv().cpu()
    want = ref.mxfp8_conv2d(*_cpu(args), relu=True)
    assert got.shape == (2, 200, 200, 128)
    _assert_mx_close(got, want)


def _block_stages(block: blocks.RefinerBlock, x: torch.Tensor):
    """Stage by stage: GPU codes vs oracle codes from the same inputs, and the next stage fed with the GPU's codes."""
    b, h, w, c = x.shape
    xn_dev = x.permute(0, 3, 1, 2)
    xn = xn_dev.cpu()
    dw_w, dw_b = block.dw_weight, block.dw_bias
    if block.preset == "mxfp8":
        e1, e2 = block.in_scale, block.hidden_scale
        q1 = ops.depthwise5x5_gelu(xn_dev, dw_w, dw_b, exponent=e1)
        want1 = ref.depthwise5x5_gelu(xn, dw_w.cpu(), dw_b.cpu(), exponent=e1.cpu())
        _assert_codes_close(q1.cpu(), want1, torch.exp2(e1.cpu().float()).repeat_interleave(32))
        q1 = q1.view(b, h, w, c)
        w1, w2 = block.w1, block.w2
        q2 = ops.mxfp8_conv2d(q1, e1, w1.values, w1.scale_exponent, block.b1, *ONE, gelu=True, out_exponent=e2)
        want2 = ref.mxfp8_conv2d(q1.cpu(), e1.cpu(), w1.values.cpu(), w1.scale_exponent.cpu(), block.b1.cpu(), *ONE,
                                 gelu=True, out_exponent=e2.cpu())
        _assert_codes_close(q2.cpu(), want2, torch.exp2(e2.cpu().float()).repeat_interleave(32))
        out = ops.mxfp8_conv2d(q2, e2, w2.values, w2.scale_exponent, block.b2, *ONE, residual=x)
        args3 = (q2.cpu(), e2.cpu(), w2.values.cpu(), w2.scale_exponent.cpu(), block.b2.cpu(), *ONE)
        _assert_mx_close(out.cpu(), ref.mxfp8_conv2d(*args3, residual=x.cpu()), pre=ref.mxfp8_conv2d(*args3))
        if c == hip_gemm.MLP_CHANNELS:
            fused = hip_gemm.refiner_mlp(q1, e1, w1.values, w1.scale_exponent, block.b1, e2, w2.values,
                                         w2.scale_exponent, block.b2, x)
            assert torch.equal(fused.view(torch.int16), out.view(torch.int16))
    else:
        s1, s2 = block.in_scale, block.hidden_scale
        q1 = ops.depthwise5x5_gelu(xn_dev, dw_w, dw_b, scale=s1)
        _assert_codes_close(q1.cpu(), ref.depthwise5x5_gelu(xn, dw_w.cpu(), dw_b.cpu(), scale=s1.cpu()), None)
        q1 = q1.view(b, h, w, c)
        q2 = ops.int8_conv2d(q1, block.w1_q, s1, block.w1_s, block.b1, *ONE, gelu=True, out_scale=s2)
        want2 = ref.int8_conv2d(q1.cpu(), block.w1_q.cpu(), s1.cpu(), block.w1_s.cpu(), block.b1.cpu(), *ONE,
                                gelu=True, out_scale=s2.cpu())
        _assert_codes_close(q2.cpu(), want2, None)
        out = ops.int8_conv2d(q2, block.w2_q, s2, block.w2_s, block.b2, *ONE, residual=x)
        want3 = ref.int8_conv2d(q2.cpu(), block.w2_q.cpu(), s2.cpu(), block.w2_s.cpu(), block.b2.cpu(), *ONE,
                                residual=x.cpu())
        assert torch.equal(out.cpu(), want3)
        if c == hip_gemm.MLP_CHANNELS:
            fused = hip_gemm.refiner_mlp(q1, s1, block.w1_q, block.w1_s, block.b1, s2, block.w2_q, block.w2_s,
                                         block.b2, x)
            assert torch.equal(fused.view(torch.int16), out.view(torch.int16))


def _oracle_block(block: blocks.RefinerBlock, x: torch.Tensor) -> torch.Tensor:
    b, h, w, c = x.shape
    xn = x.permute(0, 3, 1, 2)
    dw_w, dw_b = block.dw_weight.cpu(), block.dw_bias.cpu()
    if block.preset == "mxfp8":
        e1, e2 = block.in_scale.cpu(), block.hidden_scale.cpu()
        q1 = ref.depthwise5x5_gelu(xn, dw_w, dw_b, exponent=e1).view(b, h, w, c)
        q2 = ref.mxfp8_conv2d(q1, e1, block.w1.values.cpu(), block.w1.scale_exponent.cpu(), block.b1.cpu(), *ONE,
                              gelu=True, out_exponent=e2)
        return ref.mxfp8_conv2d(q2, e2, block.w2.values.cpu(), block.w2.scale_exponent.cpu(), block.b2.cpu(), *ONE,
                                residual=x)
    s1, s2 = block.in_scale.cpu(), block.hidden_scale.cpu()
    q1 = ref.depthwise5x5_gelu(xn, dw_w, dw_b, scale=s1).view(b, h, w, c)
    q2 = ref.int8_conv2d(q1, block.w1_q.cpu(), s1, block.w1_s.cpu(), block.b1.cpu(), *ONE, gelu=True, out_scale=s2)
    return ref.int8_conv2d(q2, block.w2_q.cpu(), s2, block.w2_s.cpu(), block.b2.cpu(), *ONE, residual=x)


TOL = {"mxfp8": 1e-2, "int8": 2e-2}


@pytest.mark.parametrize("preset", ["mxfp8", "int8"])
def test_config4_block_full_size(preset):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 400, 400, 64, generator=g).to(torch.bfloat16).to(DEV)
    block = blocks.RefinerBlock(blocks.BlockWeights.random(64, g, DEV), preset).calibrate(x)
    _block_stages(block, x)
    got = block(x).cpu().float()
    want = _oracle_block(block, x.cpu()).float()
    rel = ((got - want).norm() / want.norm()).item()
    assert rel <= TOL[preset], rel


@pytest.mark.parametrize("preset", ["mxfp8", "int8"])
@pytest.mark.parametrize("scale_index", range(len(blocks.STACK_SCALES)))
def test_config5_stack_scale_block_full_size(preset, scale_index):
    """One block at stack scale ``scale_index``'s width on its pixel count (both images of the scale stacked as the
    stack runs them: batch 2 of (800/s)^2 and batch 2 of (1024/s)^2)."""
    stride, channels = blocks.STACK_SCALES[scale_index]
    g = torch.Generator().manual_seed(50 + scale_index)
    xs = [torch.randn(2, size // stride, size // stride, channels, generator=g).to(torch.bfloat16).to(DEV)
          for size in blocks.STACK_SIZES]
    pixels = sum(x.shape[0] * x.shape[1] * x.shape[2] for x in xs)
    assert pixels == 2 * ((800 // stride) ** 2 + (1024 // stride) ** 2)
    block = blocks.RefinerBlock(blocks.BlockWeights.random(channels, g, DEV), preset).calibrate(xs[0])
    for x in xs:
        if scale_index == len(blocks.STACK_SCALES) - 1 or x is xs[0]:
            _block_stages(block, x)
        got = block(x).cpu().float()
        want = _oracle_block(block, x.cpu()).float()
        rel = ((got - want).norm() / want.norm()).item()
        assert rel <= TOL[preset], (x.shape, rel)


@pytest.mark.parametrize("preset", ["mxfp8", "int8"])
def test_config5_stack_chained_blocks(preset):
    """The stack's own construction (blocks.build_stack), its coarsest scale's first two blocks chained."""
    scales = blocks.build_stack(preset, DEV)
    inputs, stack_blocks = scales[0]
    x = inputs[1]
    got, want = x, x.cpu()
    for block in stack_blocks[:2]:
        got = block(got)
        want = _oracle_block(block, want)
    rel = ((got.cpu().float() - want.float()).norm() / want.float().norm()).item()
    assert rel <= 2 * TOL[preset], rel
