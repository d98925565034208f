"""The conv-refiner block of BASELINE configs 4-5 and a stack of them, composed from this package's ops.

Block (channels ``C``, hidden ``4C``), the depthwise-then-pointwise structure of FlashIM's refiners
(``flashim/layers/conv.py:62-87``, ``flashim/quant/passes/separable_conv_block.py``) with an expand/contract MLP:

1. depthwise 5x5 (pad 2) + folded BatchNorm (``fold_block_batchnorm``, separable_conv_block.py:58-66) -> BF16;
2. GELU -> the expand conv's static input quantize      (``ops.depthwise5x5_gelu``, one kernel);
3. 1x1 expand C -> 4C, bias, GELU -> the contract conv's static input quantize  (``mxfp8_conv2d`` / ``int8_conv2d``
   with ``gelu=True`` and the chained quant-out epilogue, quant/methods/conv2d.py:102-125, 207-251);
4. 1x1 contract 4C -> C, bias, + residual (the block input) -> BF16 (the residual epilogue, ops/conv.py:198-203).

At C = 64, steps 3-4 run as one fused launch (``refiner_mlp``: the quantized hidden layer never leaves LDS), computing
exactly what the two conv launches compute.

Presets: ``"mxfp8"`` (E4M3, static per-32-channel exponents, per-(row, 32) weight exponents) and ``"int8"`` (per-tensor
static activation scales, per-output-channel weights). Activations are NHWC BF16 ``[B, H, W, C]`` between blocks.
Static activation scales come from one calibration pass over a sample input (what FlashIM's calibration tables hold).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from flashim_amd import ops, quant
from flashim_amd.backends.hip import gemm as _gemm

BN_EPS = 1e-5


@dataclass
class BlockWeights:
    """Float parameters of one block (what a checkpoint holds), on the device."""

    dw_weight: Tensor  # [C, 1, 5, 5]
    dw_bias: Tensor  # [C]
    bn_gamma: Tensor
    bn_beta: Tensor
    bn_mean: Tensor
    bn_var: Tensor
    w1: Tensor  # [4C, C]
    b1: Tensor  # [4C]
    w2: Tensor  # [C, 4C]
    b2: Tensor  # [C]

    @classmethod
    def random(cls, channels: int, generator: torch.Generator, device) -> BlockWeights:
        c, h = channels, 4 * channels

        def r(*shape, scale=1.0):
            return (torch.randn(*shape, generator=generator) * scale).to(device)

        return cls(
            dw_weight=r(c, 1, 5, 5, scale=0.2), dw_bias=r(c, scale=0.1),
            bn_gamma=(torch.rand(c, generator=generator) + 0.5).to(device), bn_beta=r(c, scale=0.1),
            bn_mean=r(c, scale=0.1), bn_var=(torch.rand(c, generator=generator) + 0.5).to(device),
            w1=r(h, c, scale=c ** -0.5), b1=r(h, scale=0.1), w2=r(c, h, scale=h ** -0.5), b2=r(c, scale=0.1),
        )

    def folded_depthwise(self) -> tuple[Tensor, Tensor]:
        """BatchNorm folded into the depthwise conv (``nn.utils.fusion.fuse_conv_bn_eval`` arithmetic), packed
        ``[25, C]`` BF16 (ky, kx major) and FP32 bias."""
        inv = self.bn_gamma / torch.sqrt(self.bn_var + BN_EPS)
        weight = self.dw_weight * inv[:, None, None, None]
        bias = (self.dw_bias - self.bn_mean) * inv + self.bn_beta
        channels = weight.shape[0]
        packed = weight[:, 0].permute(1, 2, 0).reshape(25, channels).to(torch.bfloat16).contiguous()
        return packed, bias.float().contiguous()


class RefinerBlock:
    """One packed block; ``forward(x)`` with ``x`` NHWC BF16 ``[B, H, W, C]``."""

    def __init__(self, weights: BlockWeights, preset: str) -> None:
        if preset not in ("mxfp8", "int8"):
            raise ValueError(f"unknown preset {preset!r}")
        self.preset = preset
        self.channels = weights.w2.shape[0]
        self.dw_weight, self.dw_bias = weights.folded_depthwise()
        self.b1 = weights.b1.to(torch.bfloat16).contiguous()
        self.b2 = weights.b2.to(torch.bfloat16).contiguous()
        if preset == "mxfp8":
            self.w1 = quant.QuantizedWeight.from_float(weights.w1)
            self.w2 = quant.QuantizedWeight.from_float(weights.w2)
        else:
            self.w1_q, self.w1_s = quant.weight_scales_and_values(weights.w1)
            self.w2_q, self.w2_s = quant.weight_scales_and_values(weights.w2)
        self.in_scale = None  # expand input: [C/32] exponents or an FP32 scale
        self.hidden_scale = None  # contract input

    # -- calibration ------------------------------------------------------------------------------------------

    def calibrate(self, x: Tensor) -> RefinerBlock:
        """Static activation scales from one pass over ``x``: the expand input (GELU of the depthwise output) and the
        contract input (GELU of the expand output)."""
        b, h, w, c = x.shape
        dense = ops.depthwise5x5_gelu(x.permute(0, 3, 1, 2), self.dw_weight, self.dw_bias)  # BF16 [P, C]
        if self.preset == "mxfp8":
            self.in_scale = quant.calibrate_block32_exponent(dense)
            q1 = ops.quantize_mxfp8(dense, self.in_scale).values.view(b, h, w, c)
            hidden = ops.mxfp8_conv2d(q1, self.in_scale, self.w1.values, self.w1.scale_exponent, self.b1,
                                      1, 1, 1, 1, 0, 0, 1, 1, gelu=True)
            self.hidden_scale = quant.calibrate_block32_exponent(hidden)
        else:
            self.in_scale = (dense.float().abs().amax() / 127).clamp_min(1e-8).reshape(())
            q1 = ops.quantize_int8(dense, self.in_scale).values.view(b, h, w, c)
            hidden = ops.int8_conv2d(q1, self.w1_q, self.in_scale, self.w1_s, self.b1, 1, 1, 1, 1, 0, 0, 1, 1,
                                     gelu=True)
            self.hidden_scale = (hidden.float().abs().amax() / 127).clamp_min(1e-8).reshape(())
        return self

    # -- forward -----------------------------------------------------------------------------------------------

    def forward(self, x: Tensor) -> Tensor:
        b, h, w, c = x.shape
        fused = c == _gemm.MLP_CHANNELS  # the pointwise pair in one launch (bit-identical to the two convs)
        if self.preset == "mxfp8":
            q1 = ops.depthwise5x5_gelu(x.permute(0, 3, 1, 2), self.dw_weight, self.dw_bias, exponent=self.in_scale)
            if fused:
                return _gemm.refiner_mlp(q1.view(b, h, w, c), self.in_scale, self.w1.values, self.w1.scale_exponent,
                                         self.b1, self.hidden_scale, self.w2.values, self.w2.scale_exponent, self.b2,
                                         x)
            q2 = ops.mxfp8_conv2d(q1.view(b, h, w, c), self.in_scale, self.w1.values, self.w1.scale_exponent, self.b1,
                                  1, 1, 1, 1, 0, 0, 1, 1, gelu=True, out_exponent=self.hidden_scale)
            return ops.mxfp8_conv2d(q2, self.hidden_scale, self.w2.values, self.w2.scale_exponent, self.b2,
                                    1, 1, 1, 1, 0, 0, 1, 1, residual=x)
        q1 = ops.depthwise5x5_gelu(x.permute(0, 3, 1, 2), self.dw_weight, self.dw_bias, scale=self.in_scale)
        if fused:
            return _gemm.refiner_mlp(q1.view(b, h, w, c), self.in_scale, self.w1_q, self.w1_s, self.b1,
                                     self.hidden_scale, self.w2_q, self.w2_s, self.b2, x)
        q2 = ops.int8_conv2d(q1.view(b, h, w, c), self.w1_q, self.in_scale, self.w1_s, self.b1,
                             1, 1, 1, 1, 0, 0, 1, 1, gelu=True, out_scale=self.hidden_scale)
        return ops.int8_conv2d(q2, self.w2_q, self.hidden_scale, self.w2_s, self.b2, 1, 1, 1, 1, 0, 0, 1, 1,
                               residual=x)

    __call__ = forward

    def ops_per_pixel(self) -> int:
        c = self.channels
        return 2 * 25 * c + 2 * c * 4 * c * 2


# -- config 4 / config 5 ---------------------------------------------------------------------------------------

STACK_SCALES = ((8, 512), (4, 256), (2, 128), (1, 64))
STACK_BLOCKS = 8
STACK_SIZES = (800, 1024)  # image A and image B, each a batch of 2 (both matching directions)


def bench_block(preset: str, device="cuda", seed: int = 4):
    """Config 4: one block, NHWC N=2, 400x400, C=64. Returns (fn, info)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(2, 400, 400, 64, generator=g).to(torch.bfloat16).to(device)
    block = RefinerBlock(BlockWeights.random(64, g, device), preset).calibrate(x)
    pixels = 2 * 400 * 400
    # bytes each kernel must move once: dw (2C in, C out), expand (C in, 4C out), contract (4C + 2C in, 2C out)
    return (lambda: block(x)), {"ops": pixels * block.ops_per_pixel(), "bytes": 16 * pixels * 64}


def build_stack(preset: str, device="cuda", seed: int = 5):
    g = torch.Generator(device="cpu").manual_seed(seed)
    scales = []
    for stride, channels in STACK_SCALES:
        inputs = [torch.randn(2, size // stride, size // stride, channels, generator=g).to(torch.bfloat16).to(device)
                  for size in STACK_SIZES]
        blocks = []
        for _ in range(STACK_BLOCKS):
            blocks.append(RefinerBlock(BlockWeights.random(channels, g, device), preset).calibrate(inputs[0]))
        scales.append((inputs, blocks))
    return scales


def run_stack(scales, side: torch.cuda.Stream | None = None) -> list[Tensor]:
    """Every scale's blocks over each of its inputs; ``[scale 0 image A, scale 0 image B, scale 1 image A, ...]``.
    With ``side``, the second input of every scale (the other matching direction, independent of the first) runs on
    that stream concurrently with the first on the current stream: the same launches, so the same bits, but the
    coarse scales' small launches overlap instead of each leaving most of the GPU idle. Eagerly, every tensor that
    crosses streams is recorded on the stream that reads it; under graph capture the capture's private pool keeps
    them alive for the graph's lifetime."""
    def chain(x, blocks):
        for block in blocks:
            x = block(x)
        return x

    if side is None:
        return [chain(x, blocks) for inputs, blocks in scales for x in inputs]
    current = torch.cuda.current_stream()
    side.wait_stream(current)  # the inputs are ready
    outs = []
    for inputs, blocks in scales:
        first, *rest = inputs
        with torch.cuda.stream(side):
            others = [chain(x, blocks) for x in rest]
        if not torch.cuda.is_current_stream_capturing():
            for o in others:  # read on the current stream: not reused by the side stream's allocations before that
                o.record_stream(current)
            for x in rest:  # read on the side stream: a caller freeing an input early cannot hand it to new work
                x.record_stream(side)
        outs += [chain(first, blocks), *others]
    current.wait_stream(side)  # every output is complete on the current stream
    return outs


def bench_stack(preset: str, device="cuda"):
    """Config 5: 4 scales (stride 8/4/2/1, C 512/256/128/64) x 8 blocks, images 800^2 and 1024^2, batch 2 each; the
    two matching directions on two streams (default priority)."""
    scales = build_stack(preset, device)
    side = torch.cuda.Stream(device=device)
    ops_total, pixels = 0, []
    for (inputs, blocks) in scales:
        p = sum(x.shape[0] * x.shape[1] * x.shape[2] for x in inputs)
        pixels.append(p)
        ops_total += p * sum(b.ops_per_pixel() for b in blocks)
    return (lambda: run_stack(scales, side)), {"ops": ops_total, "blocks": STACK_BLOCKS * len(STACK_SCALES),
                                         "pixels": pixels}
