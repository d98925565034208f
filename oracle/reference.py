"""CPU oracle: a torch (CPU) restatement of FlashIM's torch reference path for the quantized conv ops.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg import
this module, and only as the checker (or as the timed CPU baseline) -- never as a product path.

Each function follows the reference file:line it cites, call for call, so its arithmetic is torch's CPU arithmetic at
the same rounding points. How each is pinned (known answers from FlashIM's tests, closed forms, brute force) is in
``tests/test_oracle.py``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

FP8_MAX = 448.0
BLOCK = 32
INT8_MAX = 127.0
_EPS = torch.finfo(torch.float32).eps


def padded_channels(channels: int) -> int:
    return ((channels + BLOCK - 1) // BLOCK) * BLOCK


# -- quant/formats/mx.py -----------------------------------------------------------------------------------------


def scale_exponent_from_amax(amax: Tensor) -> Tensor:
    """quant/formats/mx.py:22-26."""
    exponent = torch.ceil(torch.log2(amax / FP8_MAX))
    exponent = torch.where(amax == 0, torch.full_like(exponent, -127), exponent)
    return exponent.clamp(-127, 127).to(torch.int8)


def quantize_blocks(blocks: Tensor, scale_exponent: Tensor) -> Tensor:
    """quant/formats/mx.py:29-38."""
    scales = torch.exp2(scale_exponent.float())
    if scale_exponent.ndim == 1:
        scales = scales[None, :, None]
    else:
        scales = scales[..., None]
    return (blocks / scales).clamp(-FP8_MAX, FP8_MAX)


def calibrate_block32_exponent(value: Tensor) -> Tensor:
    """quant/formats/mx.py:41-47."""
    padded = padded_channels(value.shape[-1])
    blocks = F.pad(value.float(), (0, padded - value.shape[-1])).reshape(-1, padded // BLOCK, BLOCK)
    return scale_exponent_from_amax(blocks.abs().amax(dim=(0, 2)))


def quantize_dynamic_2d(value: Tensor) -> tuple[Tensor, Tensor]:
    """quant/formats/mx.py:50-60."""
    rows, cols = value.shape
    blocks = value.float().contiguous().reshape(rows, cols // BLOCK, BLOCK)
    exponent = scale_exponent_from_amax(blocks.abs().amax(dim=-1))
    quantized = (blocks * torch.exp2(-exponent.float())[..., None]).clamp(-FP8_MAX, FP8_MAX)
    return quantized.to(torch.float8_e4m3fn).reshape(rows, cols), exponent


def exponent_to_e8m0(exponent: Tensor) -> Tensor:
    """quant/formats/mx.py:63-64 (as bytes)."""
    return (exponent.to(torch.int16) + 127).to(torch.uint8)


def swizzle_scales(exponent: Tensor) -> Tensor:
    """quant/formats/mx.py:67-86: [rows, K/32] int8 -> cuBLAS 128x4 swizzled E8M0 bytes (uint8)."""
    scales = exponent_to_e8m0(exponent)
    rows, cols = scales.shape
    padded_rows = ((rows + 127) // 128) * 128
    padded_cols = ((cols + 3) // 4) * 4
    if rows != padded_rows or cols != padded_cols:
        padded = torch.zeros((padded_rows, padded_cols), dtype=torch.uint8)
        padded[:rows, :cols] = scales
        scales = padded
    return (
        scales.view(padded_rows // 128, 128, padded_cols // 4, 4)
        .permute(0, 2, 1, 3).reshape(-1, 4, 32, 4).transpose(1, 2).reshape(-1).contiguous()
    )


def dequantize_swizzled(values: Tensor, swizzled: Tensor) -> Tensor:
    """ops/gemm.py:21-37."""
    rows, k = values.shape
    groups = k // 32
    padded_rows = ((rows + 127) // 128) * 128
    padded_cols = ((groups + 3) // 4) * 4
    scales = (
        swizzled.view(torch.uint8).reshape(-1, 32, 4, 4).transpose(1, 2)
        .reshape(padded_rows // 128, padded_cols // 4, 128, 4).permute(0, 2, 1, 3)
        .reshape(padded_rows, padded_cols)[:rows, :groups]
    )
    exponent = scales.to(torch.int16).float() - 127.0
    blocks = values.float().reshape(rows, groups, 32) * torch.exp2(exponent)[..., None]
    return blocks.reshape(rows, k)


# -- quant/formats/int8.py ---------------------------------------------------------------------------------------


def safe_scale(scale: Tensor) -> Tensor:
    """quant/formats/int8.py:13-16."""
    scale = scale.float()
    return torch.where(torch.isfinite(scale) & (scale > _EPS), scale, torch.full_like(scale, _EPS))


def weight_scales(weight: Tensor) -> Tensor:
    """quant/formats/int8.py:19-21."""
    return safe_scale(weight.float().abs().amax(dim=1) / INT8_MAX)


def quantize_symmetric(value: Tensor, scale: Tensor) -> Tensor:
    """quant/formats/int8.py:24-27."""
    return (value.float() / scale).round().clamp(-INT8_MAX, INT8_MAX).to(torch.int8)


# -- quant/tensor.py ---------------------------------------------------------------------------------------------


def quantize_static(value: Tensor, scale_exponent: Tensor) -> Tensor:
    """quant/tensor.py:97-121: E4M3 values [..., Cpad]."""
    padded = padded_channels(value.shape[-1])
    scale_exponent = scale_exponent.to(torch.int8)
    dense = value.contiguous().float()
    if padded != value.shape[-1]:
        dense = F.pad(dense, (0, padded - value.shape[-1]))
    quantized = quantize_blocks(dense.reshape(-1, padded // BLOCK, BLOCK), scale_exponent)
    return quantized.reshape(*value.shape[:-1], padded).to(torch.float8_e4m3fn)


def quantize_int8_static(value: Tensor, scale: Tensor) -> Tensor:
    """quant/tensor.py:148-151: int8 values, packed."""
    scale = scale.to(dtype=torch.float32).reshape(())
    return quantize_symmetric(value, scale).contiguous()


def quantized_weight_from_float(weight: Tensor) -> tuple[Tensor, Tensor]:
    """quant/tensor.py:77-87 (QuantizedWeight.from_float): (E4M3 [Npad, Kpad], int8 [Npad, Kpad/32])."""
    out_padded, in_padded = padded_channels(weight.shape[0]), padded_channels(weight.shape[1])
    padded = F.pad(weight.float(), (0, in_padded - weight.shape[1], 0, out_padded - weight.shape[0]))
    blocks = padded.reshape(out_padded, in_padded // BLOCK, BLOCK)
    exponent = scale_exponent_from_amax(blocks.abs().amax(dim=-1))
    quantized = quantize_blocks(blocks, exponent).reshape(out_padded, in_padded)
    return quantized.to(torch.float8_e4m3fn), exponent


def quantize_int8_rows(value: Tensor) -> tuple[Tensor, Tensor]:
    """ops/quantize.py:148-154: per-row dynamic INT8 (reciprocal product for the scale)."""
    scale = safe_scale(value.float().abs().amax(-1, keepdim=True) * (1 / INT8_MAX))
    return quantize_symmetric(value, scale), scale


# -- ops/quantize.py ---------------------------------------------------------------------------------------------


def quantize_mxfp8(value: Tensor, scale_exponent: Tensor) -> Tensor:
    """ops/quantize.py:80-82."""
    return quantize_static(value, scale_exponent)


def quantize_int8(value: Tensor, scale: Tensor, channel_scale: Tensor | None = None) -> Tensor:
    """ops/quantize.py:91-97."""
    if channel_scale is not None:
        value = value.float() * channel_scale.float()
    return quantize_int8_static(value, scale)


def gelu_quantize(value: Tensor, scale_exponent: Tensor, approximate: str = "none", *,
                  input_bias: Tensor | None = None) -> Tensor:
    """ops/quantize.py:63-74: GELU in value's dtype, or in FP32 of value + input_bias rounded back to value's dtype."""
    if input_bias is not None:
        activated = F.gelu(value.float() + input_bias.float(), approximate=approximate).to(value.dtype)
        return quantize_static(activated, scale_exponent)
    return quantize_static(F.gelu(value, approximate=approximate), scale_exponent)


def gelu_quantize_int8(value: Tensor, scale: Tensor, approximate: str = "none") -> Tensor:
    """ops/quantize.py:128-131."""
    return quantize_int8_static(F.gelu(value, approximate=approximate), scale)


# -- ops/gemm.py -------------------------------------------------------------------------------------------------


def int8_linear(a: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None, *,
                relu: bool = False, gelu: bool = False, residual: Tensor | None = None) -> Tensor:
    """ops/gemm.py:78-98 (CPU branch: int64 accumulation)."""
    acc = a.long() @ weight.long().t()
    out = acc.float() * (a_scale.float() * w_scale.float())
    if bias is not None:
        out = out + bias.float()
    if relu:
        out = out.relu()
    out = out.to(torch.bfloat16)
    if gelu:
        out = F.gelu(out)
    if residual is not None:
        out = residual + out
    return out


def int8_linear_quantize(a: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None,
                         out_scale: Tensor) -> Tensor:
    """ops/gemm.py:104-116: the INT8 values the reference copies into ``out``."""
    return quantize_int8_static(int8_linear(a, weight, a_scale, w_scale, bias), out_scale)


def int8_accumulators(a: Tensor, weight: Tensor) -> Tensor:
    """The int64 accumulators of int8_linear (ops/gemm.py:87)."""
    return a.long() @ weight.long().t()


def mxfp8_linear(values: Tensor, scale_exponent: Tensor, bias: Tensor | None, w_values: Tensor,
                 w_exponent: Tensor) -> Tensor:
    """ops/gemm.py:58-69: dequantize both operands, FP32 matmul, + bias, BF16."""
    a = values.reshape(-1, values.shape[-1]).float() * torch.exp2(scale_exponent.float()).repeat_interleave(32)
    w = w_values.float() * torch.exp2(w_exponent.float()).repeat_interleave(32, dim=1)
    out = a @ w.t()
    if bias is not None:
        out = out + bias.float()
    return out.to(torch.bfloat16)


def mxfp8_gelu_mlp(values: Tensor, scale_exponent: Tensor, w1_values: Tensor, w1_exponent: Tensor, b1: Tensor,
                   hidden_exponent: Tensor, w2_values: Tensor, w2_exponent: Tensor) -> Tensor:
    """ops/gemm.py:146-157: hidden = mxfp8_linear(x, None, w1) (BF16); gelu(hidden.float() + b1.float()) -> BF16;
    quantize_static(., hidden_exponent); mxfp8_linear(., None, w2) -> BF16."""
    hidden = mxfp8_linear(values, scale_exponent, None, w1_values, w1_exponent)
    activated = F.gelu(hidden.float() + b1.float()).to(torch.bfloat16)
    return mxfp8_linear(quantize_static(activated, hidden_exponent), hidden_exponent, None, w2_values, w2_exponent)


def mxfp8_scaled_mm(a: Tensor, b_t: Tensor, a_scale: Tensor, b_scale: Tensor, bias: Tensor | None = None) -> Tensor:
    """ops/gemm.py:40-49."""
    a_dense = dequantize_swizzled(a, a_scale)
    b_dense = dequantize_swizzled(b_t.t(), b_scale)
    out = a_dense @ b_dense.t()
    if bias is not None:
        out = out + bias.float()
    return out.to(torch.bfloat16)


# -- ops/conv.py -------------------------------------------------------------------------------------------------


def im2col_gather(x: Tensor, kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int) -> Tensor:
    """ops/conv.py:144-165."""
    b, h, w, _ = x.shape
    raw = x.view(torch.uint8)
    if ph or pw:
        raw = F.pad(raw, (0, 0, pw, pw, ph, ph))
    ho = (h + 2 * ph - dh * (kh - 1) - 1) // sh + 1
    wo = (w + 2 * pw - dw * (kw - 1) - 1) // sw + 1
    taps = [
        raw[:, ky * dh: ky * dh + (ho - 1) * sh + 1: sh, kx * dw: kx * dw + (wo - 1) * sw + 1: sw]
        for ky in range(kh)
        for kx in range(kw)
    ]
    cols = taps[0] if len(taps) == 1 else torch.cat(taps, dim=-1)
    return cols.reshape(b * ho * wo, -1).view(x.dtype)


def _out_size(h, w, kh, kw, sh, sw, ph, pw, dh, dw):
    return (h + 2 * ph - dh * (kh - 1) - 1) // sh + 1, (w + 2 * pw - dw * (kw - 1) - 1) // sw + 1


def add_residual(out: Tensor, residual: Tensor, relu: bool) -> Tensor:
    """ops/conv.py:198-203."""
    channels = residual.shape[-1]
    summed = out.float()
    summed[..., :channels] += residual.float()
    return (summed.relu() if relu else summed).to(torch.bfloat16)


def int8_conv2d(x: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None,
                kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int, *, relu: bool = False,
                residual: Tensor | None = None, out_scale: Tensor | None = None, gelu: bool = False) -> Tensor:
    """ops/conv.py:174-195. ``gelu`` is the backend's extra epilogue: int8_linear's GELU (ops/gemm.py:94-95), before
    the residual."""
    b, h, w, _ = x.shape
    ho, wo = _out_size(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    cols = im2col_gather(x, kh, kw, sh, sw, ph, pw, dh, dw)
    out = int8_linear(cols, weight, a_scale, w_scale, bias, relu=relu and residual is None, gelu=gelu)
    out = out.reshape(b, ho, wo, -1)
    out = out if residual is None else add_residual(out, residual, relu)
    return out if out_scale is None else quantize_int8_static(out, out_scale)


def int8_conv2d_maxpool(x: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None,
                        kh, kw, sh, sw, ph, pw, dh, dw, *, relu: bool = False, out_scale: Tensor):
    """ops/conv.py:209-219: (BF16 conv output, INT8 quantize of its 2x2 max pool)."""
    out = int8_conv2d(x, weight, a_scale, w_scale, bias, kh, kw, sh, sw, ph, pw, dh, dw, relu=relu)
    pooled = F.max_pool2d(out.permute(0, 3, 1, 2), 2).permute(0, 2, 3, 1)
    return out, quantize_int8_static(pooled, out_scale)


def int8_conv2d_accumulators(x: Tensor, weight: Tensor, kh, kw, sh, sw, ph, pw, dh, dw) -> Tensor:
    """The int32 accumulators ``[B, Ho, Wo, Cout]`` of int8_conv2d (im2col -> int64 matmul)."""
    b, h, w, _ = x.shape
    ho, wo = _out_size(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    cols = im2col_gather(x, kh, kw, sh, sw, ph, pw, dh, dw)
    return int8_accumulators(cols, weight).reshape(b, ho, wo, -1)


def mxfp8_conv2d(x: Tensor, channel_exponent: Tensor, weight: Tensor, weight_exponent: Tensor, bias: Tensor | None,
                 kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int, *, relu: bool = False,
                 residual: Tensor | None = None, out_exponent: Tensor | None = None, gelu: bool = False) -> Tensor:
    """ops/conv.py:309-339 (+ the backend's GELU epilogue, as int8_conv2d)."""
    b, h, w, _ = x.shape
    ho, wo = _out_size(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    taps = kh * kw
    cols = im2col_gather(x, kh, kw, sh, sw, ph, pw, dh, dw)
    out = mxfp8_linear(cols, channel_exponent.repeat(taps), bias, weight, weight_exponent).reshape(b, ho, wo, -1)
    if gelu:
        if relu and residual is None:
            out = F.relu(out)
        out = F.gelu(out)
        if residual is not None:
            out = add_residual(out, residual, relu)
    elif residual is not None:
        out = add_residual(out, residual, relu)
    elif relu:
        out = F.relu(out)
    return out if out_exponent is None else quantize_static(out, out_exponent)


def depthwise5x5_relu_mxfp8(value: Tensor, weight: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    """ops/conv.py:30-41: E4M3 [B*H*W, C] and swizzled E8M0 bytes."""
    channels = value.shape[1]
    kernel = weight.float().t().reshape(channels, 1, 5, 5)
    rounded = value.to(torch.bfloat16).float()
    out = F.relu(F.conv2d(rounded, kernel, bias.float(), padding=2, groups=channels))
    quantized, exponent = quantize_dynamic_2d(out.permute(0, 2, 3, 1).reshape(-1, channels))
    return quantized, swizzle_scales(exponent)


def depthwise5x5_relu_int8(value: Tensor, weight: Tensor, bias: Tensor, scale: Tensor) -> Tensor:
    """ops/conv.py:50-58."""
    channels = value.shape[1]
    kernel = weight.float().t().reshape(channels, 1, 5, 5)
    out = F.relu(F.conv2d(value.to(torch.bfloat16).float(), kernel, bias.float(), padding=2, groups=channels))
    return quantize_symmetric(out.to(torch.bfloat16).permute(0, 2, 3, 1).reshape(-1, channels), scale)


def depthwise5x5_gelu(value: Tensor, weight: Tensor, bias: Tensor, *, scale: Tensor | None = None,
                      exponent: Tensor | None = None) -> Tensor:
    """The backend's refiner producer: a BF16 depthwise conv (FP32 accumulate, rounded to BF16) then nn.GELU in BF16
    (``F.gelu`` of a BF16 tensor) and the consumer's quantize: quantize_int8 (ops/quantize.py:91-97) or
    quantize_mxfp8 (ops/quantize.py:80-82). [B*H*W, C]."""
    channels = value.shape[1]
    kernel = weight.float().t().reshape(channels, 1, 5, 5)
    out = F.conv2d(value.to(torch.bfloat16).float(), kernel, bias.float(), padding=2, groups=channels)
    out = F.gelu(out.to(torch.bfloat16))
    rows = out.permute(0, 2, 3, 1).reshape(-1, channels)
    if scale is not None:
        return quantize_int8_static(rows, scale)
    if exponent is not None:
        return quantize_static(rows, exponent)
    return rows.contiguous()


def depthwise5x5_relu_pointwise(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                                pw_bias: Tensor) -> Tensor:
    """ops/conv.py:67-81: BF16 depthwise 5x5 + bias + ReLU (FP32 accumulate) rounded to BF16, then the 1x1 conv with
    the [C_out, C_in] weight and bias in FP32, rounded to BF16; a [B, C_out, H, W] view of NHWC BF16."""
    channels = value.shape[1]
    kernel = dw_weight.float().t().reshape(channels, 1, 5, 5)
    hidden = F.conv2d(value.to(torch.bfloat16).float(), kernel, dw_bias.float(), padding=2, groups=channels)
    hidden = F.relu(hidden).to(torch.bfloat16).float()
    out = F.conv2d(hidden, pw_weight.float()[:, :, None, None], pw_bias.float())
    return out.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)


def depthwise5x5_relu_pointwise_mxfp8(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                                      pw_scale_swizzled: Tensor, pw_scale_u8: Tensor, pw_bias: Tensor) -> Tensor:
    """ops/conv.py:93-107: the dynamic MXFP8 producer then mxfp8_scaled_mm; a [B, C, H, W] view of NHWC BF16."""
    batch, channels, height, width = value.shape
    quantized, scale = depthwise5x5_relu_mxfp8(value, dw_weight, dw_bias)
    out = mxfp8_scaled_mm(quantized, pw_weight.t(), scale, pw_scale_swizzled, pw_bias)
    return out.reshape(batch, height, width, channels).permute(0, 3, 1, 2)


def depthwise5x5_relu_pointwise_int8(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                                     pw_wscale: Tensor, pw_bias: Tensor, scale: Tensor) -> Tensor:
    """ops/conv.py:119-132: the static INT8 producer then int8_linear; a [B, C, H, W] view of NHWC BF16."""
    batch, channels, height, width = value.shape
    quantized = depthwise5x5_relu_int8(value, dw_weight, dw_bias, scale)
    out = int8_linear(quantized, pw_weight, scale, pw_wscale, pw_bias)
    return out.reshape(batch, height, width, channels).permute(0, 3, 1, 2)


# -- ops/quantize.py:134-142 and ops/conv.py:225-235: the VGG stem ------------------------------------------------


def bias_relu_quantize_int8(raw: Tensor, bias: Tensor, scale: Tensor) -> Tensor:
    """ops/quantize.py:134-142: ``quantize_int8_static(relu(raw + bias))`` of a bias-free NCHW conv output, the bias
    added in the promoted dtype (BF16 + BF16 rounds to BF16, BF16 + FP32 stays FP32); int8 NHWC values."""
    return quantize_int8_static(F.relu(raw + bias.view(1, -1, 1, 1)).permute(0, 2, 3, 1), scale)


def conv2d_small_cin_quantize_int8(x: Tensor, scale: Tensor, weight: Tensor, bias: Tensor) -> Tensor:
    """ops/conv.py:225-235: the 3x3 / pad 1 conv of a small-Cin BF16 NCHW image rounded to BF16 (torch's BF16 conv:
    FP32 accumulation, one rounding), then :func:`bias_relu_quantize_int8`; int8 NHWC values."""
    return bias_relu_quantize_int8(F.conv2d(x, weight, None, padding=1), bias, scale)

