"""HIP impls of the quantized convolution ops, with the signatures of FlashIM's torch references:

* ``int8_conv2d``  (``flashim/ops/conv.py:174-206``) -> ``fim_int8_conv2d``
* ``mxfp8_conv2d`` (``flashim/ops/conv.py:309-342``) -> ``fim_mxfp8_conv2d``
* ``depthwise5x5_relu_mxfp8`` / ``depthwise5x5_relu_int8`` (``flashim/ops/conv.py:30-61``) -> ``fim_depthwise5x5``
* ``depthwise5x5_gelu`` (this backend's refiner-block producer: folded BatchNorm + GELU, BF16 / static INT8 / static
  MXFP8 out) -> ``fim_depthwise5x5``
* ``conv2d_small_cin_quantize_int8`` (``flashim/ops/conv.py:225-235``) -> ``fim_conv3x3_small_cin_quantize_int8``
* ``bias_relu_quantize_int8`` (``flashim/ops/quantize.py:134-142``) -> ``fim_bias_relu_quantize_int8``
* ``depthwise5x5_relu_pointwise`` (``flashim/ops/conv.py:67-84``, BF16) -> the producer's ReLU + BF16 mode then
  ``fim_pointwise_bf16``
* ``depthwise5x5_relu_pointwise_mxfp8`` (``flashim/ops/conv.py:93-113``) -> at C = 128 with a 128 x 128 pointwise
  weight ``fim_depthwise5x5_relu_pointwise_mxfp8`` (one kernel, the reference's fused shapes
  ``flashim/backends/triton/conv.py:310-508``), else the producer then ``fim_mxfp8_scaled_mm``
* ``depthwise5x5_relu_pointwise_int8`` (``flashim/ops/conv.py:119-138``) -> the producer then ``fim_int8_linear``

``gelu=`` on the two convs is an epilogue FlashIM's conv ops do not have: it is ``int8_linear``'s GELU
(``flashim/ops/gemm.py:94-95``): ``F.gelu`` of the BF16 result, rounded to BF16, before the residual.
"""

from __future__ import annotations

import torch
from torch import Tensor

from flashim_amd import library, quant
from flashim_amd.platforms import is_gfx950


conv_output_size = library.conv_out_hw


def _bias(bias: Tensor | None, device: torch.device) -> Tensor | None:
    """FP32 or BF16 ``[N]`` on ``device`` (other dtypes promoted to FP32), or ``None``."""
    if bias is None:
        return None
    if bias.dtype not in (torch.float32, torch.bfloat16):
        bias = bias.float()
    return bias.to(device).contiguous()


def _residual(residual: Tensor | None, device: torch.device, out_shape: tuple[int, int, int, int]) -> Tensor | None:
    """The residual as the kernels read it: ``[B, Ho, Wo, <= Cout]`` FP32 or BF16, any strides."""
    if residual is None:
        return None
    if residual.ndim != 4 or tuple(residual.shape[:3]) != tuple(out_shape[:3]) or residual.shape[3] > out_shape[3]:
        raise ValueError(f"residual {tuple(residual.shape)} does not fit the output {tuple(out_shape)}")
    if residual.device != device:
        raise ValueError("residual must be on the output's device")
    if residual.dtype not in (torch.float32, torch.bfloat16):
        residual = residual.to(torch.bfloat16)
    return residual


def _scalar(t: Tensor, device) -> Tensor:
    return t.to(device=device, dtype=torch.float32).reshape(1).contiguous()


def _same_scale(scale: Tensor, device) -> Tensor:
    """The caller's scale object itself when it is already one FP32 value on ``device``: FlashIM's layers recognise
    an input quantized for them by the identity of its scale."""
    if scale.dtype == torch.float32 and scale.numel() == 1 and scale.device == device:
        return scale
    return scale.to(device=device, dtype=torch.float32).reshape(())


def int8_conv2d(
    x: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None,
    kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int, *, relu: bool = False,
    residual: Tensor | None = None, out_scale: Tensor | None = None, gelu: bool = False,
) -> Tensor:
    """``x`` int8 ``[B, H, W, Cin]`` (packed), ``weight`` int8 ``[Cout, kh*kw*Cin]`` (ky, kx, c) -> BF16
    ``[B, Ho, Wo, Cout]``, or int8 with ``out_scale``."""
    b, h, w, _ = x.shape
    cout = weight.shape[0]
    ho, wo = conv_output_size(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    return library.int8_conv2d(
        x.contiguous(), weight.contiguous(), _scalar(a_scale, x.device),
        w_scale.to(device=x.device, dtype=torch.float32).contiguous(), _bias(bias, x.device),
        kh, kw, sh, sw, ph, pw, dh, dw, bool(relu), bool(gelu), _residual(residual, x.device, (b, ho, wo, cout)),
        None if out_scale is None else _scalar(out_scale, x.device))


def int8_conv2d_maxpool(
    x: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None,
    kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int, *, relu: bool = False, out_scale: Tensor,
) -> tuple[Tensor, Tensor]:
    """``(out, pooled)``: the BF16 ``[B, Ho, Wo, Cout]`` conv output and the INT8 ``[B, Ho/2, Wo/2, Cout]`` 2x2 max pool
    of it quantized with ``out_scale`` (``ops/conv.py:209-222``), the pool from the conv's epilogue."""
    return library.int8_conv2d_maxpool(
        x.contiguous(), weight.contiguous(), _scalar(a_scale, x.device),
        w_scale.to(device=x.device, dtype=torch.float32).contiguous(), _bias(bias, x.device),
        kh, kw, sh, sw, ph, pw, dh, dw, bool(relu), _scalar(out_scale, x.device))


def mxfp8_conv2d(
    x: Tensor, channel_exponent: Tensor, weight: Tensor, weight_exponent: Tensor, bias: Tensor | None,
    kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int, *, relu: bool = False,
    residual: Tensor | None = None, out_exponent: Tensor | None = None, gelu: bool = False,
) -> Tensor:
    """``x`` E4M3 ``[B, H, W, Cin]`` (``Cin % 32 == 0``), ``channel_exponent`` int8 ``[Cin / 32]``, ``weight`` E4M3
    ``[Cout, kh*kw*Cin]`` with ``weight_exponent`` ``[Cout, kh*kw*Cin / 32]`` -> BF16 ``[B, Ho, Wo, Cout]``, or E4M3
    with ``out_exponent``."""
    b, h, w, _ = x.shape
    cout = weight.shape[0]
    ho, wo = conv_output_size(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    if out_exponent is not None:
        out_exponent = out_exponent.to(device=x.device, dtype=torch.int8).contiguous()
    out = library.mxfp8_conv2d(
        x.contiguous().view(torch.uint8), channel_exponent.to(device=x.device, dtype=torch.int8).contiguous(),
        weight.contiguous().view(torch.uint8), weight_exponent.to(device=x.device, dtype=torch.int8).contiguous(),
        _bias(bias, x.device), kh, kw, sh, sw, ph, pw, dh, dw, bool(relu), bool(gelu),
        _residual(residual, x.device, (b, ho, wo, cout)), out_exponent)
    return out if out_exponent is None else out.view(torch.float8_e4m3fn)


# -- depthwise 5x5 producers ------------------------------------------------------------------------------------


def _nhwc_bf16(value: Tensor) -> Tensor:
    """``[B, C, H, W]`` -> its channels-last memory as a packed BF16 ``[B, H, W, C]`` (rounded to BF16 on load, as the
    references do with ``value.to(torch.bfloat16)``)."""
    if value.dtype != torch.bfloat16:
        value = value.to(torch.bfloat16)
    return value.permute(0, 2, 3, 1).contiguous()


def _dw_operands(value: Tensor, weight: Tensor, bias: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """BF16 NHWC input, BF16 weight, and the bias as given when it is FP32 or BF16 (the kernels read either; the
    BF16 -> FP32 widening is exact), else widened to FP32."""
    return (_nhwc_bf16(value), weight.to(device=value.device, dtype=torch.bfloat16).contiguous(), _bias(bias, value.device))


def depthwise5x5_relu_mxfp8(value: Tensor, weight: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    """E4M3 ``[B*H*W, C]`` and the swizzled E8M0 scales of ``relu(dwconv5x5(value) + bias)``."""
    codes, swizzled = library.depthwise5x5_mx_dynamic(*_dw_operands(value, weight, bias))
    return codes.view(torch.float8_e4m3fn), swizzled.view(torch.float8_e8m0fnu)


def depthwise5x5_relu_int8(value: Tensor, weight: Tensor, bias: Tensor, scale: Tensor) -> Tensor:
    """int8 ``[B*H*W, C]``: ``relu(dwconv5x5(value) + bias)`` rounded to BF16, statically quantized."""
    return library.depthwise5x5(*_dw_operands(value, weight, bias), 0, library.DW_INT8, _scalar(scale, value.device),
                                None)


def depthwise5x5_gelu(value: Tensor, weight: Tensor, bias: Tensor, *, scale: Tensor | None = None,
                      exponent: Tensor | None = None) -> Tensor:
    """``gelu(bf16(dwconv5x5(value) + bias))`` rounded to BF16 -> BF16 ``[B*H*W, C]``; with ``scale`` that tensor
    statically quantized to INT8, with ``exponent`` (``[C/32]``) to E4M3."""
    if scale is not None and exponent is not None:
        raise ValueError("scale (INT8) and exponent (MXFP8) are exclusive")
    operands = _dw_operands(value, weight, bias)
    if scale is not None:
        return library.depthwise5x5(*operands, 1, library.DW_INT8, _scalar(scale, value.device), None)
    if exponent is not None:
        e = exponent.to(device=value.device, dtype=torch.int8).contiguous()
        return library.depthwise5x5(*operands, 1, library.DW_MX_STATIC, None, e).view(torch.float8_e4m3fn)
    return library.depthwise5x5(*operands, 1, library.DW_BF16, None, None)


# -- im2col and the depthwise-then-pointwise composites ------------------------------------------------------------


def im2col_gather(x: Tensor, kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int) -> Tensor:
    """``x`` ``[B, H, W, C]`` of a 1-byte dtype -> ``[B*Ho*Wo, kh*kw*C]`` in (ky, kx, c) order, zero padding."""
    return library.im2col_gather(x.contiguous().view(torch.uint8), kh, kw, sh, sw, ph, pw, dh, dw).view(x.dtype)


def _fused_pointwise_shape(value: Tensor, pw_weight: Tensor) -> bool:
    """The one-kernel block's shapes (``flashim/backends/triton/conv.py:561-599``): 128 channels in, 128 x 128
    pointwise weight."""
    return value.shape[1] == 128 and tuple(pw_weight.shape) == (128, 128)


@torch.compiler.assume_constant_result
def _compute_units(index: int) -> int:
    return torch.cuda.get_device_properties(index).multi_processor_count


def _one_kernel_block_wins(value: Tensor) -> bool:
    """Whether the one-kernel depthwise-pointwise block beats its two-launch composite at this image: it takes
    32 x 8-pixel tiles with all 128 channels on a workgroup (two per CU), so with few tiles each workgroup's four
    channel slices in sequence are the latency, and with many the composite's producer (six workgroups per CU, one
    channel slice each) and pointwise GEMM run faster. Measured on MI355X (256 CUs), MXFP8 / INT8, us, one kernel
    against composite: 70 tiles 19.7 / 15.5 and 22.5 / 12.8; 140 tiles 20.7 / 15.6 and 23.3 / 16.3; 200 tiles
    21.8 / 23.2 and 24.3 / 24.9; 256 tiles 23.2 / 23.7 and 25.9 / 26.6; 280 tiles 26.6 / 28.3 and 29.1 / 28.5; 456
    tiles 29.3 / 40.3 and 31.8 / 36.0; 520 tiles 42.7 / 39.7 and 47.2 / 38.8; 675 tiles 43.9 / 39.9 and 49.1 / 41.4;
    1300 tiles (2 x 400 x 400) 74.8 / 59.3 and 81.2 / 62.9. Hence the band
    [3/4, 2] x CUs."""
    batch, _, height, width = value.shape
    tiles = batch * -(-height // 8) * -(-width // 32)
    index = value.device.index if value.device.index is not None else torch.cuda.current_device()
    cus = _compute_units(index)
    return 3 * cus <= 4 * tiles <= 8 * cus


def depthwise5x5_relu_pointwise(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                                pw_bias: Tensor) -> Tensor:
    """The BF16 refiner block (``flashim/ops/conv.py:67-84``) -> ``[B, C_out, H, W]`` view of NHWC BF16 (channels-last
    memory): the depthwise producer's ReLU + BF16 mode (``relu(dwconv + bias)`` rounded to BF16, the reference's hidden
    tensor), then the BF16 pointwise GEMM with FP32 accumulation and bias."""
    batch, _, height, width = value.shape
    hidden = library.depthwise5x5(*_dw_operands(value, dw_weight, dw_bias), 0, library.DW_BF16, None, None)
    out = library.pointwise_bf16(hidden, pw_weight.to(device=value.device, dtype=torch.bfloat16).contiguous(),
                                 _bias(pw_bias, value.device))
    return out.reshape(batch, height, width, -1).permute(0, 3, 1, 2)


def depthwise5x5_relu_pointwise_mxfp8(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                                      pw_scale_swizzled: Tensor, pw_scale_u8: Tensor, pw_bias: Tensor) -> Tensor:
    """The MXFP8 refiner block (``flashim/ops/conv.py:93-113``) -> ``[B, C, H, W]`` view of NHWC BF16: one kernel
    (``fim_depthwise5x5_relu_pointwise_mxfp8``: the quantized activations stay on chip) at 128 x 128 where it is the
    faster (``_one_kernel_block_wins``), otherwise the two-launch composite."""
    if not (_fused_pointwise_shape(value, pw_weight) and _one_kernel_block_wins(value)):
        return pointwise_mxfp8_composite(value, dw_weight, dw_bias, pw_weight, pw_scale_swizzled, pw_scale_u8,
                                         pw_bias)
    return pointwise_mxfp8_fused(value, dw_weight, dw_bias, pw_weight, pw_scale_swizzled, pw_scale_u8, pw_bias)


def pointwise_mxfp8_fused(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                          pw_scale_swizzled: Tensor, pw_scale_u8: Tensor, pw_bias: Tensor) -> Tensor:
    """One kernel at C = 128 with a 128 x 128 pointwise weight; bit for bit the composite."""
    if not _fused_pointwise_shape(value, pw_weight):
        raise ValueError(f"the one-kernel block needs C = 128 and a 128 x 128 weight, got {tuple(value.shape)}, "
                         f"{tuple(pw_weight.shape)}")
    x, dw_w, dw_b = _dw_operands(value, dw_weight, dw_bias)
    out = library.depthwise5x5_relu_pointwise_mxfp8(
        x, dw_w, dw_b, pw_weight.contiguous().view(torch.uint8),
        pw_scale_u8.to(value.device).contiguous().view(torch.uint8), _bias(pw_bias, value.device))
    return out.permute(0, 3, 1, 2)


def pointwise_mxfp8_composite(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                              pw_scale_swizzled: Tensor, pw_scale_u8: Tensor, pw_bias: Tensor) -> Tensor:
    """Two launches: depthwise producer (dynamic MXFP8) then the block-scaled pointwise GEMM with the weight's plain
    E8M0 bytes."""
    batch, _, height, width = value.shape
    codes, swizzled = library.depthwise5x5_mx_dynamic(*_dw_operands(value, dw_weight, dw_bias))
    n, k = pw_weight.shape
    # the weight's E8M0 bytes go to the GEMM as they are (no per-call conversion to signed exponents)
    w_e8m0 = pw_scale_u8.to(value.device).contiguous().view(torch.int8).reshape(n, k // 32)
    out = library.mxfp8_scaled_mm(codes, swizzled, pw_weight.contiguous().view(torch.uint8), w_e8m0,
                                  _bias(pw_bias, value.device), True)
    return out.reshape(batch, height, width, n).permute(0, 3, 1, 2)


def depthwise5x5_relu_pointwise_int8(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                                     pw_wscale: Tensor, pw_bias: Tensor, scale: Tensor) -> Tensor:
    """The INT8 refiner block (``flashim/ops/conv.py:119-138``) -> ``[B, C, H, W]`` view of NHWC BF16: one kernel
    (``fim_depthwise5x5_relu_pointwise_int8``) at 128 x 128 where it is the faster (``_one_kernel_block_wins``),
    otherwise the two-launch composite (the same bits either way)."""
    if _fused_pointwise_shape(value, pw_weight) and _one_kernel_block_wins(value):
        return pointwise_int8_fused(value, dw_weight, dw_bias, pw_weight, pw_wscale, pw_bias, scale)
    return pointwise_int8_composite(value, dw_weight, dw_bias, pw_weight, pw_wscale, pw_bias, scale)


def pointwise_int8_fused(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor, pw_wscale: Tensor,
                         pw_bias: Tensor, scale: Tensor) -> Tensor:
    """One kernel at C = 128 with a 128 x 128 INT8 pointwise weight; bit for bit the composite."""
    if not _fused_pointwise_shape(value, pw_weight):
        raise ValueError(f"the one-kernel block needs C = 128 and a 128 x 128 weight, got {tuple(value.shape)}, "
                         f"{tuple(pw_weight.shape)}")
    x, dw_w, dw_b = _dw_operands(value, dw_weight, dw_bias)
    out = library.depthwise5x5_relu_pointwise_int8(
        x, dw_w, dw_b, _scalar(scale, value.device), pw_weight.to(value.device).contiguous(),
        pw_wscale.to(device=value.device, dtype=torch.float32).contiguous(), _bias(pw_bias, value.device))
    return out.permute(0, 3, 1, 2)


def pointwise_int8_composite(value: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                             pw_wscale: Tensor, pw_bias: Tensor, scale: Tensor) -> Tensor:
    """Two launches: static INT8 producer then ``int8_linear``."""
    from flashim_amd.backends.hip import gemm

    batch, _, height, width = value.shape
    quantized = depthwise5x5_relu_int8(value, dw_weight, dw_bias, scale)
    out = gemm.int8_linear(quantized, pw_weight, scale, pw_wscale, pw_bias)
    return out.reshape(batch, height, width, -1).permute(0, 3, 1, 2)


# -- eligibility ----------------------------------------------------------------------------------------------------


def eligible_int8_conv2d(x, weight, a_scale, w_scale, bias, kh, kw, sh, sw, ph, pw, dh, dw, **_) -> bool:
    return (
        isinstance(x, Tensor) and is_gfx950(x.device) and x.ndim == 4 and x.dtype == torch.int8
        and weight.dtype == torch.int8 and tuple(weight.shape) == (weight.shape[0], kh * kw * x.shape[-1])
        and a_scale.numel() == 1 and w_scale.numel() == weight.shape[0]
        and (bias is None or bias.numel() == weight.shape[0])
    )


def eligible_int8_conv2d_maxpool(x, weight, a_scale, w_scale, bias, kh, kw, sh, sw, ph, pw, dh, dw, *, relu=False,
                                  out_scale=None) -> bool:
    return out_scale is not None and out_scale.numel() == 1 and eligible_int8_conv2d(
        x, weight, a_scale, w_scale, bias, kh, kw, sh, sw, ph, pw, dh, dw)


def eligible_mxfp8_conv2d(x, channel_exponent, weight, weight_exponent, bias, kh, kw, sh, sw, ph, pw, dh, dw,
                          **kwargs) -> bool:
    out_exponent = kwargs.get("out_exponent")
    return (
        isinstance(x, Tensor) and is_gfx950(x.device) and x.ndim == 4 and x.dtype == torch.float8_e4m3fn
        and x.shape[-1] % 32 == 0 and weight.dtype == torch.float8_e4m3fn
        and tuple(weight.shape) == (weight.shape[0], kh * kw * x.shape[-1])
        and tuple(weight_exponent.shape) == (weight.shape[0], kh * kw * x.shape[-1] // 32)
        and tuple(channel_exponent.shape) == (x.shape[-1] // 32,)
        and (bias is None or bias.numel() == weight.shape[0])
        and (out_exponent is None or (weight.shape[0] % 32 == 0 and out_exponent.numel() == weight.shape[0] // 32))
    )


def eligible_depthwise(value: Tensor, weight: Tensor, bias: Tensor, *rest, **kwargs) -> bool:
    return (
        isinstance(value, Tensor) and is_gfx950(value.device) and value.ndim == 4 and value.shape[1] % 32 == 0
        and tuple(weight.shape) == (25, value.shape[1]) and tuple(bias.shape) == (value.shape[1],)
        and (kwargs.get("exponent") is None or kwargs["exponent"].numel() == value.shape[1] // 32)
    )


def eligible_im2col(x, kh, kw, sh, sw, ph, pw, dh, dw) -> bool:
    return isinstance(x, Tensor) and is_gfx950(x.device) and x.ndim == 4 and x.element_size() == 1


def eligible_pointwise_bf16(value, dw_weight, dw_bias, pw_weight, pw_bias) -> bool:
    """The reference's fused-block contract (``flashim/backends/triton/conv.py:540-553``: BF16 weights) on this
    backend's kernels: C a multiple of 32 up to 128, C_out a multiple of 16 up to 128."""
    return (
        eligible_depthwise(value, dw_weight, dw_bias) and value.shape[1] <= 128 and dw_weight.dtype == torch.bfloat16
        and pw_weight.dtype == torch.bfloat16 and pw_weight.ndim == 2 and pw_weight.shape[1] == value.shape[1]
        and pw_weight.shape[0] % 16 == 0 and pw_weight.shape[0] <= 128
        and pw_bias is not None and pw_bias.numel() == pw_weight.shape[0]
    )


def eligible_pointwise_mxfp8(value, dw_weight, dw_bias, pw_weight, pw_scale_swizzled, pw_scale_u8, pw_bias) -> bool:
    return (
        eligible_depthwise(value, dw_weight, dw_bias) and pw_weight.dtype == torch.float8_e4m3fn
        and pw_weight.ndim == 2 and pw_weight.shape[1] == value.shape[1]
        and pw_scale_u8.numel() == pw_weight.shape[0] * pw_weight.shape[1] // 32
    )


def eligible_pointwise_int8(value, dw_weight, dw_bias, pw_weight, pw_wscale, pw_bias, scale) -> bool:
    return (
        eligible_depthwise(value, dw_weight, dw_bias) and pw_weight.dtype == torch.int8 and pw_weight.ndim == 2
        and pw_weight.shape[1] == value.shape[1] and pw_wscale.numel() == pw_weight.shape[0] and scale.numel() == 1
    )


# -- the VGG stem: conv2d_small_cin_quantize_int8 (flashim/ops/conv.py:225-235) and its epilogue alone,
# bias_relu_quantize_int8 (flashim/ops/quantize.py:134-142) ------------------------------------------------------

STEM_MAX_CIN = 8


def small_cin_prepare(weight: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    """``[Cout, Cin, 3, 3]`` -> BF16 ``[Cout, KP]``: taps in (c, ky, kx) order, zero-padded to KP = 32 ceil(9 Cin / 32)
    (the MFMA's K step); ``bias`` unchanged."""
    cout, cin = weight.shape[:2]
    taps = 9 * cin
    kp = -(-taps // 32) * 32
    packed = torch.nn.functional.pad(weight.detach().to(torch.bfloat16).reshape(cout, taps), (0, kp - taps))
    return packed.contiguous(), bias.detach()


def conv2d_small_cin_quantize_int8(x: Tensor, scale: Tensor, packed: Tensor, bias: Tensor) -> quant.Int8Tensor:
    """``quantize_int8(relu(bf16(conv3x3(x)) + bias))`` -> INT8 NHWC ``[B, H, W, Cout]`` (an :class:`Int8Tensor` with
    ``scale``); ``packed`` from :func:`small_cin_prepare`."""
    out = library.conv3x3_small_cin_quantize_int8(x.contiguous(), packed.to(x.device).contiguous(),
                                                  _bias(bias, x.device), _scalar(scale, x.device))
    return quant.Int8Tensor(out, _same_scale(scale, x.device))


def eligible_small_cin(x: Tensor, scale: Tensor, weight: Tensor, bias: Tensor) -> bool:
    return (
        isinstance(x, Tensor) and x.ndim == 4 and x.dtype == torch.bfloat16 and x.is_contiguous() and is_gfx950(x.device)
        and weight.dtype == torch.bfloat16 and bias.dtype in (torch.bfloat16, torch.float32) and scale.numel() == 1
        and x.shape[1] == weight.shape[1]
    )


def accepts_small_cin(weight: Tensor, bias: Tensor) -> bool:
    cout = weight.shape[0]
    return (
        weight.ndim == 4 and tuple(weight.shape[2:]) == (3, 3) and 1 <= weight.shape[1] <= STEM_MAX_CIN
        and 16 <= cout <= 128 and cout & (cout - 1) == 0 and tuple(bias.shape) == (cout,)
    )


def bias_relu_quantize_int8(raw: Tensor, bias: Tensor, scale: Tensor) -> quant.Int8Tensor:
    """``quantize_int8(relu(raw + bias))`` of a BF16 NCHW conv output -> INT8 NHWC ``[B, H, W, C]``."""
    out = library.bias_relu_quantize_int8(raw.contiguous(), _bias(bias, raw.device), _scalar(scale, raw.device))
    return quant.Int8Tensor(out, _same_scale(scale, raw.device))


def eligible_bias_relu_quantize(raw: Tensor, bias: Tensor, scale: Tensor) -> bool:
    return (
        isinstance(raw, Tensor) and raw.ndim == 4 and raw.dtype == torch.bfloat16 and is_gfx950(raw.device)
        and bias.dtype in (torch.bfloat16, torch.float32) and bias.numel() == raw.shape[1] and scale.numel() == 1
    )

