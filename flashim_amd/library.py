"""The C entry points as ``torch.library`` custom ops (namespace ``flashim_amd``), so ``torch.compile`` traces the
HIP impls instead of breaking its graph at every ctypes call (the pattern of FlashIM's CUDA backend,
``flashim/backends/cuda/conv.py:55-76, 148-161``).

Each op's body allocates its outputs with the torch caching allocator, makes one C call on the current stream and
raises on a nonzero status; its fake returns empty outputs of the same shape, dtype and device. Arguments arrive
normalized by the impls in :mod:`flashim_amd.backends.hip` (dtypes, contiguity, devices), so the bodies only read
pointers, sizes and strides. 1-byte float formats cross as their ``uint8`` views where torch's dispatcher has no use
for the float8 dtype.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from flashim_amd import _lib

NS = "flashim_amd"
BLOCK = 32


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dtype_code(t: Tensor) -> int:
    code = _lib.DTYPE_CODES.get(t.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return code


def _bias_code(t: Tensor | None) -> int:
    return 1 if t is not None and t.dtype == torch.bfloat16 else 0


def as_4d(x: Tensor) -> Tensor:
    """``[..., C]`` viewed as ``[B, H, W, C]`` without copying where the leading dims merge."""
    if x.ndim > 4:
        try:
            x = x.view(-1, *x.shape[-3:])
        except RuntimeError:
            x = x.reshape(-1, *x.shape[-3:])
    while x.ndim < 4:
        x = x.unsqueeze(0)
    return x


def conv_out_hw(h: int, w: int, kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int):
    return (h + 2 * ph - dh * (kh - 1) - 1) // sh + 1, (w + 2 * pw - dw * (kw - 1) - 1) // sw + 1


# -- quantizers -------------------------------------------------------------------------------------------------


@torch.library.custom_op(f"{NS}::quantize_mxfp8", mutates_args=())
def quantize_mxfp8(value: Tensor, exponent: Tensor, padded: int) -> Tensor:
    out = torch.empty((*value.shape[:-1], padded), device=value.device, dtype=torch.uint8)
    x = as_4d(value)
    _lib.call("fim_quantize_mxfp8", x.data_ptr(), _dtype_code(value), *x.shape, *x.stride(), exponent.data_ptr(),
              out.data_ptr(), padded, _stream(value), what=f"quantize_mxfp8 {tuple(value.shape)}")
    return out


@quantize_mxfp8.register_fake
def _(value, exponent, padded):
    return value.new_empty((*value.shape[:-1], padded), dtype=torch.uint8)


@torch.library.custom_op(f"{NS}::gelu_quantize_mxfp8", mutates_args=())
def gelu_quantize_mxfp8(value: Tensor, exponent: Tensor, padded: int, input_bias: Optional[Tensor],
                        tanh: bool = False) -> Tensor:
    out = torch.empty((*value.shape[:-1], padded), device=value.device, dtype=torch.uint8)
    x = as_4d(value)
    _lib.call("fim_gelu_quantize_mxfp8", x.data_ptr(), _dtype_code(value), *x.shape, *x.stride(), int(tanh),
              _ptr(input_bias),
              exponent.data_ptr(), out.data_ptr(), padded, _stream(value),
              what=f"gelu_quantize_mxfp8 {tuple(value.shape)}")
    return out


@gelu_quantize_mxfp8.register_fake
def _(value, exponent, padded, input_bias, tanh=False):
    return value.new_empty((*value.shape[:-1], padded), dtype=torch.uint8)


@torch.library.custom_op(f"{NS}::quantize_int8", mutates_args=())
def quantize_int8(value: Tensor, scale: Tensor, channel_scale: Optional[Tensor]) -> Tensor:
    out = torch.empty(value.shape, device=value.device, dtype=torch.int8)
    x = as_4d(value)
    _lib.call("fim_quantize_int8", x.data_ptr(), _dtype_code(value), *x.shape, *x.stride(), scale.data_ptr(),
              _ptr(channel_scale), out.data_ptr(), _stream(value), what=f"quantize_int8 {tuple(value.shape)}")
    return out


@quantize_int8.register_fake
def _(value, scale, channel_scale):
    return value.new_empty(value.shape, dtype=torch.int8)


@torch.library.custom_op(f"{NS}::gelu_quantize_int8", mutates_args=())
def gelu_quantize_int8(value: Tensor, scale: Tensor, tanh: bool = False) -> Tensor:
    out = torch.empty(value.shape, device=value.device, dtype=torch.int8)
    x = as_4d(value)
    _lib.call("fim_gelu_quantize_int8", x.data_ptr(), _dtype_code(value), *x.shape, *x.stride(), int(tanh),
              scale.data_ptr(),
              out.data_ptr(), _stream(value), what=f"gelu_quantize_int8 {tuple(value.shape)}")
    return out


@gelu_quantize_int8.register_fake
def _(value, scale, tanh=False):
    return value.new_empty(value.shape, dtype=torch.int8)


@torch.library.custom_op(f"{NS}::quantize_mxfp8_dynamic", mutates_args=())
def quantize_mxfp8_dynamic(value: Tensor, swizzled: bool) -> tuple[Tensor, Tensor]:
    """``[rows, K]`` -> E4M3 codes (``uint8``) and either int8 exponents ``[rows, K/32]`` or the swizzled E8M0 bytes."""
    rows, cols = value.shape
    if value.data_ptr() % 16:  # the kernel reads 16-byte rows
        value = value.clone(memory_format=torch.contiguous_format)
    out = torch.empty((rows, cols), device=value.device, dtype=torch.uint8)
    groups = cols // BLOCK
    if swizzled:
        size = -(-rows // 128) * 128 * -(-groups // 4) * 4
        scales = (torch.zeros if rows % 128 or groups % 4 else torch.empty)(size, device=value.device,
                                                                            dtype=torch.uint8)
        expo, swz = None, scales
    else:
        scales = torch.empty((rows, groups), device=value.device, dtype=torch.int8)
        expo, swz = scales, None
    _lib.call("fim_quantize_mxfp8_dynamic", value.data_ptr(), _dtype_code(value), rows, cols, value.stride(0),
              out.data_ptr(), _ptr(expo), _ptr(swz), _stream(value), what=f"quantize_mxfp8_dynamic {rows}x{cols}")
    return out, scales


@quantize_mxfp8_dynamic.register_fake
def _(value, swizzled):
    rows, cols = value.shape
    groups = cols // BLOCK
    if swizzled:
        return (value.new_empty((rows, cols), dtype=torch.uint8),
                value.new_empty((-(-rows // 128) * 128 * -(-groups // 4) * 4,), dtype=torch.uint8))
    return value.new_empty((rows, cols), dtype=torch.uint8), value.new_empty((rows, groups), dtype=torch.int8)


@torch.library.custom_op(f"{NS}::quantize_int8_rows", mutates_args=())
def quantize_int8_rows(value: Tensor, reciprocal: bool) -> tuple[Tensor, Tensor]:
    rows, k = value.shape
    q = torch.empty((rows, k), device=value.device, dtype=torch.int8)
    scale = torch.empty(rows, device=value.device, dtype=torch.float32)
    _lib.call("fim_quantize_int8_rows", value.data_ptr(), _dtype_code(value), rows, k, value.stride(0),
              int(reciprocal), q.data_ptr(), scale.data_ptr(), _stream(value), what=f"quantize_int8_rows {rows}x{k}")
    return q, scale


@quantize_int8_rows.register_fake
def _(value, reciprocal):
    rows, k = value.shape
    return value.new_empty((rows, k), dtype=torch.int8), value.new_empty((rows,), dtype=torch.float32)


@torch.library.custom_op(f"{NS}::calibrate_block32", mutates_args=())
def calibrate_block32(matrix: Tensor) -> Tensor:
    rows, channels = matrix.shape
    groups = -(-channels // BLOCK)
    workspace = torch.empty(groups, device=matrix.device, dtype=torch.int32)
    exponent = torch.empty(groups, device=matrix.device, dtype=torch.int8)
    _lib.call("fim_calibrate_block32", matrix.data_ptr(), _dtype_code(matrix), rows, channels, matrix.stride(0),
              workspace.data_ptr(), exponent.data_ptr(), _stream(matrix), what="calibrate_block32")
    return exponent


@calibrate_block32.register_fake
def _(matrix):
    return matrix.new_empty((-(-matrix.shape[1] // BLOCK),), dtype=torch.int8)


# -- implicit-GEMM convolutions and GEMMs -----------------------------------------------------------------------


def _residual_strides(residual: Tensor | None):
    if residual is None:
        return None, 0, 0, None
    return residual, _lib.DTYPE_CODES[residual.dtype], residual.shape[-1], (ctypes.c_int64 * 4)(*residual.stride())


@torch.library.custom_op(f"{NS}::int8_conv2d", mutates_args=())
def int8_conv2d(x: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Optional[Tensor], kh: int, kw: int,
                sh: int, sw: int, ph: int, pw: int, dh: int, dw: int, relu: bool, gelu: bool,
                residual: Optional[Tensor], out_scale: Optional[Tensor]) -> Tensor:
    b, h, w, cin = x.shape
    cout = weight.shape[0]
    ho, wo = conv_out_hw(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    out = torch.empty(b, ho, wo, cout, device=x.device, dtype=torch.int8 if out_scale is not None else torch.bfloat16)
    res, res_code, res_c, res_strides = _residual_strides(residual)
    _lib.call("fim_int8_conv2d", x.data_ptr(), b, h, w, cin, weight.data_ptr(), cout, a_scale.data_ptr(),
              w_scale.data_ptr(), _ptr(bias), _bias_code(bias), kh, kw, sh, sw, ph, pw, dh, dw, int(relu), int(gelu),
              _ptr(res), res_code, res_c, res_strides, _ptr(out_scale), out.data_ptr(), _stream(x),
              what=f"int8_conv2d {tuple(x.shape)} -> {cout} k{kh}x{kw}")
    return out


@int8_conv2d.register_fake
def _(x, weight, a_scale, w_scale, bias, kh, kw, sh, sw, ph, pw, dh, dw, relu, gelu, residual, out_scale):
    b, h, w, _ = x.shape
    ho, wo = conv_out_hw(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    return x.new_empty((b, ho, wo, weight.shape[0]), dtype=torch.int8 if out_scale is not None else torch.bfloat16)


@torch.library.custom_op(f"{NS}::int8_conv2d_maxpool", mutates_args=())
def int8_conv2d_maxpool(x: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Optional[Tensor], kh: int,
                        kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int, relu: bool,
                        out_scale: Tensor) -> tuple[Tensor, Tensor]:
    b, h, w, cin = x.shape
    cout = weight.shape[0]
    ho, wo = conv_out_hw(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    out = torch.empty(b, ho, wo, cout, device=x.device, dtype=torch.bfloat16)
    pooled = torch.empty(b, ho // 2, wo // 2, cout, device=x.device, dtype=torch.int8)
    _lib.call("fim_int8_conv2d_maxpool", x.data_ptr(), b, h, w, cin, weight.data_ptr(), cout, a_scale.data_ptr(),
              w_scale.data_ptr(), _ptr(bias), _bias_code(bias), kh, kw, sh, sw, ph, pw, dh, dw, int(relu),
              out_scale.data_ptr(), out.data_ptr(), pooled.data_ptr(), _stream(x),
              what=f"int8_conv2d_maxpool {tuple(x.shape)} -> {cout} k{kh}x{kw}")
    return out, pooled


@int8_conv2d_maxpool.register_fake
def _(x, weight, a_scale, w_scale, bias, kh, kw, sh, sw, ph, pw, dh, dw, relu, out_scale):
    b, h, w, _ = x.shape
    ho, wo = conv_out_hw(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    cout = weight.shape[0]
    return (x.new_empty((b, ho, wo, cout), dtype=torch.bfloat16),
            x.new_empty((b, ho // 2, wo // 2, cout), dtype=torch.int8))


@torch.library.custom_op(f"{NS}::mxfp8_conv2d", mutates_args=())
def mxfp8_conv2d(x: Tensor, channel_exponent: Tensor, weight: Tensor, weight_exponent: Tensor, bias: Optional[Tensor],
                 kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int, relu: bool, gelu: bool,
                 residual: Optional[Tensor], out_exponent: Optional[Tensor]) -> Tensor:
    """``x`` / ``weight``: the ``uint8`` views of E4M3 tensors; E4M3 output (``uint8``) with ``out_exponent``."""
    b, h, w, cin = x.shape
    cout = weight.shape[0]
    ho, wo = conv_out_hw(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    out = torch.empty(b, ho, wo, cout, device=x.device,
                      dtype=torch.uint8 if out_exponent is not None else torch.bfloat16)
    res, res_code, res_c, res_strides = _residual_strides(residual)
    _lib.call("fim_mxfp8_conv2d", x.data_ptr(), b, h, w, cin, channel_exponent.data_ptr(), weight.data_ptr(), cout,
              weight_exponent.data_ptr(), _ptr(bias), _bias_code(bias), kh, kw, sh, sw, ph, pw, dh, dw, int(relu),
              int(gelu), _ptr(res), res_code, res_c, res_strides, _ptr(out_exponent), out.data_ptr(), _stream(x),
              what=f"mxfp8_conv2d {tuple(x.shape)} -> {cout} k{kh}x{kw}")
    return out


@mxfp8_conv2d.register_fake
def _(x, channel_exponent, weight, weight_exponent, bias, kh, kw, sh, sw, ph, pw, dh, dw, relu, gelu, residual,
      out_exponent):
    b, h, w, _ = x.shape
    ho, wo = conv_out_hw(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    return x.new_empty((b, ho, wo, weight.shape[0]),
                       dtype=torch.uint8 if out_exponent is not None else torch.bfloat16)


@torch.library.custom_op(f"{NS}::int8_linear", mutates_args=())
def int8_linear(a: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Optional[Tensor], relu: bool,
                gelu: bool, residual: Optional[Tensor]) -> Tensor:
    """``a_scale``: one value, or ``[M]`` per-row scales."""
    m, k = a.shape
    n = weight.shape[0]
    per_row = a_scale.numel() != 1
    out = torch.empty(m, n, device=a.device, dtype=torch.bfloat16)
    res_code = res_c = res_stride = 0
    if residual is not None:
        res_code, res_c, res_stride = _lib.DTYPE_CODES[residual.dtype], residual.shape[-1], residual.stride(0)
    _lib.call("fim_int8_linear", a.data_ptr(), m, k, weight.data_ptr(), n, None if per_row else a_scale.data_ptr(),
              a_scale.data_ptr() if per_row else None, w_scale.data_ptr(), _ptr(bias), _bias_code(bias), int(relu),
              int(gelu), _ptr(residual), res_code, res_c, res_stride, None, out.data_ptr(), _stream(a),
              what=f"int8_linear {m}x{k} -> {n}")
    return out


@int8_linear.register_fake
def _(a, weight, a_scale, w_scale, bias, relu, gelu, residual):
    return a.new_empty((a.shape[0], weight.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{NS}::int8_linear_quantize_", mutates_args=("out",))
def int8_linear_quantize_(a: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Optional[Tensor],
                          out_scale: Tensor, out: Tensor) -> None:
    """Writes the INT8 result into ``out`` (``[M, N]``, unit column stride, any row stride)."""
    m, k = a.shape
    n = weight.shape[0]
    per_row = a_scale.numel() != 1
    _lib.call("fim_int8_linear_quantize", a.data_ptr(), m, k, weight.data_ptr(), n,
              None if per_row else a_scale.data_ptr(), a_scale.data_ptr() if per_row else None, w_scale.data_ptr(),
              _ptr(bias), _bias_code(bias), out_scale.data_ptr(), out.data_ptr(), out.stride(0), _stream(a),
              what=f"int8_linear_quantize {m}x{k} -> {n}")


@torch.library.custom_op(f"{NS}::mxfp8_scaled_mm", mutates_args=())
def mxfp8_scaled_mm(a: Tensor, a_scale_swizzled: Tensor, weight: Tensor, weight_exponent: Tensor,
                    bias: Optional[Tensor], weight_scale_e8m0: bool = False) -> Tensor:
    """``a [M, K]`` / ``weight [N, K]``: ``uint8`` views of E4M3; ``a_scale_swizzled`` ``uint8`` E8M0 bytes;
    ``weight_exponent`` ``[N, K/32]`` int8 exponents, or (``weight_scale_e8m0``) their E8M0 bytes."""
    m, k = a.shape
    n = weight.shape[0]
    out = torch.empty(m, n, device=a.device, dtype=torch.bfloat16)
    _lib.call("fim_mxfp8_scaled_mm", a.data_ptr(), m, k, a_scale_swizzled.data_ptr(), weight.data_ptr(), n,
              weight_exponent.data_ptr(), int(weight_scale_e8m0), _ptr(bias), _bias_code(bias), out.data_ptr(),
              _stream(a), what=f"mxfp8_scaled_mm {m}x{k} -> {n}")
    return out


@mxfp8_scaled_mm.register_fake
def _(a, a_scale_swizzled, weight, weight_exponent, bias, weight_scale_e8m0=False):
    return a.new_empty((a.shape[0], weight.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{NS}::im2col_gather", mutates_args=())
def im2col_gather(x: Tensor, kh: int, kw: int, sh: int, sw: int, ph: int, pw: int, dh: int, dw: int) -> Tensor:
    """``x``: ``uint8`` ``[B, H, W, C]`` -> ``uint8`` ``[B*Ho*Wo, kh*kw*C]``."""
    b, h, w, c = x.shape
    ho, wo = conv_out_hw(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    out = torch.empty(b * ho * wo, kh * kw * c, device=x.device, dtype=torch.uint8)
    _lib.call("fim_im2col_gather", x.data_ptr(), b, h, w, c, kh, kw, sh, sw, ph, pw, dh, dw, out.data_ptr(),
              _stream(x), what="im2col_gather")
    return out


@im2col_gather.register_fake
def _(x, kh, kw, sh, sw, ph, pw, dh, dw):
    b, h, w, c = x.shape
    ho, wo = conv_out_hw(h, w, kh, kw, sh, sw, ph, pw, dh, dw)
    return x.new_empty((b * ho * wo, kh * kw * c), dtype=torch.uint8)


@torch.library.custom_op(f"{NS}::refiner_mlp", mutates_args=())
def refiner_mlp(kind: int, semantics: int, x: Tensor, x_scale: Tensor, w1: Tensor, w1_scale: Tensor,
                b1: Optional[Tensor], h_scale: Tensor, w2: Tensor, w2_scale: Tensor, b2: Optional[Tensor],
                residual: Optional[Tensor]) -> Tensor:
    """The fused 64 -> 256 -> 64 MLP over ``x`` (``uint8`` view) ``[rows, 64]`` -> BF16 ``[rows, 64]``."""
    rows, c = x.shape
    h = w1.shape[0]
    out = torch.empty(rows, w2.shape[0], device=x.device, dtype=torch.bfloat16)
    _lib.call("fim_refiner_mlp", kind, semantics, x.data_ptr(), rows, c, h, x_scale.data_ptr(), w1.data_ptr(),
              w1_scale.data_ptr(), _ptr(b1), _bias_code(b1), h_scale.data_ptr(), w2.data_ptr(), w2_scale.data_ptr(),
              _ptr(b2), _bias_code(b2), _ptr(residual), out.data_ptr(), _stream(x), what=f"refiner_mlp {rows}x{c}")
    return out


@refiner_mlp.register_fake
def _(kind, semantics, x, x_scale, w1, w1_scale, b1, h_scale, w2, w2_scale, b2, residual):
    return x.new_empty((x.shape[0], w2.shape[0]), dtype=torch.bfloat16)


# -- depthwise producers and the one-kernel refiner block -------------------------------------------------------

DW_MX_DYNAMIC, DW_INT8, DW_BF16, DW_MX_STATIC = 0, 1, 2, 3
_DW_OUT_DTYPE = {DW_INT8: torch.int8, DW_BF16: torch.bfloat16, DW_MX_STATIC: torch.uint8}


@torch.library.custom_op(f"{NS}::depthwise5x5", mutates_args=())
def depthwise5x5(x: Tensor, weight: Tensor, bias: Tensor, act: int, mode: int, scale: Optional[Tensor],
                 exponent: Optional[Tensor]) -> Tensor:
    """``x`` BF16 NHWC ``[B, H, W, C]`` -> ``[B*H*W, C]``: INT8 (mode 1), BF16 (2) or E4M3 codes (3, ``uint8``)."""
    b, h, w, c = x.shape
    out = torch.empty(b * h * w, c, device=x.device, dtype=_DW_OUT_DTYPE[mode])
    _lib.call("fim_depthwise5x5", x.data_ptr(), b, h, w, c, weight.data_ptr(), bias.data_ptr(), _bias_code(bias), act,
              mode, _ptr(scale), _ptr(exponent), out.data_ptr(), None, None, _stream(x),
              what=f"depthwise5x5 {tuple(x.shape)}")
    return out


@depthwise5x5.register_fake
def _(x, weight, bias, act, mode, scale, exponent):
    b, h, w, c = x.shape
    return x.new_empty((b * h * w, c), dtype=_DW_OUT_DTYPE[mode])


@torch.library.custom_op(f"{NS}::depthwise5x5_mx_dynamic", mutates_args=())
def depthwise5x5_mx_dynamic(x: Tensor, weight: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    """``relu(dwconv5x5(x) + bias)`` -> dynamic MXFP8: E4M3 codes ``[B*H*W, C]`` and swizzled E8M0 bytes."""
    b, h, w, c = x.shape
    rows, groups = b * h * w, c // BLOCK
    out = torch.empty(rows, c, device=x.device, dtype=torch.uint8)
    size = -(-rows // 128) * 128 * -(-groups // 4) * 4
    swz = (torch.zeros if rows % 128 or groups % 4 else torch.empty)(size, device=x.device, dtype=torch.uint8)
    _lib.call("fim_depthwise5x5", x.data_ptr(), b, h, w, c, weight.data_ptr(), bias.data_ptr(), _bias_code(bias), 0,
              DW_MX_DYNAMIC, None, None, out.data_ptr(), None, swz.data_ptr(), _stream(x),
              what=f"depthwise5x5 {tuple(x.shape)}")
    return out, swz


@depthwise5x5_mx_dynamic.register_fake
def _(x, weight, bias):
    b, h, w, c = x.shape
    rows, groups = b * h * w, c // BLOCK
    return (x.new_empty((rows, c), dtype=torch.uint8),
            x.new_empty((-(-rows // 128) * 128 * -(-groups // 4) * 4,), dtype=torch.uint8))


@torch.library.custom_op(f"{NS}::depthwise5x5_relu_pointwise_mxfp8", mutates_args=())
def depthwise5x5_relu_pointwise_mxfp8(x: Tensor, dw_weight: Tensor, dw_bias: Tensor, pw_weight: Tensor,
                                      pw_e8m0: Tensor, pw_bias: Optional[Tensor]) -> Tensor:
    """The one-kernel MXFP8 block at C = N = 128: ``x`` BF16 NHWC -> BF16 NHWC ``[B, H, W, N]``."""
    b, h, w, c = x.shape
    n = pw_weight.shape[0]
    out = torch.empty(b, h, w, n, device=x.device, dtype=torch.bfloat16)
    _lib.call("fim_depthwise5x5_relu_pointwise_mxfp8", x.data_ptr(), b, h, w, c, dw_weight.data_ptr(),
              dw_bias.data_ptr(), _bias_code(dw_bias), pw_weight.data_ptr(), n, pw_e8m0.data_ptr(), _ptr(pw_bias),
              _bias_code(pw_bias),
              out.data_ptr(), _stream(x), what=f"depthwise5x5_relu_pointwise_mxfp8 {tuple(x.shape)}")
    return out


@depthwise5x5_relu_pointwise_mxfp8.register_fake
def _(x, dw_weight, dw_bias, pw_weight, pw_e8m0, pw_bias):
    b, h, w, _ = x.shape
    return x.new_empty((b, h, w, pw_weight.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{NS}::depthwise5x5_relu_pointwise_int8", mutates_args=())
def depthwise5x5_relu_pointwise_int8(x: Tensor, dw_weight: Tensor, dw_bias: Tensor, scale: Tensor, pw_weight: Tensor,
                                     pw_wscale: Tensor, pw_bias: Optional[Tensor]) -> Tensor:
    """The one-kernel INT8 block at C = N = 128: ``x`` BF16 NHWC -> BF16 NHWC ``[B, H, W, N]``; ``scale`` the static
    activation scale (FP32, one value), ``pw_wscale`` FP32 ``[N]``."""
    b, h, w, c = x.shape
    n = pw_weight.shape[0]
    out = torch.empty(b, h, w, n, device=x.device, dtype=torch.bfloat16)
    _lib.call("fim_depthwise5x5_relu_pointwise_int8", x.data_ptr(), b, h, w, c, dw_weight.data_ptr(),
              dw_bias.data_ptr(), _bias_code(dw_bias), scale.data_ptr(), pw_weight.data_ptr(), n, pw_wscale.data_ptr(),
              _ptr(pw_bias),
              _bias_code(pw_bias), out.data_ptr(), _stream(x), what=f"depthwise5x5_relu_pointwise_int8 {tuple(x.shape)}")
    return out


@depthwise5x5_relu_pointwise_int8.register_fake
def _(x, dw_weight, dw_bias, scale, pw_weight, pw_wscale, pw_bias):
    b, h, w, _ = x.shape
    return x.new_empty((b, h, w, pw_weight.shape[0]), dtype=torch.bfloat16)


# -- the VGG stem ---------------------------------------------------------------------------------------------------


@torch.library.custom_op(f"{NS}::conv3x3_small_cin_quantize_int8", mutates_args=())
def conv3x3_small_cin_quantize_int8(x: Tensor, packed: Tensor, bias: Tensor, scale: Tensor) -> Tensor:
    b, cin, h, w = x.shape
    cout = packed.shape[0]
    out = torch.empty(b, h, w, cout, device=x.device, dtype=torch.int8)
    _lib.call("fim_conv3x3_small_cin_quantize_int8", x.data_ptr(), b, cin, h, w, packed.data_ptr(), cout,
              bias.data_ptr(), _bias_code(bias), scale.data_ptr(), out.data_ptr(), _stream(x),
              what=f"conv2d_small_cin_quantize_int8 {tuple(x.shape)} -> {cout}")
    return out


@conv3x3_small_cin_quantize_int8.register_fake
def _(x, packed, bias, scale):
    b, _, h, w = x.shape
    return x.new_empty((b, h, w, packed.shape[0]), dtype=torch.int8)


@torch.library.custom_op(f"{NS}::bias_relu_quantize_int8", mutates_args=())
def bias_relu_quantize_int8(raw: Tensor, bias: Tensor, scale: Tensor) -> Tensor:
    b, c, h, w = raw.shape
    out = torch.empty(b, h, w, c, device=raw.device, dtype=torch.int8)
    _lib.call("fim_bias_relu_quantize_int8", raw.data_ptr(), b, c, h, w, bias.data_ptr(), _bias_code(bias),
              scale.data_ptr(), out.data_ptr(), _stream(raw), what=f"bias_relu_quantize_int8 {tuple(raw.shape)}")
    return out


@bias_relu_quantize_int8.register_fake
def _(raw, bias, scale):
    b, c, h, w = raw.shape
    return raw.new_empty((b, h, w, c), dtype=torch.int8)


@torch.library.custom_op(f"{NS}::pointwise_bf16", mutates_args=())
def pointwise_bf16(x: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
    """``x`` BF16 ``[M, K]`` times ``weight`` BF16 ``[N, K]`` transposed, plus FP32 or BF16 ``bias`` -> BF16 ``[M, N]``."""
    m, k = x.shape
    n = weight.shape[0]
    out = torch.empty(m, n, device=x.device, dtype=torch.bfloat16)
    _lib.call("fim_pointwise_bf16", x.data_ptr(), m, k, weight.data_ptr(), n, _ptr(bias), _bias_code(bias),
              out.data_ptr(), _stream(x),
              what=f"pointwise_bf16 {m}x{k}x{n}")
    return out


@pointwise_bf16.register_fake
def _(x, weight, bias):
    return x.new_empty((x.shape[0], weight.shape[0]), dtype=torch.bfloat16)
