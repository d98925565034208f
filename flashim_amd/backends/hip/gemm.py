"""HIP impls of the GEMM-shaped ops of the path (a 1x1 conv is this GEMM), FlashIM's signatures:

* ``int8_linear``     (``flashim/ops/gemm.py:78-101``)  -> ``fim_int8_linear``
* ``mxfp8_linear``    (``flashim/ops/gemm.py:58-72``)   -> ``fim_mxfp8_conv2d`` on a 1 x rows image
* ``mxfp8_scaled_mm`` (``flashim/ops/gemm.py:40-52``)   -> ``fim_mxfp8_scaled_mm`` (per-row swizzled scales)
* ``mxfp8_gelu_mlp``  (``flashim/ops/gemm.py:146-157``) -> ``fim_refiner_mlp`` (the fused MLP, hidden kept in LDS;
  64 -> 256 -> 64 channels), and the refiner block's pointwise pair on the same kernel (:func:`refiner_mlp`)
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from flashim_amd import _lib, quant
from flashim_amd.platforms import is_gfx950


def _bias(bias: Tensor | None, device) -> tuple[Tensor | None, int]:
    if bias is None:
        return None, 0
    if bias.dtype not in (torch.float32, torch.bfloat16):
        bias = bias.float()
    bias = bias.to(device).contiguous()
    return bias, 1 if bias.dtype == torch.bfloat16 else 0


def int8_linear(a: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None, *,
                relu: bool = False, gelu: bool = False, residual: Tensor | None = None) -> Tensor:
    """``[M, K] int8 x [N, K] int8^T`` -> BF16 ``[M, N]``: ``acc * (a_scale * w_scale) + bias``, ReLU, BF16, GELU,
    ``+ residual`` (BF16). ``a_scale`` one value or per-row ``[M, 1]``."""
    m, k = a.shape
    n = weight.shape[0]
    a = a.contiguous()
    weight = weight.contiguous()
    per_row = a_scale.numel() != 1
    a_scale = a_scale.to(device=a.device, dtype=torch.float32).reshape(-1).contiguous()
    w_scale = w_scale.to(device=a.device, dtype=torch.float32).contiguous()
    bias, bias_code = _bias(bias, a.device)
    res_code, res_channels, res_stride = 0, 0, 0
    if residual is not None:
        if residual.dtype not in (torch.float32, torch.bfloat16):
            residual = residual.to(torch.bfloat16)
        if residual.stride(-1) != 1:
            residual = residual.contiguous()
        res_code, res_channels, res_stride = _lib.DTYPE_CODES[residual.dtype], residual.shape[-1], residual.stride(0)
    out = torch.empty(m, n, device=a.device, dtype=torch.bfloat16)
    _lib.call(
        "fim_int8_linear", a.data_ptr(), m, k, weight.data_ptr(), n, None if per_row else a_scale.data_ptr(),
        a_scale.data_ptr() if per_row else None, w_scale.data_ptr(), _lib.ptr(bias), bias_code, int(relu), int(gelu),
        _lib.ptr(residual), res_code, res_channels, res_stride, None, out.data_ptr(), _lib.stream_of(a),
        what=f"int8_linear {m}x{k} -> {n}",
    )
    return out


def mxfp8_linear(activation: quant.QuantizedTensor, bias: Tensor | None, weight: quant.QuantizedWeight) -> Tensor:
    """Static MXFP8 linear: padded BF16 ``[rows, Npad]`` (``ops/gemm.py:58-69``)."""
    a = activation.matrix().contiguous()
    rows, kpad = a.shape
    npad = weight.values.shape[0]
    bias, bias_code = _bias(bias, a.device)
    out = torch.empty(rows, npad, device=a.device, dtype=torch.bfloat16)
    _lib.call(
        "fim_mxfp8_conv2d", a.data_ptr(), 1, 1, rows, kpad, activation.scale_exponent.contiguous().data_ptr(),
        weight.values.contiguous().data_ptr(), npad, weight.scale_exponent.contiguous().data_ptr(), _lib.ptr(bias),
        bias_code, 1, 1, 1, 1, 0, 0, 1, 1, 0, 0, None, 0, 0, None, None, out.data_ptr(), _lib.stream_of(a),
        what=f"mxfp8_linear {rows}x{kpad} -> {npad}",
    )
    return out


def mxfp8_scaled_mm(a: Tensor, b_t: Tensor, a_scale: Tensor, b_scale: Tensor, bias: Tensor | None = None) -> Tensor:
    """``a [M, K]`` x ``b_t [K, N]`` E4M3 with swizzled E8M0 scales on both -> BF16 ``[M, N]`` (+ bias)."""
    m, k = a.shape
    n = b_t.shape[1]
    a = a.contiguous()
    weight = b_t.t().contiguous()  # [N, K]: a view of the usual transposed weight, no copy
    w_exponent = quant.unswizzle_scales(b_scale, n, k // 32).contiguous()
    bias, bias_code = _bias(bias, a.device)
    out = torch.empty(m, n, device=a.device, dtype=torch.bfloat16)
    _lib.call(
        "fim_mxfp8_scaled_mm", a.data_ptr(), m, k, a_scale.contiguous().view(torch.uint8).data_ptr(),
        weight.view(torch.uint8).data_ptr(), n, w_exponent.data_ptr(), _lib.ptr(bias), bias_code, out.data_ptr(),
        _lib.stream_of(a), what=f"mxfp8_scaled_mm {m}x{k} -> {n}",
    )
    return out


MLP_CHANNELS, MLP_HIDDEN = 64, 256  # the fused MLP kernel's shape


def mxfp8_gelu_mlp(x: quant.QuantizedTensor, w1: quant.QuantizedWeight, b1: Tensor, hidden_exponent: Tensor,
                   w2: quant.QuantizedWeight) -> Tensor:
    """``quantize_static(GELU(x W1^T [BF16] + b1) [BF16], hidden_exponent) W2^T`` -> BF16 ``[rows, N2]``
    (``flashim/ops/gemm.py:146-157``) in one launch."""
    a = x.matrix().contiguous()
    rows = a.shape[0]
    b1 = b1.to(device=a.device).contiguous()
    b1_code = 1 if b1.dtype == torch.bfloat16 else 0
    if b1_code == 0:
        b1 = b1.float()
    out = torch.empty(rows, w2.values.shape[0], device=a.device, dtype=torch.bfloat16)
    _lib.call(
        "fim_refiner_mlp", 1, 1, a.data_ptr(), rows, MLP_CHANNELS, MLP_HIDDEN, x.scale_exponent.contiguous().data_ptr(),
        w1.values.contiguous().data_ptr(), w1.scale_exponent.contiguous().data_ptr(), b1.data_ptr(), b1_code,
        hidden_exponent.to(torch.int8).contiguous().data_ptr(), w2.values.contiguous().data_ptr(),
        w2.scale_exponent.contiguous().data_ptr(), None, 0, None, out.data_ptr(), _lib.stream_of(a),
        what=f"mxfp8_gelu_mlp {rows}x{MLP_CHANNELS}",
    )
    return out


def eligible_mxfp8_gelu_mlp(x, w1, b1, hidden_exponent, w2) -> bool:
    return (
        isinstance(x, quant.QuantizedTensor) and is_gfx950(x.device) and x.channels == MLP_CHANNELS
        and isinstance(w1, quant.QuantizedWeight) and isinstance(w2, quant.QuantizedWeight)
        and tuple(w1.values.shape) == (MLP_HIDDEN, MLP_CHANNELS) and tuple(w2.values.shape) == (MLP_CHANNELS, MLP_HIDDEN)
        and hidden_exponent.numel() == MLP_HIDDEN // 32 and b1.numel() == MLP_HIDDEN
    )


def refiner_mlp(x: Tensor, x_scale: Tensor, w1: Tensor, w1_scale: Tensor, b1: Tensor | None, hidden_scale: Tensor,
                w2: Tensor, w2_scale: Tensor, b2: Tensor | None, residual: Tensor | None) -> Tensor:
    """The refiner block's pointwise pair in one launch, bit for bit what the two 1x1 conv launches it replaces
    compute: ``conv1x1(x; W1, b1, GELU, static quantize with hidden_scale)`` then ``conv1x1(.; W2, b2) + residual``.
    INT8 (``x`` int8, FP32 scalar scales, FP32 per-channel weight scales) or MXFP8 (``x`` E4M3, int8 exponents).
    ``x``: ``[..., 64]``; returns BF16 of the same leading shape."""
    mx = x.dtype == torch.float8_e4m3fn
    lead = x.shape[:-1]
    a = x.reshape(-1, MLP_CHANNELS).contiguous()
    rows = a.shape[0]

    def scale(t: Tensor) -> Tensor:
        return t.to(device=a.device, dtype=torch.int8 if mx else torch.float32).contiguous()

    b1, b1_code = _bias(b1, a.device)
    b2, b2_code = _bias(b2, a.device)
    res = None
    if residual is not None:
        res = residual.reshape(-1, MLP_CHANNELS).to(torch.bfloat16).contiguous()
    out = torch.empty(rows, MLP_CHANNELS, device=a.device, dtype=torch.bfloat16)
    xs, w1s, hs, w2s = scale(x_scale), scale(w1_scale), scale(hidden_scale), scale(w2_scale)
    _lib.call(
        "fim_refiner_mlp", 1 if mx else 0, 0, a.view(torch.uint8).data_ptr(), rows, MLP_CHANNELS, MLP_HIDDEN,
        xs.data_ptr(), w1.contiguous().view(torch.uint8).data_ptr(), w1s.data_ptr(), _lib.ptr(b1), b1_code,
        hs.data_ptr(), w2.contiguous().view(torch.uint8).data_ptr(), w2s.data_ptr(), _lib.ptr(b2), b2_code,
        _lib.ptr(res), out.data_ptr(), _lib.stream_of(a), what=f"refiner_mlp {rows}x{MLP_CHANNELS}",
    )
    return out.view(*lead, MLP_CHANNELS)


# -- eligibility ----------------------------------------------------------------------------------------------------


def eligible_int8_linear(a, weight, a_scale, w_scale, bias, *, relu=False, gelu=False, residual=None) -> bool:
    return (
        isinstance(a, Tensor) and is_gfx950(a.device) and a.ndim == 2 and a.dtype == torch.int8
        and weight.dtype == torch.int8 and weight.ndim == 2 and weight.shape[1] == a.shape[1]
        and (a_scale.numel() == 1 or a_scale.numel() == a.shape[0]) and w_scale.numel() == weight.shape[0]
        and (residual is None or tuple(residual.shape) == (a.shape[0], weight.shape[0]))
    )


def eligible_mxfp8_linear(activation, bias, weight) -> bool:
    return (
        isinstance(activation, quant.QuantizedTensor) and is_gfx950(activation.device)
        and isinstance(weight, quant.QuantizedWeight) and weight.values.shape[1] == activation.channels
    )


def eligible_mxfp8_scaled_mm(a, b_t, a_scale, b_scale, bias=None) -> bool:
    if not (isinstance(a, Tensor) and is_gfx950(a.device) and a.ndim == 2 and b_t.ndim == 2):
        return False
    m, k = a.shape
    n = b_t.shape[1]
    return (
        a.dtype == torch.float8_e4m3fn and b_t.dtype == torch.float8_e4m3fn and b_t.shape[0] == k and k % 32 == 0
        and a_scale.numel() == quant.swizzled_size(m, k // 32) and b_scale.numel() == quant.swizzled_size(n, k // 32)
    )


_ = ctypes  # the C signatures live in flashim_amd._lib
