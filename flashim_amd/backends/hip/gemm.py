"""HIP impls of the GEMM-shaped ops of the path (a 1x1 conv is this GEMM), FlashIM's signatures:

* ``int8_linear``     (``flashim/ops/gemm.py:78-101``)  -> ``fim_int8_linear``
* ``int8_linear_quantize`` (``flashim/ops/gemm.py:104-116``) -> ``fim_int8_linear_quantize`` (INT8 into a strided
  ``out``)
* ``mxfp8_linear``    (``flashim/ops/gemm.py:58-72``)   -> ``fim_mxfp8_conv2d`` on a 1 x rows image
* ``mxfp8_scaled_mm`` (``flashim/ops/gemm.py:40-52``)   -> ``fim_mxfp8_scaled_mm`` (per-row swizzled scales)
* ``mxfp8_gelu_mlp``  (``flashim/ops/gemm.py:146-157``) -> ``fim_refiner_mlp`` (the fused MLP, hidden kept in LDS;
  64 -> 256 -> 64 channels), and the refiner block's pointwise pair on the same kernel (:func:`refiner_mlp`)
"""

from __future__ import annotations

import torch
from torch import Tensor

from flashim_amd import library, quant
from flashim_amd.platforms import is_gfx950


def _bias(bias: Tensor | None, device) -> Tensor | None:
    """FP32 or BF16 ``[N]`` on ``device`` (other dtypes promoted to FP32), or ``None``."""
    if bias is None:
        return None
    if bias.dtype not in (torch.float32, torch.bfloat16):
        bias = bias.float()
    return bias.to(device).contiguous()


def _a_scale(a_scale: Tensor, device) -> Tensor:
    return a_scale.to(device=device, dtype=torch.float32).reshape(-1).contiguous()


def int8_linear(a: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None, *,
                relu: bool = False, gelu: bool = False, residual: Tensor | None = None) -> Tensor:
    """``[M, K] int8 x [N, K] int8^T`` -> BF16 ``[M, N]``: ``acc * (a_scale * w_scale) + bias``, ReLU, BF16, GELU,
    ``+ residual`` (BF16). ``a_scale`` one value or per-row ``[M, 1]``."""
    if residual is not None:
        if residual.dtype not in (torch.float32, torch.bfloat16):
            residual = residual.to(torch.bfloat16)
        if residual.stride(-1) != 1:
            residual = residual.contiguous()
    return library.int8_linear(a.contiguous(), weight.contiguous(), _a_scale(a_scale, a.device),
                               w_scale.to(device=a.device, dtype=torch.float32).contiguous(), _bias(bias, a.device),
                               bool(relu), bool(gelu), residual)


def int8_linear_quantize(a: Tensor, weight: Tensor, a_scale: Tensor, w_scale: Tensor, bias: Tensor | None,
                         out_scale: Tensor, out: Tensor) -> Tensor:
    """``out[...] = quantize_int8(int8_linear(a, ...), out_scale).values`` written in place: ``out`` INT8 ``[M, N]``
    with unit column stride and any row stride (``flashim/ops/gemm.py:104-116``). Returns ``out``."""
    library.int8_linear_quantize_(a.contiguous(), weight.contiguous(), _a_scale(a_scale, a.device),
                                  w_scale.to(device=a.device, dtype=torch.float32).contiguous(),
                                  _bias(bias, a.device), out_scale.to(device=a.device, dtype=torch.float32).reshape(1)
                                  .contiguous(), out)
    return out


def mxfp8_linear(activation: quant.QuantizedTensor, bias: Tensor | None, weight: quant.QuantizedWeight) -> Tensor:
    """Static MXFP8 linear: padded BF16 ``[rows, Npad]`` (``ops/gemm.py:58-69``), a 1x1 conv over a 1 x rows image."""
    a = activation.matrix().contiguous().view(torch.uint8)
    rows, kpad = a.shape
    out = library.mxfp8_conv2d(
        a.view(1, 1, rows, kpad), activation.scale_exponent.contiguous(), weight.values.contiguous().view(torch.uint8),
        weight.scale_exponent.contiguous(), _bias(bias, a.device), 1, 1, 1, 1, 0, 0, 1, 1, False, False, None, None)
    return out.view(rows, -1)


def mxfp8_scaled_mm(a: Tensor, b_t: Tensor, a_scale: Tensor, b_scale: Tensor, bias: Tensor | None = None) -> Tensor:
    """``a [M, K]`` x ``b_t [K, N]`` E4M3 with swizzled E8M0 scales on both -> BF16 ``[M, N]`` (+ bias)."""
    k = a.shape[1]
    n = b_t.shape[1]
    weight = b_t.t().contiguous()  # [N, K]: a view of the usual transposed weight, no copy
    w_exponent = quant.unswizzle_scales(b_scale, n, k // 32).contiguous()
    return library.mxfp8_scaled_mm(a.contiguous().view(torch.uint8), a_scale.contiguous().view(torch.uint8),
                                   weight.view(torch.uint8), w_exponent, _bias(bias, a.device))


MLP_CHANNELS, MLP_HIDDEN = 64, 256  # the fused MLP kernel's shape


def mxfp8_gelu_mlp(x: quant.QuantizedTensor, w1: quant.QuantizedWeight, b1: Tensor, hidden_exponent: Tensor,
                   w2: quant.QuantizedWeight) -> Tensor:
    """``quantize_static(GELU(x W1^T [BF16] + b1) [BF16], hidden_exponent) W2^T`` -> BF16 ``[rows, N2]``
    (``flashim/ops/gemm.py:146-157``) in one launch."""
    a = x.matrix().contiguous().view(torch.uint8)
    b1 = b1.to(device=a.device)
    if b1.dtype != torch.bfloat16:
        b1 = b1.float()
    return library.refiner_mlp(
        1, 1, a, x.scale_exponent.contiguous(), w1.values.contiguous().view(torch.uint8),
        w1.scale_exponent.contiguous(), b1.contiguous(), hidden_exponent.to(device=a.device, dtype=torch.int8)
        .contiguous(), w2.values.contiguous().view(torch.uint8), w2.scale_exponent.contiguous(), None, None)


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
    a = x.reshape(-1, MLP_CHANNELS).contiguous().view(torch.uint8)

    def scale(t: Tensor) -> Tensor:
        return t.to(device=a.device, dtype=torch.int8 if mx else torch.float32).contiguous()

    res = None
    if residual is not None:
        res = residual.reshape(-1, MLP_CHANNELS).to(torch.bfloat16).contiguous()
    out = library.refiner_mlp(
        1 if mx else 0, 0, a, scale(x_scale), w1.contiguous().view(torch.uint8), scale(w1_scale), _bias(b1, a.device),
        scale(hidden_scale), w2.contiguous().view(torch.uint8), scale(w2_scale), _bias(b2, a.device), res)
    return out.view(*lead, MLP_CHANNELS)


# -- eligibility ----------------------------------------------------------------------------------------------------


def eligible_int8_linear(a, weight, a_scale, w_scale, bias, *, relu=False, gelu=False, residual=None) -> bool:
    return (
        isinstance(a, Tensor) and is_gfx950(a.device) and a.ndim == 2 and a.dtype == torch.int8
        and weight.dtype == torch.int8 and weight.ndim == 2 and weight.shape[1] == a.shape[1]
        and (a_scale.numel() == 1 or a_scale.numel() == a.shape[0]) and w_scale.numel() == weight.shape[0]
        and (residual is None or tuple(residual.shape) == (a.shape[0], weight.shape[0]))
    )


def eligible_int8_linear_quantize(a, weight, a_scale, w_scale, bias, out_scale, out) -> bool:
    return (
        eligible_int8_linear(a, weight, a_scale, w_scale, bias) and out_scale.numel() == 1
        and isinstance(out, Tensor) and out.dtype == torch.int8 and out.device == a.device and out.ndim == 2
        and tuple(out.shape) == (a.shape[0], weight.shape[0]) and out.stride(1) == 1 and out.stride(0) >= out.shape[1]
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

