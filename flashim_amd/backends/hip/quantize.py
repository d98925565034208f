"""HIP impls of the activation quantize ops (``flashim/ops/quantize.py:63-131``), with the torch references'
signatures and return types:

* ``quantize_mxfp8`` (``:80-85``) and ``quantize_int8`` (``:91-100``): the static quantizers;
* ``quantize_int8_rows`` (``:148-154``): per-row dynamic INT8 with the reciprocal-product scale;
* ``gelu_quantize`` (``:63-74``) and ``gelu_quantize_int8`` (``:128-131``): GELU (erf form, ``approximate="none"``,
  or tanh form, ``approximate="tanh"``) in the input's dtype, then the same quantizers, in one pass.
"""

from __future__ import annotations

import torch
from torch import Tensor

from flashim_amd import quant
from flashim_amd.platforms import is_gfx950

_FLOATS = (torch.float32, torch.bfloat16, torch.float16)


def quantize_mxfp8(value: Tensor, scale_exponent: Tensor) -> quant.QuantizedTensor:
    """``ops.quantize_mxfp8``: static block-32 E4M3, channels padded to 32; the NHWC view of NCHW memory is read in
    place."""
    return quant.quantize_static(value, scale_exponent)


def quantize_int8(value: Tensor, scale: Tensor, *, channel_scale: Tensor | None = None) -> quant.Int8Tensor:
    """``ops.quantize_int8``: ``round(value [* channel_scale] / scale)`` saturated to +-127, one FP32 division."""
    scale = scale.to(device=value.device, dtype=torch.float32).reshape(())
    return quant.Int8Tensor(quant.quantize_int8_values(value, scale, channel_scale), scale)


def quantize_int8_rows(value: Tensor) -> tuple[Tensor, Tensor]:
    """``ops.quantize_int8_rows``: ``scale = safe_scale(amax(|row|) * float32(1 / 127))``, ``round(value / scale)``
    saturated to +-127 (one IEEE division). Returns int8 values of ``value``'s shape and FP32 scales ``[*leading, 1]``."""
    matrix = value.reshape(-1, value.shape[-1])
    if matrix.stride(-1) != 1:
        matrix = matrix.contiguous()
    q, scale = quant.quantize_int8_rows(matrix)
    return q.reshape(value.shape), scale.reshape(*value.shape[:-1], 1)


def gelu_quantize(value: Tensor, scale_exponent: Tensor, approximate: str = "none", *,
                  input_bias: Tensor | None = None) -> quant.QuantizedTensor:
    """``ops.gelu_quantize``: ``quantize_static(GELU(value [+ input_bias]))``."""
    return quant.gelu_quantize_static(value, scale_exponent, input_bias, approximate)


def gelu_quantize_int8(value: Tensor, scale: Tensor, approximate: str = "none") -> quant.Int8Tensor:
    """``ops.gelu_quantize_int8``: ``quantize_int8(GELU(value))``."""
    return quant.gelu_quantize_int8_static(value, scale, approximate)


def eligible_quantize_mxfp8(value: Tensor, scale_exponent: Tensor) -> bool:
    return isinstance(value, Tensor) and is_gfx950(value.device) and value.ndim >= 2 and value.dtype in _FLOATS


def eligible_quantize_int8(value: Tensor, scale: Tensor, *, channel_scale: Tensor | None = None) -> bool:
    return (
        isinstance(value, Tensor) and is_gfx950(value.device) and value.ndim >= 1 and value.dtype in _FLOATS
        and scale.numel() == 1 and (channel_scale is None or channel_scale.numel() == value.shape[-1])
    )


def eligible_quantize_int8_rows(value: Tensor) -> bool:
    return (isinstance(value, Tensor) and is_gfx950(value.device) and value.ndim >= 1 and value.dtype in _FLOATS
            and value.shape[-1] > 0)


def eligible_gelu_quantize(value: Tensor, scale_exponent: Tensor, approximate: str = "none", *,
                           input_bias: Tensor | None = None) -> bool:
    return (
        approximate in ("none", "tanh") and eligible_quantize_mxfp8(value, scale_exponent)
        and (input_bias is None or input_bias.numel() == value.shape[-1])
    )


def eligible_gelu_quantize_int8(value: Tensor, scale: Tensor, approximate: str = "none") -> bool:
    return approximate in ("none", "tanh") and eligible_quantize_int8(value, scale)
