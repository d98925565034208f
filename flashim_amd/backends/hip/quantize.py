"""HIP impls of the activation quantize ops (``flashim/ops/quantize.py:80-100``), with the torch references' signatures
and return types."""

from __future__ import annotations

import torch
from torch import Tensor

from flashim_amd import quant
from flashim_amd.platforms import is_gfx950


def quantize_mxfp8(value: Tensor, scale_exponent: Tensor) -> quant.QuantizedTensor:
    """``ops.quantize_mxfp8``: static block-32 E4M3, channels padded to 32; the NHWC view of NCHW memory is read in
    place."""
    return quant.quantize_static(value, scale_exponent)


def quantize_int8(value: Tensor, scale: Tensor, *, channel_scale: Tensor | None = None) -> quant.Int8Tensor:
    """``ops.quantize_int8``: ``round(value [* channel_scale] / scale)`` saturated to +-127, one FP32 division."""
    scale = scale.to(device=value.device, dtype=torch.float32).reshape(())
    return quant.Int8Tensor(quant.quantize_int8_values(value, scale, channel_scale), scale)


def eligible_quantize_mxfp8(value: Tensor, scale_exponent: Tensor) -> bool:
    return (
        isinstance(value, Tensor) and is_gfx950(value.device) and value.ndim >= 2
        and value.dtype in (torch.float32, torch.bfloat16, torch.float16)
    )


def eligible_quantize_int8(value: Tensor, scale: Tensor, *, channel_scale: Tensor | None = None) -> bool:
    return (
        isinstance(value, Tensor) and is_gfx950(value.device) and value.ndim >= 1
        and value.dtype in (torch.float32, torch.bfloat16, torch.float16) and scale.numel() == 1
        and (channel_scale is None or channel_scale.numel() == value.shape[-1])
    )
