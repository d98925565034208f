"""MXFP8 / INT8 formats and the quantized containers, with FlashIM's layouts (``flashim/quant/formats/mx.py``,
``flashim/quant/formats/int8.py``, ``flashim/quant/tensor.py``), every arithmetic step on the HIP kernels.

Layouts (unchanged from FlashIM, so tensors move between the two without conversion):

* :class:`QuantizedTensor`: E4M3 ``values [*leading, Cpad]`` (``Cpad`` = channels rounded up to 32), one static int8
  exponent per 32-channel block ``[Cpad / 32]`` shared by every row, ``logical_shape`` the unpadded shape;
* :class:`QuantizedWeight`: E4M3 ``[Npad, Kpad]`` with one exponent per (row, 32 inputs) ``[Npad, Kpad / 32]``;
* :class:`Int8Tensor`: int8 values with one FP32 scale;
* swizzled scales: E8M0 bytes (``e + 127``) in cuBLAS' 128 x 4 ``SWIZZLE_32_4_4`` layout (byte permutations only,
  done with tensor views).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

from flashim_amd import _lib, library

FP8_MAX = 448.0
INT8_MAX = 127.0
BLOCK = 32


def padded_channels(channels: int) -> int:
    return ((channels + BLOCK - 1) // BLOCK) * BLOCK


def _require_gpu(t: Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what}: flashim_amd computes on the GPU only (got a {t.device.type} tensor)")


def _dtype_code(t: Tensor, what: str) -> int:
    code = _lib.DTYPE_CODES.get(t.dtype)
    if code is None:
        raise TypeError(f"{what}: unsupported dtype {t.dtype}")
    return code


@dataclass(frozen=True)
class QuantizedTensor:
    values: Tensor
    scale_exponent: Tensor
    logical_shape: tuple[int, ...]

    def __post_init__(self) -> None:
        if self.values.dtype != torch.float8_e4m3fn:
            raise ValueError(f"Expected float8_e4m3fn values, got {self.values.dtype}")
        if self.scale_exponent.dtype != torch.int8:
            raise ValueError("scale_exponent must be int8 unbiased exponents")
        channels = self.values.shape[-1]
        if channels % BLOCK or channels < self.logical_shape[-1]:
            raise ValueError(f"Bad physical channels {channels} for {self.logical_shape}")
        if tuple(self.scale_exponent.shape) != (channels // BLOCK,):
            raise ValueError(f"Expected scale shape {(channels // BLOCK,)}")

    @property
    def device(self) -> torch.device:
        return self.values.device

    @property
    def channels(self) -> int:
        return self.values.shape[-1]

    @property
    def rows(self) -> int:
        return math.prod(self.values.shape[:-1])

    def matrix(self) -> Tensor:
        return self.values.reshape(-1, self.channels)


@dataclass(frozen=True)
class QuantizedWeight:
    values: Tensor
    scale_exponent: Tensor
    logical_shape: tuple[int, int]

    @property
    def out_features(self) -> int:
        return self.values.shape[0]

    @property
    def in_features(self) -> int:
        return self.values.shape[1]

    @classmethod
    def from_float(cls, weight: Tensor) -> QuantizedWeight:
        """Pad ``[N, K]`` to multiples of 32, one exponent per (row, 32 inputs) from the block amax, E4M3 values
        (``flashim/quant/tensor.py:77-87``): the dynamic per-(row, 32) quantizer on the padded FP32 weight."""
        if weight.ndim != 2:
            raise ValueError(f"Unsupported weight shape: {tuple(weight.shape)}")
        _require_gpu(weight, "QuantizedWeight.from_float")
        if not torch.isfinite(weight).all():
            raise ValueError("Cannot quantize non-finite weights")
        n_pad, k_pad = padded_channels(weight.shape[0]), padded_channels(weight.shape[1])
        padded = F.pad(weight.float(), (0, k_pad - weight.shape[1], 0, n_pad - weight.shape[0])).contiguous()
        values, exponent = quantize_dynamic_2d(padded)
        return cls(values, exponent, tuple(weight.shape))


@dataclass(frozen=True)
class Int8Tensor:
    values: Tensor
    scale: Tensor

    def __post_init__(self) -> None:
        if self.values.dtype != torch.int8:
            raise ValueError(f"Expected int8 values, got {self.values.dtype}")
        if self.scale.dtype != torch.float32 or self.scale.numel() != 1:
            raise ValueError("scale must be a single FP32 value")

    @property
    def logical_shape(self) -> tuple[int, ...]:
        return tuple(self.values.shape)

    def matrix(self) -> Tensor:
        return self.values.reshape(-1, self.values.shape[-1])


# -- quantizers (HIP) ---------------------------------------------------------------------------------------------


def quantize_static(value: Tensor, scale_exponent: Tensor) -> QuantizedTensor:
    """Static block-32 E4M3 quantization, channels padded to 32 (``flashim/quant/tensor.py:97-121``)."""
    if value.ndim < 2:
        raise ValueError(f"Expected a channelized tensor, got {tuple(value.shape)}")
    _require_gpu(value, "quantize_static")
    _dtype_code(value, "quantize_static")
    padded = padded_channels(value.shape[-1])
    scale_exponent = scale_exponent.to(device=value.device, dtype=torch.int8).contiguous()
    if tuple(scale_exponent.shape) != (padded // BLOCK,):
        raise ValueError(f"Expected scale shape {(padded // BLOCK,)}, got {tuple(scale_exponent.shape)}")
    codes = library.quantize_mxfp8(value, scale_exponent, padded)
    return QuantizedTensor(codes.view(torch.float8_e4m3fn), scale_exponent, tuple(value.shape))


def gelu_quantize_static(value: Tensor, scale_exponent: Tensor, input_bias: Tensor | None = None,
                         approximate: str = "none") -> QuantizedTensor:
    """``quantize_static(GELU(value [+ input_bias]))``, GELU (``approximate`` "none": erf form, "tanh": tanh form)
    rounded to ``value``'s dtype (``flashim/ops/quantize.py:63-74``)."""
    tanh = _gelu_form(approximate)
    if value.ndim < 2:
        raise ValueError(f"Expected a channelized tensor, got {tuple(value.shape)}")
    _require_gpu(value, "gelu_quantize")
    _dtype_code(value, "gelu_quantize")
    padded = padded_channels(value.shape[-1])
    scale_exponent = scale_exponent.to(device=value.device, dtype=torch.int8).contiguous()
    if tuple(scale_exponent.shape) != (padded // BLOCK,):
        raise ValueError(f"Expected scale shape {(padded // BLOCK,)}, got {tuple(scale_exponent.shape)}")
    if input_bias is not None:
        input_bias = input_bias.to(device=value.device, dtype=torch.float32).contiguous()
    codes = library.gelu_quantize_mxfp8(value, scale_exponent, padded, input_bias, tanh)
    return QuantizedTensor(codes.view(torch.float8_e4m3fn), scale_exponent, tuple(value.shape))


def quantize_int8_values(value: Tensor, scale: Tensor, channel_scale: Tensor | None = None) -> Tensor:
    """``round(value * channel_scale / scale)`` saturated to +-127, packed int8 of ``value``'s shape."""
    _require_gpu(value, "quantize_int8")
    _dtype_code(value, "quantize_int8")
    scale = scale.to(device=value.device, dtype=torch.float32).reshape(1)
    if channel_scale is not None:
        channel_scale = channel_scale.to(device=value.device, dtype=torch.float32).contiguous()
    return library.quantize_int8(value, scale, channel_scale)


def quantize_int8_static(value: Tensor, scale: Tensor) -> Int8Tensor:
    """Static per-tensor INT8 (``flashim/quant/tensor.py:148-151``)."""
    scale = scale.to(device=value.device, dtype=torch.float32).reshape(())
    return Int8Tensor(quantize_int8_values(value, scale), scale)


def _gelu_form(approximate: str) -> bool:
    if approximate not in ("none", "tanh"):
        raise ValueError(f"approximate must be 'none' or 'tanh', got {approximate!r}")
    return approximate == "tanh"


def gelu_quantize_int8_static(value: Tensor, scale: Tensor, approximate: str = "none") -> Int8Tensor:
    """``quantize_int8_static(GELU(value))``, GELU (erf or tanh form) rounded to ``value``'s dtype
    (``flashim/ops/quantize.py:128-131``)."""
    tanh = _gelu_form(approximate)
    _require_gpu(value, "gelu_quantize_int8")
    _dtype_code(value, "gelu_quantize_int8")
    scale = scale.to(device=value.device, dtype=torch.float32).reshape(())
    return Int8Tensor(library.gelu_quantize_int8(value, scale.reshape(1), tanh), scale)


def _dynamic_input(value: Tensor, what: str) -> Tensor:
    if value.ndim != 2:
        raise ValueError(f"Expected a matrix, got shape {tuple(value.shape)}")
    if value.shape[1] % BLOCK:
        raise ValueError(f"MXFP8 requires K divisible by 32, got K={value.shape[1]}")
    _require_gpu(value, what)
    _dtype_code(value, what)
    if value.stride(1) != 1 or (value.stride(0) * value.element_size()) % 16:
        value = value.contiguous()
    return value  # a view at an unaligned offset is copied inside the op (not traceable here)


def quantize_dynamic_2d(value: Tensor) -> tuple[Tensor, Tensor]:
    """Per-(row, 32-block) dynamic MXFP8 of ``[rows, K]``: E4M3 values and int8 exponents ``[rows, K/32]``
    (``flashim/quant/formats/mx.py:50-60``)."""
    codes, exponent = library.quantize_mxfp8_dynamic(_dynamic_input(value, "quantize_dynamic_2d"), False)
    return codes.view(torch.float8_e4m3fn), exponent


def quantize_dynamic_swizzled(value: Tensor) -> tuple[Tensor, Tensor]:
    """:func:`quantize_dynamic_2d` with the scales written straight into the swizzled E8M0 layout."""
    codes, swizzled = library.quantize_mxfp8_dynamic(_dynamic_input(value, "quantize_dynamic_swizzled"), True)
    return codes.view(torch.float8_e4m3fn), swizzled.view(torch.float8_e8m0fnu)


def weight_scales_and_values(weight: Tensor) -> tuple[Tensor, Tensor]:
    """Per-output-channel symmetric INT8 of an ``[N, K]`` weight: ``(q, scale)`` with ``scale = safe_scale(amax/127)``
    (``flashim/quant/formats/int8.py:19-27``, as ``StaticInt8Conv2d.from_conv`` uses them)."""
    _require_gpu(weight, "weight_scales")
    _dtype_code(weight, "weight_scales")
    return library.quantize_int8_rows(weight.contiguous(), False)


def quantize_int8_rows(matrix: Tensor) -> tuple[Tensor, Tensor]:
    """Per-row dynamic INT8 of a row-major ``[rows, K]`` matrix (unit column stride, any row stride): ``(q, scale)``
    with ``scale = safe_scale(amax * float32(1 / 127))`` (``flashim/ops/quantize.py:148-154``)."""
    _require_gpu(matrix, "quantize_int8_rows")
    _dtype_code(matrix, "quantize_int8_rows")
    return library.quantize_int8_rows(matrix, True)


def calibrate_block32_exponent(value: Tensor) -> Tensor:
    """One static exponent per padded 32-channel block from the amax over every row (``mx.py:41-47``)."""
    if value.ndim < 2:
        raise ValueError(f"Expected a channelized tensor, got {tuple(value.shape)}")
    _require_gpu(value, "calibrate_block32_exponent")
    _dtype_code(value, "calibrate_block32_exponent")
    matrix = value.reshape(-1, value.shape[-1])
    if matrix.stride(1) != 1:
        matrix = matrix.contiguous()
    return library.calibrate_block32(matrix)


# -- E8M0 layouts (byte permutations) ------------------------------------------------------------------------------


def exponent_to_e8m0(exponent: Tensor) -> Tensor:
    return (exponent.to(torch.int16) + 127).to(torch.uint8).view(torch.float8_e8m0fnu)


def swizzled_size(rows: int, groups: int) -> int:
    return ((rows + 127) // 128) * 128 * ((groups + 3) // 4) * 4


def swizzle_scales(exponent: Tensor) -> Tensor:
    """``[rows, K/32]`` int8 exponents -> cuBLAS 128x4 swizzled E8M0 bytes (``mx.py:67-86``)."""
    if exponent.ndim != 2:
        raise ValueError(f"Expected [rows, groups] exponents, got {tuple(exponent.shape)}")
    scales = exponent_to_e8m0(exponent).view(torch.uint8)
    rows, cols = scales.shape
    padded_rows, padded_cols = ((rows + 127) // 128) * 128, ((cols + 3) // 4) * 4
    if (rows, cols) != (padded_rows, padded_cols):
        padded = torch.zeros((padded_rows, padded_cols), device=scales.device, dtype=torch.uint8)
        padded[:rows, :cols] = scales
        scales = padded
    out = (scales.view(padded_rows // 128, 4, 32, padded_cols // 4, 4)
           .permute(0, 3, 2, 1, 4).reshape(-1).contiguous())
    return out.view(torch.float8_e8m0fnu)


def unswizzle_scales(swizzled: Tensor, rows: int, groups: int) -> Tensor:
    """Inverse of :func:`swizzle_scales`: int8 exponents ``[rows, groups]``."""
    padded_rows, padded_cols = ((rows + 127) // 128) * 128, ((groups + 3) // 4) * 4
    raw = swizzled.view(torch.uint8).reshape(padded_rows // 128, padded_cols // 4, 32, 4, 4)
    dense = raw.permute(0, 3, 2, 1, 4).reshape(padded_rows, padded_cols)[:rows, :groups]
    return (dense.to(torch.int16) - 127).to(torch.int8)


def static_input_scales(exponent: Tensor, rows: int) -> Tensor:
    """A static ``[K/32]`` exponent broadcast over ``rows`` and swizzled (``mx.py:89-95``)."""
    if exponent.ndim != 1:
        raise ValueError("Expected a 1D static block-32 exponent")
    if rows <= 0:
        raise ValueError(f"Expected a positive row count, got {rows}")
    return swizzle_scales(exponent.to(torch.int8).expand(rows, -1))
