"""``nn.Module`` callers of the path: static INT8 / MXFP8 ``nn.Linear`` and ``nn.Conv2d`` (``groups == 1``), mirroring
FlashIM's ``StaticInt8Linear`` (``flashim/quant/methods/int8_linear.py:14-112``), ``StaticMXFP8Linear``
(``flashim/quant/methods/linear.py:15-140``), ``StaticInt8Conv2d`` and ``StaticMXFP8Conv2d``
(``flashim/quant/methods/conv2d.py:79-254``): same constructors, buffers, ``from_*`` packers and ``forward`` contracts,
computed by this package's ops (HIP only).

Differences, all on the side of doing less work:

* the MXFP8 conv always takes the fused implicit GEMM (``use_fused`` is True): the gfx950 kernel applies the E8M0
  scales inside the block-scaled MFMA, so there is no shape where the im2col + GEMM pipeline wins;
* ``chain_output`` (the conv writes the next conv's quantized input from its epilogue, bit-identical to the separate
  quantize) is on for every gfx950 device.

Weight packing runs on the GPU (the HIP quantizers): pass modules whose weights live on the target device.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from flashim_amd import ops, quant
from flashim_amd.platforms import is_gfx950
from flashim_amd.quant import Int8Tensor, QuantizedTensor, QuantizedWeight

BLOCK = 32
_EPS = torch.finfo(torch.float32).eps


def _pair(value) -> tuple[int, int]:
    return (value, value) if isinstance(value, int) else tuple(value)


def _safe_scale(scale: Tensor) -> Tensor:
    """``flashim/quant/formats/int8.py:13-16``: non-finite or vanishing scales become FP32 eps."""
    scale = scale.float()
    return torch.where(torch.isfinite(scale) & (scale > _EPS), scale, torch.full_like(scale, _EPS))


def _pixels(x: Tensor) -> Tensor:
    """``[B, C, H, W]`` -> its ``[B, H, W, C]`` view (``conv2d.py:53-57``): channels-last memory is packed and
    NCHW-contiguous memory is read in place by the quantizers; other layouts are copied."""
    pixels = x.permute(0, 2, 3, 1)
    return pixels if pixels.is_contiguous() or x.is_contiguous() else pixels.contiguous()


def _geometry(conv: nn.Conv2d) -> dict:
    """``conv2d.py:60-73``: groups == 1, zero padding, ``'same'`` for odd kernels at stride 1."""
    if conv.groups != 1:
        raise ValueError("quantized convolutions must have groups == 1")
    if conv.padding_mode != "zeros":
        raise ValueError("quantized convolutions need zero padding")
    padding = conv.padding
    if padding == "same":
        if any(k % 2 == 0 for k in conv.kernel_size) or _pair(conv.stride) != (1, 1):
            raise ValueError("padding='same' is supported for odd kernels at stride 1")
        padding = tuple(d * (k - 1) // 2 for k, d in zip(conv.kernel_size, _pair(conv.dilation)))
    elif isinstance(padding, str):
        raise ValueError(f"unsupported padding {padding!r}")
    return {"kernel": _pair(conv.kernel_size), "stride": _pair(conv.stride), "padding": _pair(padding),
            "dilation": _pair(conv.dilation)}


def _geometry_args(geometry: dict) -> tuple[int, ...]:
    (kh, kw), (sh, sw), (ph, pw), (dh, dw) = (
        geometry["kernel"], geometry["stride"], geometry["padding"], geometry["dilation"])
    return kh, kw, sh, sw, ph, pw, dh, dw


def _same_scale(a: Tensor, b: Tensor) -> bool:
    return a is b or (a.shape == b.shape and a.device == b.device and bool(torch.equal(a, b)))


# -- INT8 -------------------------------------------------------------------------------------------------------------


class StaticInt8Linear(nn.Module):
    """``nn.Linear`` as an INT8 GEMM: per-output-row weight scales ``amax / 127``, one static activation scale, INT32
    accumulation, ``acc * (s * w_scale) + bias`` in FP32, BF16 out cast to the input dtype."""

    def __init__(self, weight_int8: Tensor, weight_scale: Tensor, bias: Tensor | None, input_scale: Tensor) -> None:
        super().__init__()
        self.out_features, self.in_features = weight_int8.shape
        device = weight_int8.device
        self.register_buffer("weight_int8", weight_int8.contiguous())
        self.register_buffer("weight_scale", weight_scale.to(device=device, dtype=torch.float32))
        self.register_buffer("input_scale", _safe_scale(input_scale.to(device)).reshape(()))
        self.register_buffer("bias", None if bias is None else bias.detach().to(device=device, dtype=torch.bfloat16))

    @classmethod
    def from_linear(cls, linear: nn.Linear, input_scale: Tensor) -> StaticInt8Linear:
        weight = linear.weight.detach()
        if not torch.isfinite(weight).all():
            raise ValueError("Cannot quantize non-finite weights")
        values, scale = quant.weight_scales_and_values(weight)
        return cls(values, scale, None if linear.bias is None else linear.bias.detach(), input_scale)

    def quantize(self, x: Tensor) -> Int8Tensor:
        return ops.quantize_int8(x, self.input_scale)

    def forward_prequantized(self, quantized: Int8Tensor, relu: bool = False) -> Tensor:
        if not _same_scale(quantized.scale, self.input_scale):
            raise ValueError("Prequantized activation uses a different static scale")
        out = ops.int8_linear(quantized.matrix(), self.weight_int8, self.input_scale, self.weight_scale, self.bias,
                              relu=relu)
        return out.reshape(*quantized.logical_shape[:-1], self.out_features)

    def forward(self, x: Tensor) -> Tensor:
        return self.forward_prequantized(self.quantize(x)).to(x.dtype)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, int8"


class StaticInt8Conv2d(StaticInt8Linear):
    """``nn.Conv2d`` as one INT8 implicit GEMM (``ops.int8_conv2d``); ``forward(x, relu=True)`` applies a following
    ReLU in the epilogue, ``residual`` (``[B, Cout, Ho, Wo]``) is added there too."""

    fuses_relu = True

    def __init__(self, weight_int8, weight_scale, bias, input_scale, *, in_channels: int, **geometry) -> None:
        super().__init__(weight_int8, weight_scale, bias, input_scale)
        self.in_channels, self.geometry = in_channels, geometry
        self.chain_output = is_gfx950(weight_int8.device)

    @classmethod
    def from_conv(cls, conv: nn.Conv2d, input_scale: Tensor) -> StaticInt8Conv2d:
        """Weight laid out ``(ky, kx, c)`` (``conv2d.py:92-100``), per-Cout ``amax / 127`` scales."""
        geometry = _geometry(conv)
        weight = conv.weight.detach().permute(0, 2, 3, 1).reshape(conv.out_channels, -1)
        if not torch.isfinite(weight).all():
            raise ValueError("Cannot quantize non-finite weights")
        values, scale = quant.weight_scales_and_values(weight)
        bias = None if conv.bias is None else conv.bias.detach().to(torch.bfloat16)
        return cls(values, scale, bias, input_scale, in_channels=conv.in_channels, **geometry)

    def feeds(self, consumer: nn.Module) -> bool:
        """Whether ``forward(x, quantize_for=consumer)`` may return ``consumer``'s quantized input."""
        return self.chain_output and isinstance(consumer, StaticInt8Conv2d) and consumer.in_channels == self.out_features

    def _quantized_input(self, x: Tensor | Int8Tensor) -> tuple[Int8Tensor, torch.dtype]:
        if isinstance(x, Int8Tensor):
            if not _same_scale(x.scale, self.input_scale):
                raise ValueError("prequantized input was not produced for this layer")
            return x, torch.bfloat16
        return ops.quantize_int8(_pixels(x), self.input_scale), x.dtype

    def forward(self, x: Tensor | Int8Tensor, relu: bool = False, residual: Tensor | None = None,
                quantize_for: nn.Module | None = None) -> Tensor | Int8Tensor:
        """``relu(conv(x) [+ residual])`` (``conv2d.py:109-125``); with ``quantize_for`` (a layer this one
        :meth:`feeds`) the result comes back as that layer's :class:`Int8Tensor` input."""
        q, dtype = self._quantized_input(x)
        chained = quantize_for is not None and dtype == torch.bfloat16 and self.feeds(quantize_for)
        out = ops.int8_conv2d(
            q.values, self.weight_int8, self.input_scale, self.weight_scale, self.bias, *_geometry_args(self.geometry),
            relu=relu, residual=None if residual is None else residual.permute(0, 2, 3, 1),
            **({"out_scale": quantize_for.input_scale} if chained else {}),
        )
        if chained:
            return Int8Tensor(out, quantize_for.input_scale)
        return out.permute(0, 3, 1, 2).to(dtype)

    def pools_into(self, pool: nn.Module, consumer: nn.Module) -> bool:
        """Whether :meth:`forward_pooled` stands for this layer, the 2x2 / stride-2 ``MaxPool2d`` ``pool`` and the
        quantized conv ``consumer`` after it (``conv2d.py:136-145``)."""
        return (
            isinstance(pool, nn.MaxPool2d) and isinstance(consumer, StaticInt8Conv2d)
            and pool.kernel_size in (2, (2, 2)) and pool.stride in (2, (2, 2)) and pool.padding in (0, (0, 0))
            and pool.dilation in (1, (1, 1)) and not pool.ceil_mode and not pool.return_indices
            and consumer.in_channels == self.out_features
        )

    def forward_pooled(self, x: Tensor | Int8Tensor, consumer: StaticInt8Conv2d, relu: bool = False):
        """``(y, consumer's input)``: this layer's output and the quantized 2x2 max pool of it, both from the conv
        (``ops.int8_conv2d_maxpool``; ``conv2d.py:147-157``)."""
        q, dtype = self._quantized_input(x)
        out, pooled = ops.int8_conv2d_maxpool(
            q.values, self.weight_int8, self.input_scale, self.weight_scale, self.bias, *_geometry_args(self.geometry),
            relu=relu, out_scale=consumer.input_scale,
        )
        return out.permute(0, 3, 1, 2).to(dtype), Int8Tensor(pooled, consumer.input_scale)

    def extra_repr(self) -> str:
        return f"{self.in_channels}->{self.out_features}, {self.geometry['kernel']}, int8"


# -- MXFP8 ------------------------------------------------------------------------------------------------------------


class StaticMXFP8Linear(nn.Module):
    """``nn.Linear`` as a block-scaled MXFP8 GEMM: E4M3 weights with one exponent per (row, 32 inputs), activations
    quantized with static per-32-channel exponents; BF16 GEMM result plus BF16 bias, cast to the input dtype."""

    def __init__(self, weight: QuantizedWeight, bias: Tensor | None, input_exponent: Tensor) -> None:
        super().__init__()
        self.in_features, self.out_features = weight.logical_shape[1], weight.logical_shape[0]
        device = weight.values.device
        self.register_buffer("weight_values", weight.values.view(torch.uint8))
        self.register_buffer("weight_exponent", weight.scale_exponent)
        self.register_buffer("input_exponent", input_exponent.to(device=device, dtype=torch.int8))
        self.register_buffer(
            "bias", None if bias is None else F.pad(bias.float().to(device), (0, weight.out_features - bias.shape[0])))
        self.register_buffer("bias_bf16", None if self.bias is None else self.bias.to(torch.bfloat16))
        self._bind()

    def _bind(self) -> None:
        self.gemm = ops.mxfp8_linear.bind(self.packed_weight())

    def _apply(self, fn, recurse: bool = True):
        result = super()._apply(fn, recurse)
        self._bind()
        return result

    @classmethod
    def from_linear(cls, linear: nn.Linear, input_exponent: Tensor) -> StaticMXFP8Linear:
        weight = QuantizedWeight.from_float(linear.weight.detach())
        expected = (weight.in_features // BLOCK,)
        if tuple(input_exponent.shape) != expected:
            raise ValueError(f"Input exponent shape {tuple(input_exponent.shape)} != {expected}")
        return cls(weight, None if linear.bias is None else linear.bias.detach(), input_exponent)

    def packed_weight(self) -> QuantizedWeight:
        return QuantizedWeight(self.weight_values.view(torch.float8_e4m3fn), self.weight_exponent,
                               (self.out_features, self.in_features))

    def _finish(self, out: Tensor, leading: tuple[int, ...], dtype: torch.dtype) -> Tensor:
        """``linear.py:83-86``: the BF16 bias added after the GEMM's rounding, padded columns dropped."""
        if self.bias_bf16 is not None:
            out = out + self.bias_bf16
        return out[:, : self.out_features].reshape(*leading, self.out_features).to(dtype)

    def quantize(self, value: Tensor) -> QuantizedTensor:
        return ops.quantize_mxfp8(value, self.input_exponent)

    def forward_prequantized(self, quantized: QuantizedTensor) -> Tensor:
        if not _same_scale(quantized.scale_exponent, self.input_exponent):
            raise ValueError("Prequantized activation uses a different static scale")
        return self._finish(self.gemm(quantized, None), quantized.logical_shape[:-1], torch.bfloat16)

    def forward(self, x: Tensor) -> Tensor:
        return self._finish(self.gemm(self.quantize(x), None), tuple(x.shape[:-1]), x.dtype)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, mxfp8"


class StaticMXFP8Conv2d(StaticMXFP8Linear):
    """``nn.Conv2d`` as one block-scaled MXFP8 implicit GEMM (``ops.mxfp8_conv2d``); ``channel_exponent`` is per
    padded input-channel block, shared by all taps; the weight keeps one exponent per (Cout, tap, 32 channels)."""

    fuses_relu = True

    def __init__(self, weight: QuantizedWeight, bias, input_exponent, *, in_channels: int, taps: int, **geometry):
        super().__init__(weight, bias, input_exponent.repeat(taps))
        self.in_channels, self.taps, self.geometry = in_channels, taps, geometry
        self.register_buffer("channel_exponent", input_exponent.to(device=weight.values.device, dtype=torch.int8))
        self.use_fused = True
        self.chain_output = is_gfx950(weight.values.device)

    @classmethod
    def from_conv(cls, conv: nn.Conv2d, input_exponent: Tensor) -> StaticMXFP8Conv2d:
        """Input channels padded to 32, weight ``(ky, kx, c)`` then ``QuantizedWeight.from_float`` (``conv2d.py:
        194-205``)."""
        geometry = _geometry(conv)
        cp = quant.padded_channels(conv.in_channels)
        if tuple(input_exponent.shape) != (cp // BLOCK,):
            raise ValueError(f"exponent shape {tuple(input_exponent.shape)} != {(cp // BLOCK,)}")
        w = F.pad(conv.weight.detach().permute(0, 2, 3, 1), (0, cp - conv.in_channels))
        taps = w.shape[1] * w.shape[2]
        return cls(QuantizedWeight.from_float(w.reshape(conv.out_channels, -1)),
                   None if conv.bias is None else conv.bias.detach(), input_exponent,
                   in_channels=conv.in_channels, taps=taps, **geometry)

    def feeds(self, consumer: nn.Module) -> bool:
        return (
            self.chain_output and isinstance(consumer, StaticMXFP8Conv2d) and consumer.in_channels == self.out_features
            and consumer.channel_exponent.shape[0] * BLOCK == self.weight_values.shape[0]
        )

    def forward(self, x: Tensor | QuantizedTensor, relu: bool = False, residual: Tensor | None = None,
                quantize_for: nn.Module | None = None) -> Tensor | QuantizedTensor:
        """``relu(conv(x) [+ residual])`` with ReLU and residual in the epilogue (``conv2d.py:217-251``)."""
        if isinstance(x, QuantizedTensor):
            if not _same_scale(x.scale_exponent, self.channel_exponent):
                raise ValueError("prequantized input was not produced for this layer")
            q, dtype = x, torch.bfloat16
        else:
            q, dtype = ops.quantize_mxfp8(_pixels(x), self.channel_exponent), x.dtype
        chained = quantize_for is not None and dtype == torch.bfloat16 and self.feeds(quantize_for)
        out = ops.mxfp8_conv2d(
            q.values, self.channel_exponent, self.weight_values.view(torch.float8_e4m3fn), self.weight_exponent,
            self.bias_bf16, *_geometry_args(self.geometry), relu=relu,
            residual=None if residual is None else residual.permute(0, 2, 3, 1),
            **({"out_exponent": quantize_for.channel_exponent} if chained else {}),
        )
        if chained:
            return QuantizedTensor(out, quantize_for.channel_exponent, (*out.shape[:-1], self.out_features))
        return out[..., : self.out_features].to(dtype).permute(0, 3, 1, 2)

    def extra_repr(self) -> str:
        return f"{self.in_channels}->{self.out_features}, {self.geometry['kernel']}, mxfp8"
