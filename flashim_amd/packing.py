"""Weight packing for the implicit-GEMM convs, on the GPU quantizers: what FlashIM's static conv layers do once at load
time (``flashim/quant/methods/conv2d.py:92-100`` for INT8, ``:194-205`` for MXFP8), written as plain functions so a
caller holding an ``nn.Conv2d`` (FlashIM's own layers, which call ``ops.*`` and are unchanged by this backend, or a
standalone user) gets the operands ``ops.int8_conv2d`` / ``ops.mxfp8_conv2d`` take.

Layout: the GEMM's K index runs over (ky, kx, c) with c fastest, because the activations are NHWC and each tap reads a
contiguous channel run. For MXFP8 every tap's channel run is padded to 32 so each E8M0 block covers channels of one tap.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from flashim_amd import quant


def kykxc_matrix(weight: Tensor, channel_multiple: int = 1) -> Tensor:
    """``[Cout, Cin, kh, kw]`` -> ``[Cout, kh * kw * Cp]`` with K in (ky, kx, c) order, ``Cp`` = ``Cin`` rounded up to
    ``channel_multiple`` (zero channels)."""
    cout, cin, kh, kw = weight.shape
    cp = -(-cin // channel_multiple) * channel_multiple
    taps = weight.detach().permute(0, 2, 3, 1)  # [Cout, kh, kw, Cin]
    if cp != cin:
        taps = F.pad(taps, (0, cp - cin))
    return taps.reshape(cout, kh * kw * cp)


def pack_int8_conv(weight: Tensor) -> tuple[Tensor, Tensor]:
    """INT8 operands of a conv weight: codes ``[Cout, kh*kw*Cin]`` and per-output-channel FP32 scales
    ``safe_scale(amax / 127)``."""
    return quant.weight_scales_and_values(kykxc_matrix(weight).float())


def pack_mxfp8_conv(weight: Tensor) -> quant.QuantizedWeight:
    """MXFP8 operands of a conv weight: E4M3 ``[Npad, kh*kw*Cp]`` with one exponent per (output channel, 32 inputs),
    ``Cp`` = ``Cin`` rounded up to 32 per tap."""
    return quant.QuantizedWeight.from_float(kykxc_matrix(weight, quant.BLOCK).float())


def conv_geometry(conv: nn.Conv2d) -> tuple[int, int, int, int, int, int, int, int]:
    """``(kh, kw, sh, sw, ph, pw, dh, dw)`` of a groups-1, zero-padded ``nn.Conv2d``; ``padding='same'`` resolves to
    ``dilation * (k - 1) / 2`` per side (odd kernels, stride 1 only, as the implicit GEMM pads symmetrically)."""
    if conv.groups != 1 or conv.padding_mode != "zeros":
        raise ValueError("the implicit-GEMM convs take groups == 1 with zero padding")
    (kh, kw), (sh, sw), (dh, dw) = conv.kernel_size, conv.stride, conv.dilation
    if conv.padding == "same":
        if kh % 2 == 0 or kw % 2 == 0 or (sh, sw) != (1, 1):
            raise ValueError("padding='same' needs odd kernels and stride 1")
        ph, pw = dh * (kh - 1) // 2, dw * (kw - 1) // 2
    elif isinstance(conv.padding, str):
        raise ValueError(f"padding {conv.padding!r} is not supported")
    else:
        ph, pw = conv.padding
    return kh, kw, sh, sw, ph, pw, dh, dw
