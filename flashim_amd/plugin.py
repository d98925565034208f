"""Registration into an installed FlashIM: the ``flashim.backends`` entry point (``flashim/backends/_loader.py:63-70``
calls the loaded object) points here.

For each op this backend implements, ``register()`` adds an impl named ``"hip"`` to FlashIM's own op object
(``ops.<op>.register(name, device=DeviceSpec("rocm"), priority=..., when=...)``, ``flashim/ops/_registry.py:185-210``)
with the torch reference's signature. FlashIM's ROCm platform carries no gfx950 ISA features
(``flashim/platforms/others.py:16-30``), so the ``when`` predicates check the architecture (gfx950) and that the HIP
library is built; on any other call FlashIM's own torch reference stays the fallback, unchanged. Results are returned as
FlashIM's container types (``flashim.quant.tensor.QuantizedTensor`` / ``Int8Tensor``), which share this package's
field layout.
"""

from __future__ import annotations

import importlib
import logging
from collections.abc import Callable

import torch

from flashim_amd import _lib
from flashim_amd.backends.hip import conv as _conv
from flashim_amd.backends.hip import gemm as _gemm
from flashim_amd.backends.hip import quantize as _quantize

logger = logging.getLogger(__name__)

HIP = "hip"
PRIORITY = 2  # above FlashIM's NVIDIA-only impls, which never match "rocm" anyway

REGISTERED: list[str] = []


@torch.compiler.assume_constant_result  # a process constant: keeps FlashIM's dispatch traceable under torch.compile
def _available() -> bool:
    return _lib.available()


def _guard(when: Callable[..., bool]) -> Callable[..., bool]:
    def predicate(*args, **kwargs) -> bool:
        return _available() and bool(when(*args, **kwargs))

    return predicate


def _adapt_quantized(upstream_tensor_module):
    def quantize_mxfp8(value, scale_exponent):
        q = _quantize.quantize_mxfp8(value, scale_exponent)
        return upstream_tensor_module.QuantizedTensor(q.values, q.scale_exponent, q.logical_shape)

    def quantize_int8(value, scale, *, channel_scale=None):
        q = _quantize.quantize_int8(value, scale, channel_scale=channel_scale)
        return upstream_tensor_module.Int8Tensor(q.values, q.scale)

    def gelu_quantize(value, scale_exponent, approximate="none", *, input_bias=None):
        q = _quantize.gelu_quantize(value, scale_exponent, approximate, input_bias=input_bias)
        return upstream_tensor_module.QuantizedTensor(q.values, q.scale_exponent, q.logical_shape)

    def gelu_quantize_int8(value, scale, approximate="none"):
        q = _quantize.gelu_quantize_int8(value, scale, approximate)
        return upstream_tensor_module.Int8Tensor(q.values, q.scale)

    return quantize_mxfp8, quantize_int8, gelu_quantize, gelu_quantize_int8


def _as_local(activation, weight):
    """FlashIM's ``QuantizedTensor`` / ``QuantizedWeight`` share this package's field layout: re-wrap without copying."""
    from flashim_amd import quant

    act = quant.QuantizedTensor(activation.values, activation.scale_exponent, tuple(activation.logical_shape))
    wgt = quant.QuantizedWeight(weight.values, weight.scale_exponent, tuple(weight.logical_shape))
    return act, wgt


def _mxfp8_linear(activation, bias, weight):
    act, wgt = _as_local(activation, weight)
    return _gemm.mxfp8_linear(act, bias, wgt)


def _eligible_mxfp8_linear(activation, bias, weight) -> bool:
    try:
        act, wgt = _as_local(activation, weight)
    except (AttributeError, ValueError, TypeError):
        return False
    return _gemm.eligible_mxfp8_linear(act, bias, wgt)


def _as_local_weight(weight):
    from flashim_amd import quant

    return quant.QuantizedWeight(weight.values, weight.scale_exponent, tuple(weight.logical_shape))


def _mxfp8_gelu_mlp(x, w1, b1, hidden_exponent, w2):
    act, lw1 = _as_local(x, w1)
    return _gemm.mxfp8_gelu_mlp(act, lw1, b1, hidden_exponent, _as_local_weight(w2))


def _eligible_mxfp8_gelu_mlp(x, w1, b1, hidden_exponent, w2) -> bool:
    try:
        act, lw1 = _as_local(x, w1)
        lw2 = _as_local_weight(w2)
    except (AttributeError, ValueError, TypeError):
        return False
    return _gemm.eligible_mxfp8_gelu_mlp(act, lw1, b1, hidden_exponent, lw2)


def _adapt_stem(upstream_tensor_module):
    def conv2d_small_cin_quantize_int8(x, scale, packed, bias):
        q = _conv.conv2d_small_cin_quantize_int8(x, scale, packed, bias)
        return upstream_tensor_module.Int8Tensor(q.values, q.scale)

    def bias_relu_quantize_int8(raw, bias, scale):
        q = _conv.bias_relu_quantize_int8(raw, bias, scale)
        return upstream_tensor_module.Int8Tensor(q.values, q.scale)

    return conv2d_small_cin_quantize_int8, bias_relu_quantize_int8


def impls(upstream_tensor_module) -> dict[str, tuple[Callable, Callable]]:
    """``{op name: (impl, when)}`` for the FlashIM ops this backend replaces."""
    quantize_mxfp8, quantize_int8, gelu_quantize, gelu_quantize_int8 = _adapt_quantized(upstream_tensor_module)
    _, bias_relu_quantize_int8 = _adapt_stem(upstream_tensor_module)
    return {
        "quantize_mxfp8": (quantize_mxfp8, _quantize.eligible_quantize_mxfp8),
        "quantize_int8": (quantize_int8, _quantize.eligible_quantize_int8),
        "quantize_int8_rows": (_quantize.quantize_int8_rows, _quantize.eligible_quantize_int8_rows),
        "gelu_quantize": (gelu_quantize, _quantize.eligible_gelu_quantize),
        "gelu_quantize_int8": (gelu_quantize_int8, _quantize.eligible_gelu_quantize_int8),
        "int8_conv2d": (_conv.int8_conv2d, _conv.eligible_int8_conv2d),
        "mxfp8_conv2d": (_conv.mxfp8_conv2d, _conv.eligible_mxfp8_conv2d),
        "depthwise5x5_relu_mxfp8": (_conv.depthwise5x5_relu_mxfp8, _conv.eligible_depthwise),
        "depthwise5x5_relu_int8": (_conv.depthwise5x5_relu_int8, _conv.eligible_depthwise),
        "depthwise5x5_relu_pointwise": (_conv.depthwise5x5_relu_pointwise, _conv.eligible_pointwise_bf16),
        "depthwise5x5_relu_pointwise_mxfp8": (_conv.depthwise5x5_relu_pointwise_mxfp8,
                                              _conv.eligible_pointwise_mxfp8),
        "depthwise5x5_relu_pointwise_int8": (_conv.depthwise5x5_relu_pointwise_int8, _conv.eligible_pointwise_int8),
        "im2col_gather": (_conv.im2col_gather, _conv.eligible_im2col),
        "int8_conv2d_maxpool": (_conv.int8_conv2d_maxpool, _conv.eligible_int8_conv2d_maxpool),
        "int8_linear": (_gemm.int8_linear, _gemm.eligible_int8_linear),
        "int8_linear_quantize": (_gemm.int8_linear_quantize, _gemm.eligible_int8_linear_quantize),
        "mxfp8_scaled_mm": (_gemm.mxfp8_scaled_mm, _gemm.eligible_mxfp8_scaled_mm),
        "mxfp8_linear": (_mxfp8_linear, _eligible_mxfp8_linear),
        "mxfp8_gelu_mlp": (_mxfp8_gelu_mlp, _eligible_mxfp8_gelu_mlp),
        "bias_relu_quantize_int8": (bias_relu_quantize_int8, _conv.eligible_bias_relu_quantize),
    }


# ops whose impl packs its weights once per bind: {op name: (impl, when, accepts, prepare)}
def prepared_impls(upstream_tensor_module) -> dict[str, tuple[Callable, Callable, Callable, Callable]]:
    conv2d_small_cin_quantize_int8, _ = _adapt_stem(upstream_tensor_module)
    return {
        "conv2d_small_cin_quantize_int8": (conv2d_small_cin_quantize_int8, _conv.eligible_small_cin,
                                           _conv.accepts_small_cin, _conv.small_cin_prepare),
    }


def register(flashim_ops=None, flashim_registry=None, flashim_tensor=None) -> list[str]:
    """Register the HIP impls into FlashIM (modules injectable for tests). Returns the op names registered."""
    flashim_ops = flashim_ops or importlib.import_module("flashim.ops")
    flashim_registry = flashim_registry or importlib.import_module("flashim.ops._registry")
    flashim_tensor = flashim_tensor or importlib.import_module("flashim.quant.tensor")
    device = flashim_registry.DeviceSpec("rocm")
    done = []
    for name, (fn, when) in impls(flashim_tensor).items():
        op = getattr(flashim_ops, name, None)
        if op is None:
            logger.info("FlashIM has no op %s; skipped", name)
            continue
        if any(impl.name == HIP for impl in getattr(op, "impls", [])):
            continue
        op.register(HIP, device=device, priority=PRIORITY, when=_guard(when))(fn)
        done.append(name)
    for name, (fn, when, accepts, prepare) in prepared_impls(flashim_tensor).items():
        op = getattr(flashim_ops, name, None)
        if op is None:
            logger.info("FlashIM has no op %s; skipped", name)
            continue
        if any(impl.name == HIP for impl in getattr(op, "impls", [])):
            continue
        op.register(HIP, device=device, priority=PRIORITY, when=_guard(when), accepts=accepts, prepare=prepare)(fn)
        done.append(name)
    REGISTERED.extend(done)
    return done
