"""The FlashIM plugin registration (flashim_amd.plugin) against a stand-in of FlashIM's op / registry / container API
(this package's registry has FlashIM's register() signature): impl names, device key, the guarded predicates and the
container adaptation. FlashIM itself is not imported."""

import types
from dataclasses import dataclass

import torch

from flashim_amd import plugin, registry


def _stub_flashim():
    ops = types.SimpleNamespace()
    for name in ("quantize_mxfp8", "quantize_int8", "int8_conv2d", "mxfp8_conv2d", "depthwise5x5_relu_mxfp8",
                 "depthwise5x5_relu_int8", "depthwise5x5_relu_pointwise_mxfp8", "depthwise5x5_relu_pointwise_int8",
                 "im2col_gather", "int8_conv2d_maxpool", "int8_linear", "mxfp8_scaled_mm", "mxfp8_linear",
                 "mxfp8_gelu_mlp", "bias_relu_quantize_int8"):
        registry.OPS.pop("stub_" + name, None)
        setattr(ops, name, registry.Op("stub_" + name, lambda *a, **k: "reference"))
    registry.OPS.pop("stub_conv2d_small_cin_quantize_int8", None)
    ops.conv2d_small_cin_quantize_int8 = registry.Op("stub_conv2d_small_cin_quantize_int8", lambda *a, **k: "reference",
                                                     composite=True, weights=2)

    @dataclass(frozen=True)
    class QuantizedTensor:
        values: torch.Tensor
        scale_exponent: torch.Tensor
        logical_shape: tuple

    @dataclass(frozen=True)
    class Int8Tensor:
        values: torch.Tensor
        scale: torch.Tensor

    tensor = types.SimpleNamespace(QuantizedTensor=QuantizedTensor, Int8Tensor=Int8Tensor)
    return ops, registry, tensor


def test_plugin_registers_hip_impls_for_rocm():
    ops, reg, tensor = _stub_flashim()
    done = plugin.register(ops, reg, tensor)
    assert set(done) == {"quantize_mxfp8", "quantize_int8", "int8_conv2d", "mxfp8_conv2d",
                         "depthwise5x5_relu_mxfp8", "depthwise5x5_relu_int8", "depthwise5x5_relu_pointwise_mxfp8",
                         "depthwise5x5_relu_pointwise_int8", "im2col_gather", "int8_conv2d_maxpool", "int8_linear", "mxfp8_scaled_mm",
                         "mxfp8_linear", "mxfp8_gelu_mlp", "bias_relu_quantize_int8", "conv2d_small_cin_quantize_int8"}
    for name in done:
        impl = getattr(ops, name).impls[-1]
        assert impl.name == "hip" and impl.device == reg.DeviceSpec("rocm") and impl.priority == plugin.PRIORITY
    # registering twice is a no-op
    assert plugin.register(ops, reg, tensor) == []
    # CPU tensors: the guarded predicate rejects, FlashIM's reference runs
    x = torch.randint(-127, 127, (1, 4, 4, 16), dtype=torch.int8)
    w = torch.randint(-127, 127, (8, 144), dtype=torch.int8)
    assert ops.int8_conv2d(x, w, torch.tensor(0.1), torch.ones(8), None, 3, 3, 1, 1, 1, 1, 1, 1) == "reference"
    assert ops.int8_conv2d.get("hip")(x, w, torch.tensor(0.1), torch.ones(8), None, 3, 3, 1, 1, 1, 1, 1, 1) == "reference"


def test_plugin_adapts_containers(monkeypatch):
    ops, reg, tensor = _stub_flashim()
    from flashim_amd import quant
    from flashim_amd.backends.hip import quantize as hq

    monkeypatch.setattr(hq, "quantize_mxfp8", lambda v, e: quant.QuantizedTensor(
        torch.zeros(2, 32, dtype=torch.float8_e4m3fn), e, (2, 30)))
    monkeypatch.setattr(hq, "quantize_int8", lambda v, s, channel_scale=None: quant.Int8Tensor(
        torch.zeros(2, 3, dtype=torch.int8), s))
    fns = plugin.impls(tensor)
    q = fns["quantize_mxfp8"][0](torch.zeros(2, 30), torch.zeros(1, dtype=torch.int8))
    assert isinstance(q, tensor.QuantizedTensor) and q.logical_shape == (2, 30)
    i8 = fns["quantize_int8"][0](torch.zeros(2, 3), torch.tensor(1.0))
    assert isinstance(i8, tensor.Int8Tensor)
