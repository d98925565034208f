"""The FlashIM plugin registration (``flashim_amd.plugin``) against a minimal, independent stand-in of the three FlashIM
modules it touches: an op object exposing ``register(name, *, device, requires=(), priority=0, when=None,
prepare=None, accepts=None)`` (the contract of ``flashim/ops/_registry.py:185-210``) and ``impls``, a ``DeviceSpec``
constructor, and the two container dataclasses of ``flashim/quant/tensor.py``. Checks the impl name, device key and
priority, the guarded ``when`` predicates (CPU tensors are refused so FlashIM's reference runs), idempotence and the
container adaptation. FlashIM itself is not imported and none of this package's dispatcher is used."""

import types
from dataclasses import dataclass

import torch

from flashim_amd import plugin


@dataclass(frozen=True)
class _Device:
    type: str


@dataclass
class _Registered:
    name: str
    fn: object
    device: _Device
    priority: int
    when: object
    prepare: object
    accepts: object


class _StubOp:
    def __init__(self, name):
        self.name, self.impls = name, []

    def register(self, name, *, device, requires=(), priority=0, when=None, prepare=None, accepts=None):
        def add(fn):
            self.impls.append(_Registered(name, fn, device, priority, when, prepare, accepts))
            return fn
        return add


OP_NAMES = ("quantize_mxfp8", "quantize_int8", "quantize_int8_rows", "gelu_quantize", "gelu_quantize_int8", "int8_conv2d", "mxfp8_conv2d",
            "depthwise5x5_relu_mxfp8", "depthwise5x5_relu_int8", "depthwise5x5_relu_pointwise",
            "depthwise5x5_relu_pointwise_mxfp8",
            "depthwise5x5_relu_pointwise_int8", "im2col_gather", "int8_conv2d_maxpool", "int8_linear",
            "int8_linear_quantize", "mxfp8_scaled_mm", "mxfp8_linear", "mxfp8_gelu_mlp", "bias_relu_quantize_int8",
            "conv2d_small_cin_quantize_int8")


def _stub_flashim(missing=()):
    ops = types.SimpleNamespace(**{n: _StubOp(n) for n in OP_NAMES if n not in missing})
    registry = types.SimpleNamespace(DeviceSpec=_Device)

    @dataclass(frozen=True)
    class QuantizedTensor:
        values: torch.Tensor
        scale_exponent: torch.Tensor
        logical_shape: tuple

    @dataclass(frozen=True)
    class Int8Tensor:
        values: torch.Tensor
        scale: torch.Tensor

    return ops, registry, types.SimpleNamespace(QuantizedTensor=QuantizedTensor, Int8Tensor=Int8Tensor)


def test_plugin_registers_hip_impls_for_rocm():
    ops, reg, tensor = _stub_flashim()
    done = plugin.register(ops, reg, tensor)
    assert set(done) == set(OP_NAMES)
    for name in done:
        (impl,) = getattr(ops, name).impls
        assert impl.name == "hip" and impl.device == _Device("rocm") and impl.priority == plugin.PRIORITY
    stem = ops.conv2d_small_cin_quantize_int8.impls[0]
    assert stem.prepare is not None and stem.accepts is not None
    assert plugin.register(ops, reg, tensor) == []  # registering twice is a no-op
    # CPU tensors: the guarded predicate refuses, so FlashIM would run its reference
    x = torch.randint(-127, 127, (1, 4, 4, 16), dtype=torch.int8)
    w = torch.randint(-127, 127, (8, 144), dtype=torch.int8)
    when = ops.int8_conv2d.impls[0].when
    assert not when(x, w, torch.tensor(0.1), torch.ones(8), None, 3, 3, 1, 1, 1, 1, 1, 1)
    assert not ops.gelu_quantize.impls[0].when(torch.randn(4, 32), torch.zeros(1, dtype=torch.int8))


def test_plugin_skips_ops_flashim_lacks():
    ops, reg, tensor = _stub_flashim(missing=("gelu_quantize", "int8_linear_quantize"))
    done = plugin.register(ops, reg, tensor)
    assert "gelu_quantize" not in done and "int8_conv2d" in done


def test_plugin_adapts_containers(monkeypatch):
    _, _, tensor = _stub_flashim()
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
