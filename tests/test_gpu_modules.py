"""The module callers (``StaticInt8Conv2d`` / ``StaticMXFP8Conv2d`` / the static linears, flashim/quant/methods/
conv2d.py:79-254) on the HIP ops vs the oracle: weight packing bit-exact, INT8 forward bit-exact, MXFP8 forward within
the MXFP8 tolerance, and the chaining contracts of tests/quant/test_conv2d.py:79-125 (the chained quantized output is
byte-identical to quantizing the BF16 output separately; the pooled output to pooling then quantizing)."""

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from flashim_amd import ops
from flashim_amd.modules import StaticInt8Conv2d, StaticInt8Linear, StaticMXFP8Conv2d, StaticMXFP8Linear
from flashim_amd.quant import Int8Tensor, QuantizedTensor
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _conv(cin, cout, k, stride=1, padding=1, dilation=1, bias=True, seed=0):
    torch.manual_seed(seed)
    conv = nn.Conv2d(cin, cout, k, stride=stride, padding=padding, dilation=dilation, bias=bias)
    with torch.no_grad():
        conv.weight.mul_(3)
    return conv


def _x(b, c, h, w, seed=1, channels_last=False):
    torch.manual_seed(seed)
    x = torch.randn(b, c, h, w).to(torch.bfloat16)
    return x.contiguous(memory_format=torch.channels_last) if channels_last else x


def _assert_mx_close(fast, want):
    fast, want = fast.float(), want.float()
    rms = want.pow(2).mean().sqrt()
    assert (fast - want).norm() / want.norm() <= 1e-3
    assert ((fast - want).abs() <= torch.maximum(1e-2 * rms, want.abs() * 2**-7)).all()


def _int8_reference(conv, scale, x, relu=False, residual=None):
    """conv2d.py:92-125 restated on the oracle: pack, quantize the NHWC view, int8_conv2d, back to NCHW."""
    w = conv.weight.detach().float().permute(0, 2, 3, 1).reshape(conv.out_channels, -1)
    w_scale = ref.weight_scales(w)
    wq = ref.quantize_symmetric(w, w_scale[:, None])
    bias = None if conv.bias is None else conv.bias.detach().to(torch.bfloat16)
    q = ref.quantize_int8(x.permute(0, 2, 3, 1), scale)
    geo = (*conv.kernel_size, *conv.stride, *conv.padding, *conv.dilation)
    out = ref.int8_conv2d(q, wq, scale, w_scale, bias, *geo, relu=relu,
                          residual=None if residual is None else residual.permute(0, 2, 3, 1))
    return wq, w_scale, out.permute(0, 3, 1, 2).to(x.dtype)


@pytest.mark.parametrize("cin,cout,k,stride,padding,dilation", [
    (16, 32, 3, 1, 1, 1), (64, 64, 3, 2, 1, 1), (24, 40, 5, 1, 2, 1), (32, 32, 3, 1, 2, 2), (3, 16, 7, 2, 3, 1)])
@pytest.mark.parametrize("channels_last", [False, True])
def test_static_int8_conv2d_bit_exact(cin, cout, k, stride, padding, dilation, channels_last):
    conv = _conv(cin, cout, k, stride, padding, dilation)
    scale = torch.tensor(0.021)
    x = _x(2, cin, 19, 22, channels_last=channels_last)
    layer = StaticInt8Conv2d.from_conv(conv.to(DEV), scale.to(DEV))
    wq, w_scale, want = _int8_reference(conv.cpu(), scale, x)
    assert torch.equal(layer.weight_int8.cpu(), wq) and torch.equal(layer.weight_scale.cpu(), w_scale)
    got = layer(x.to(DEV)).cpu()
    assert got.shape == want.shape and got.dtype == torch.bfloat16
    assert torch.equal(got, want)
    assert torch.equal(layer(x.to(DEV), relu=True).cpu(), F.relu(want))


def test_static_int8_conv2d_residual_chain_and_pool():
    conv1, conv2 = _conv(32, 64, 3, seed=2), _conv(64, 64, 3, seed=3)
    s1, s2 = torch.tensor(0.02), torch.tensor(0.05)
    l1 = StaticInt8Conv2d.from_conv(conv1.to(DEV), s1.to(DEV))
    l2 = StaticInt8Conv2d.from_conv(conv2.to(DEV), s2.to(DEV))
    x = _x(2, 32, 24, 30, seed=4).to(DEV)
    residual = _x(2, 64, 24, 30, seed=5).to(DEV)
    # residual + ReLU in the epilogue: the reference's relu(out + residual) in FP32 after out's BF16 rounding
    _, _, want = _int8_reference(conv1.cpu(), s1, x.cpu(), relu=True, residual=residual.cpu())
    assert torch.equal(l1(x, relu=True, residual=residual).cpu(), want)
    assert l1.feeds(l2) and not l2.feeds(l1)
    # chaining: the epilogue's INT8 output == quantizing the BF16 output; the consumer accepts it
    y = l1(x, relu=True)
    chained = l1(x.to(torch.bfloat16), relu=True, quantize_for=l2)
    assert isinstance(chained, Int8Tensor)
    assert torch.equal(chained.values, ops.quantize_int8(y.permute(0, 2, 3, 1), l2.input_scale).values)
    assert torch.equal(l2(chained).cpu(), l2(y).cpu())
    # pooled: (output, quantize(max_pool2d(output)))
    pool = nn.MaxPool2d(2)
    assert l1.pools_into(pool, l2)
    out, pooled = l1.forward_pooled(x, l2, relu=True)
    assert torch.equal(out, y)
    want_pooled = ops.quantize_int8(F.max_pool2d(y.float(), 2).to(torch.bfloat16).permute(0, 2, 3, 1),
                                    l2.input_scale).values
    assert torch.equal(pooled.values, want_pooled)


def _mx_reference(conv, exponent, x):
    cp = ref.padded_channels(conv.in_channels)
    w = F.pad(conv.weight.detach().permute(0, 2, 3, 1), (0, cp - conv.in_channels)).reshape(conv.out_channels, -1)
    wv, we = ref.quantized_weight_from_float(w)
    bias = None if conv.bias is None else F.pad(conv.bias.detach().float(), (0, wv.shape[0] - conv.out_channels))
    q = ref.quantize_mxfp8(x.permute(0, 2, 3, 1), exponent)
    geo = (*conv.kernel_size, *conv.stride, *conv.padding, *conv.dilation)
    out = ref.mxfp8_conv2d(q, exponent, wv, we, None if bias is None else bias.to(torch.bfloat16), *geo)
    return wv, we, out[..., : conv.out_channels].permute(0, 3, 1, 2)


@pytest.mark.parametrize("cin,cout,k,stride,padding", [(32, 64, 3, 1, 1), (64, 48, 1, 1, 0), (40, 32, 3, 2, 1)])
def test_static_mxfp8_conv2d(cin, cout, k, stride, padding):
    conv = _conv(cin, cout, k, stride, padding, seed=cin)
    x = _x(2, cin, 18, 21, seed=cin + 1)
    exponent = ref.calibrate_block32_exponent(x.permute(0, 2, 3, 1).reshape(-1, cin).float())
    layer = StaticMXFP8Conv2d.from_conv(conv.to(DEV), exponent.to(DEV))
    wv, we, want = _mx_reference(conv.cpu(), exponent, x)
    assert torch.equal(layer.weight_values.cpu(), wv.view(torch.uint8)) and torch.equal(layer.weight_exponent.cpu(), we)
    got = layer(x.to(DEV)).cpu()
    assert got.shape == want.shape
    _assert_mx_close(got, want)


def test_static_mxfp8_conv2d_chain():
    conv1, conv2 = _conv(64, 64, 3, seed=7), _conv(64, 64, 3, seed=8)
    x = _x(1, 64, 20, 20, seed=9)
    e1 = ref.calibrate_block32_exponent(x.permute(0, 2, 3, 1).reshape(-1, 64).float())
    e2 = torch.full((2,), -3, dtype=torch.int8)
    l1 = StaticMXFP8Conv2d.from_conv(conv1.to(DEV), e1.to(DEV))
    l2 = StaticMXFP8Conv2d.from_conv(conv2.to(DEV), e2.to(DEV))
    assert l1.feeds(l2)
    y = l1(x.to(DEV), relu=True)
    chained = l1(x.to(DEV), relu=True, quantize_for=l2)
    assert isinstance(chained, QuantizedTensor)
    want = ops.quantize_mxfp8(y.permute(0, 2, 3, 1), l2.channel_exponent).values
    assert torch.equal(chained.values.view(torch.uint8), want.view(torch.uint8))
    assert torch.equal(l2(chained).cpu(), l2(y).cpu())


def test_static_linears():
    torch.manual_seed(11)
    lin = nn.Linear(96, 80).to(DEV)
    x = torch.randn(3, 50, 96, device=DEV).to(torch.bfloat16)
    scale = x.float().abs().amax() / 127
    layer = StaticInt8Linear.from_linear(lin, scale)
    w = lin.weight.detach().cpu()
    ws = ref.weight_scales(w)
    want = ref.int8_linear(ref.quantize_int8(x.cpu(), scale.cpu()).reshape(-1, 96), ref.quantize_symmetric(w, ws[:, None]),
                           layer.input_scale.cpu(), ws, lin.bias.detach().cpu().to(torch.bfloat16))
    assert torch.equal(layer(x).cpu(), want.reshape(3, 50, 80))
    exponent = ref.calibrate_block32_exponent(x.reshape(-1, 96).float().cpu())
    mx = StaticMXFP8Linear.from_linear(lin, exponent.to(DEV))
    wv, we = ref.quantized_weight_from_float(w)
    out = ref.mxfp8_linear(ref.quantize_mxfp8(x.cpu(), exponent), exponent, None, wv, we)
    want = (out + F.pad(lin.bias.detach().cpu().float(), (0, wv.shape[0] - 80)).to(torch.bfloat16))[:, :80]
    _assert_mx_close(mx(x).cpu().reshape(-1, 80), want)
