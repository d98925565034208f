"""``torch.compile(fullgraph=True)`` traces the HIP impls (custom ops with fakes, flashim_amd.library) and gives the
eager result, the contract of FlashIM's tests/ops/test_depthwise_cuda.py:115-119. Each compiled function runs the op
through this package's dispatcher, as FlashIM's region compile would through its own."""

import pytest
import torch

from flashim_amd import ops, quant
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _same(a, b):
    if isinstance(a, (tuple, list)):
        return all(_same(x, y) for x, y in zip(a, b))
    if isinstance(a, quant.QuantizedTensor):
        return _same(a.values, b.values) and _same(a.scale_exponent, b.scale_exponent)
    if isinstance(a, quant.Int8Tensor):
        return _same(a.values, b.values)
    if a.dtype in (torch.float8_e4m3fn, torch.float8_e8m0fnu):
        a, b = a.view(torch.uint8), b.view(torch.uint8)
    return torch.equal(a, b)


def _check(fn, *args):
    torch._dynamo.reset()
    eager = fn(*args)
    compiled = torch.compile(fn, fullgraph=True)(*args)
    assert _same(compiled, eager)


def test_compile_convs():
    g = torch.Generator().manual_seed(0)
    x = torch.randint(-127, 127, (2, 20, 21, 64), dtype=torch.int8, generator=g).to(DEV)
    w = torch.randint(-127, 127, (96, 9 * 64), dtype=torch.int8, generator=g).to(DEV)
    a_s, w_s, b = torch.tensor(0.02, device=DEV), (torch.rand(96, generator=g) * 0.01).to(DEV), torch.randn(96).to(DEV)
    _check(lambda x: ops.int8_conv2d(x, w, a_s, w_s, b, 3, 3, 1, 1, 1, 1, 1, 1, relu=True), x)
    xb = torch.randn(2, 20, 21, 64, generator=g).to(torch.bfloat16).to(DEV)
    e = ref.calibrate_block32_exponent(xb.float().cpu()).to(DEV)
    wq = quant.QuantizedWeight.from_float((torch.randn(96, 9 * 64, generator=g) * 0.05).to(DEV))

    def mx_block(xb):
        q = ops.quantize_mxfp8(xb, e)
        return ops.mxfp8_conv2d(q.values, e, wq.values, wq.scale_exponent, b, 3, 3, 1, 1, 1, 1, 1, 1, gelu=True)

    _check(mx_block, xb)


def test_compile_quantizers():
    g = torch.Generator().manual_seed(1)
    xb = (torch.randn(2, 13, 17, 96, generator=g) * 3).to(torch.bfloat16).to(DEV)
    e = ref.calibrate_block32_exponent(xb.float().cpu()).to(DEV)
    s = torch.tensor(0.03, device=DEV)
    _check(lambda v: ops.quantize_mxfp8(v, e), xb)
    _check(lambda v: ops.quantize_int8(v, s), xb)
    _check(lambda v: ops.gelu_quantize(v, e), xb)
    _check(lambda v: ops.quantize_mxfp8(v.permute(0, 2, 3, 1), e), xb.permute(0, 3, 1, 2).contiguous())


def test_compile_depthwise_and_blocks():
    g = torch.Generator().manual_seed(2)
    c = 128
    x = (torch.randn(2, c, 24, 40, generator=g) * 2).to(torch.bfloat16).contiguous(
        memory_format=torch.channels_last).to(DEV)
    dw_w = (torch.randn(25, c, generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    dw_b, pw_b = torch.randn(c, generator=g).to(DEV), torch.randn(c, generator=g).to(DEV)
    s = torch.tensor(0.03, device=DEV)
    _check(lambda v: ops.depthwise5x5_relu_mxfp8(v, dw_w, dw_b), x)
    _check(lambda v: ops.depthwise5x5_relu_int8(v, dw_w, dw_b, s), x)
    pw = quant.QuantizedWeight.from_float((torch.randn(c, c, generator=g) * 0.1).to(DEV))
    swz, e8 = quant.swizzle_scales(pw.scale_exponent), quant.exponent_to_e8m0(pw.scale_exponent)
    _check(lambda v: ops.depthwise5x5_relu_pointwise_mxfp8(v, dw_w, dw_b, pw.values, swz, e8, pw_b), x)
    w8 = torch.randint(-127, 128, (c, c), dtype=torch.int8, generator=g).to(DEV)
    ws = (torch.rand(c, generator=g) * 0.01 + 0.001).to(DEV)
    _check(lambda v: ops.depthwise5x5_relu_pointwise_int8(v, dw_w, dw_b, w8, ws, pw_b, s), x)
    pw16 = (torch.randn(c, c, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    _check(lambda v: ops.depthwise5x5_relu_pointwise(v, dw_w, dw_b, pw16, pw_b), x)
