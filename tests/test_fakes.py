"""The ``torch.library`` fakes of every HIP impl (``flashim_amd.library``), checked on the CPU: each impl runs under
``FakeTensorMode`` on fake ``cuda`` tensors (no kernel runs, no GPU is needed) and its outputs must have the shapes and
dtypes the oracle's real outputs have for the same inputs. This is what ``torch.compile`` sees when it traces the ops
(FlashIM's CUDA backend registers the same kind of fakes, ``flashim/backends/cuda/conv.py:73-76``)."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from flashim_amd import quant
from flashim_amd.backends.hip import conv as hc
from flashim_amd.backends.hip import gemm as hg
from flashim_amd.backends.hip import quantize as hq
from oracle import reference as ref

GEO = (3, 3, 2, 1, 1, 1, 1, 1)


def _fake_run(fn, *args, **kwargs):
    """``fn`` on fake cuda copies of ``args`` -> the outputs' (shape, dtype) structure."""
    mode = FakeTensorMode(allow_non_fake_inputs=False)

    def fake(v):
        if isinstance(v, torch.Tensor):
            return mode.from_tensor(v).to("cuda")
        return v

    with mode:
        out = fn(*[fake(a) for a in args], **{k: fake(v) for k, v in kwargs.items()})
    return _sig(out)


def _sig(out):
    if isinstance(out, torch.Tensor):
        return tuple(out.shape), out.dtype
    if isinstance(out, (tuple, list)):
        return tuple(_sig(o) for o in out)
    if isinstance(out, quant.QuantizedTensor):
        return _sig(out.values), _sig(out.scale_exponent)
    if isinstance(out, quant.Int8Tensor):
        return _sig(out.values)
    raise TypeError(type(out))


def _sig_mx(values):
    return tuple(values.shape), values.dtype


@pytest.fixture(autouse=True)
def _cuda_device_is_visible(monkeypatch):
    """Fake cuda tensors need no GPU, but a few torch calls ask for a current device index."""
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)


def test_conv_fakes_match_oracle_shapes():
    x = torch.randint(-127, 127, (2, 9, 11, 32), dtype=torch.int8)
    w = torch.randint(-127, 127, (48, 9 * 32), dtype=torch.int8)
    a_s, w_s, bias = torch.tensor(0.02), torch.rand(48), torch.randn(48)
    want = ref.int8_conv2d(x, w, a_s, w_s, bias, *GEO)
    assert _fake_run(hc.int8_conv2d, x, w, a_s, w_s, bias, *GEO) == _sig(want)
    want_q = ref.int8_conv2d(x, w, a_s, w_s, bias, *GEO, out_scale=torch.tensor(0.1))
    assert _fake_run(hc.int8_conv2d, x, w, a_s, w_s, bias, *GEO, out_scale=torch.tensor(0.1)) == _sig(want_q)
    geo1 = (3, 3, 1, 1, 1, 1, 1, 1)
    want_p = ref.int8_conv2d_maxpool(x, w, a_s, w_s, bias, *geo1, out_scale=torch.tensor(0.1))
    assert _fake_run(hc.int8_conv2d_maxpool, x, w, a_s, w_s, bias, *geo1, out_scale=torch.tensor(0.1)) == \
        _sig(want_p)
    xm = torch.randn(2, 9, 11, 64).to(torch.float8_e4m3fn)
    e = torch.zeros(2, dtype=torch.int8)
    wm = torch.randn(40, 9 * 64).to(torch.float8_e4m3fn)
    we = torch.zeros(40, 18, dtype=torch.int8)
    want_m = ref.mxfp8_conv2d(xm, e, wm, we, None, *GEO)
    assert _fake_run(hc.mxfp8_conv2d, xm, e, wm, we, None, *GEO) == _sig(want_m)
    wm2 = torch.randn(64, 9 * 64).to(torch.float8_e4m3fn)
    we2 = torch.zeros(64, 18, dtype=torch.int8)
    want_m2 = ref.mxfp8_conv2d(xm, e, wm2, we2, None, *GEO, out_exponent=e)
    assert _fake_run(hc.mxfp8_conv2d, xm, e, wm2, we2, None, *GEO, out_exponent=e) == _sig_mx(want_m2)
    assert _fake_run(hc.im2col_gather, x, *GEO) == _sig(ref.im2col_gather(x, *GEO))


def test_quantize_fakes_match_oracle_shapes():
    v = torch.randn(2, 5, 7, 40).to(torch.bfloat16)
    e = torch.zeros(2, dtype=torch.int8)
    got = _fake_run(hq.quantize_mxfp8, v, e)
    assert got[0] == _sig_mx(ref.quantize_mxfp8(v, e))
    assert _fake_run(hq.gelu_quantize, v, e, input_bias=torch.randn(40))[0] == \
        _sig_mx(ref.gelu_quantize(v, e, input_bias=torch.randn(40)))
    s = torch.tensor(0.05)
    assert _fake_run(hq.quantize_int8, v, s) == _sig(ref.quantize_int8(v, s))
    assert _fake_run(hq.gelu_quantize_int8, v, s) == _sig(ref.gelu_quantize_int8(v, s))
    m = torch.randn(300, 64)
    cv, ce = ref.quantize_dynamic_2d(m)
    assert _fake_run(quant.quantize_dynamic_2d, m) == (_sig_mx(cv), _sig(ce))
    got_codes, got_swz = _fake_run(quant.quantize_dynamic_swizzled, m)
    assert got_codes == _sig_mx(cv) and got_swz[0] == (ref.swizzle_scales(ce).numel(),)
    q, sc = ref.quantize_int8_rows(m)
    assert _fake_run(quant.weight_scales_and_values, m) == (_sig(q), ((300,), torch.float32))
    m3 = torch.randn(2, 150, 64)
    q3, s3 = ref.quantize_int8_rows(m3)
    assert _fake_run(hq.quantize_int8_rows, m3) == (_sig(q3), _sig(s3))
    assert _fake_run(quant.calibrate_block32_exponent, v) == _sig(ref.calibrate_block32_exponent(v))


def test_gemm_and_block_fakes_match_oracle_shapes():
    a = torch.randint(-127, 127, (70, 96), dtype=torch.int8)
    w = torch.randint(-127, 127, (80, 96), dtype=torch.int8)
    a_s, w_s = torch.tensor(0.01), torch.rand(80)
    assert _fake_run(hg.int8_linear, a, w, a_s, w_s, None) == _sig(ref.int8_linear(a, w, a_s, w_s, None))
    out = torch.empty(70, 200, dtype=torch.int8)[:, 40:120]
    assert _fake_run(hg.int8_linear_quantize, a, w, a_s, w_s, None, torch.tensor(0.1), out) == \
        _sig(ref.int8_linear_quantize(a, w, a_s, w_s, None, torch.tensor(0.1)))
    value = torch.randn(2, 64, 6, 9)
    dw_w, dw_b = torch.randn(25, 64).to(torch.bfloat16), torch.randn(64)
    codes, swz = ref.depthwise5x5_relu_mxfp8(value, dw_w, dw_b)
    got = _fake_run(hc.depthwise5x5_relu_mxfp8, value, dw_w, dw_b)
    assert got[0] == _sig_mx(codes) and got[1][0] == tuple(swz.shape)
    assert _fake_run(hc.depthwise5x5_relu_int8, value, dw_w, dw_b, torch.tensor(0.1)) == \
        _sig(ref.depthwise5x5_relu_int8(value, dw_w, dw_b, torch.tensor(0.1)))
    assert _fake_run(hc.depthwise5x5_gelu, value, dw_w, dw_b) == _sig(ref.depthwise5x5_gelu(value, dw_w, dw_b))
    pw = torch.randn(64, 64).to(torch.float8_e4m3fn)
    pe = torch.zeros(64, 2, dtype=torch.int8)
    want = ref.depthwise5x5_relu_pointwise_mxfp8(value, dw_w, dw_b, pw, ref.swizzle_scales(pe),
                                                 ref.exponent_to_e8m0(pe), torch.randn(64))
    assert _fake_run(hc.depthwise5x5_relu_pointwise_mxfp8, value, dw_w, dw_b, pw, ref.swizzle_scales(pe),
                     ref.exponent_to_e8m0(pe), torch.randn(64)) == _sig(want)
    pw16, pb16 = torch.randn(48, 64).to(torch.bfloat16), torch.randn(48).to(torch.bfloat16)
    assert _fake_run(hc.depthwise5x5_relu_pointwise, value, dw_w, dw_b, pw16, pb16) == \
        _sig(ref.depthwise5x5_relu_pointwise(value, dw_w, dw_b, pw16, pb16))
    raw = torch.randn(1, 16, 5, 6).to(torch.bfloat16)
    assert _fake_run(hc.bias_relu_quantize_int8, raw, torch.randn(16), torch.tensor(0.1)) == \
        _sig(ref.bias_relu_quantize_int8(raw, torch.randn(16), torch.tensor(0.1)))
