"""The fused refiner MLP (``fim_refiner_mlp``) on the GPU:

* ``mxfp8_gelu_mlp`` (FlashIM's op, ``flashim/ops/gemm.py:146-157``) against the oracle: relative L2 < 1e-2, the bound
  FlashIM's own test holds its MMA-based fused kernel to against the torch reference
  (``tests/ops/test_ops_cuda.py:672-699``). Two quantized stages compound the accumulation-order effect: a hidden
  E4M3 code flips whenever GEMM 1's FP32 sum order (or GELU's last BF16 rounding) moves its input across a code
  boundary, so the single-GEMM MXFP8 bar does not apply to the composite;
* the block semantics against the two conv launches it replaces, bit for bit (INT8 and MXFP8: same arithmetic,
  same accumulation order), and against the oracle composition;
* ragged row counts (not a multiple of the 64-pixel tile), a single row, and a grid-stride run (more tiles than
  workgroups).
"""

from __future__ import annotations

import pytest
import torch

from flashim_amd import ops, quant
from flashim_amd.backends.hip import gemm as _gemm
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
C, H = 64, 256


def _mx_weights(g):
    w1 = quant.QuantizedWeight.from_float((torch.randn(H, C, generator=g) * C**-0.5).to(DEV))
    w2 = quant.QuantizedWeight.from_float((torch.randn(C, H, generator=g) * H**-0.5).to(DEV))
    return w1, w2


def _rel(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.float(), want.float()
    return ((got - want).norm() / want.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("rows", [1, 63, 64, 1000, 70000])
def test_mxfp8_gelu_mlp_matches_oracle(rows):
    # FlashIM's test setup (test_ops_cuda.py:672-682) at this kernel's width: weights N(0, 0.05), b1 N(0, 0.1),
    # the hidden exponent calibrated on GELU(2 N(0, 1))
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, C, generator=g).to(torch.bfloat16)
    xe = ref.calibrate_block32_exponent(x.float())
    xq = ops.quantize_mxfp8(x.to(DEV), xe.to(DEV))
    w1 = quant.QuantizedWeight.from_float((torch.randn(H, C, generator=g) * 0.05).to(DEV))
    w2 = quant.QuantizedWeight.from_float((torch.randn(C, H, generator=g) * 0.05).to(DEV))
    b1 = torch.randn(H, generator=g) * 0.1
    he = ref.calibrate_block32_exponent(torch.nn.functional.gelu(torch.randn(64, H, generator=g) * 2))
    got = ops.mxfp8_gelu_mlp.get("hip")(xq, w1, b1.to(DEV), he.to(DEV), w2).cpu()
    want = ref.mxfp8_gelu_mlp(xq.values.cpu(), xe, w1.values.cpu(), w1.scale_exponent.cpu(), b1, he,
                              w2.values.cpu(), w2.scale_exponent.cpu())
    assert got.shape == want.shape == (rows, C)
    assert _rel(got, want) < 1e-2


def _two_convs(preset, q1, in_scale, w1, w1s, b1, hs, w2, w2s, b2, res):
    one = (1, 1, 1, 1, 0, 0, 1, 1)
    if preset == "mxfp8":
        q2 = ops.mxfp8_conv2d.get("hip")(q1, in_scale, w1, w1s, b1, *one, gelu=True, out_exponent=hs)
        return ops.mxfp8_conv2d.get("hip")(q2, hs, w2, w2s, b2, *one, residual=res)
    q2 = ops.int8_conv2d.get("hip")(q1, w1, in_scale, w1s, b1, *one, gelu=True, out_scale=hs)
    return ops.int8_conv2d.get("hip")(q2, w2, hs, w2s, b2, *one, residual=res)


@pytest.mark.parametrize("preset", ["mxfp8", "int8"])
@pytest.mark.parametrize("shape", [(1, 1, 1), (1, 7, 9), (2, 40, 33), (2, 400, 400)])
def test_block_semantics_equal_two_conv_launches(preset, shape):
    b, h, w = shape
    g = torch.Generator().manual_seed(b * 1000 + h * 10 + w)
    x = torch.randn(b, h, w, C, generator=g).to(torch.bfloat16).to(DEV)
    act = torch.randn(b, h, w, C, generator=g).to(torch.bfloat16).to(DEV)
    b1 = (torch.randn(H, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    b2 = (torch.randn(C, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    if preset == "mxfp8":
        in_scale = quant.calibrate_block32_exponent(act)
        q1 = ops.quantize_mxfp8(act, in_scale).values
        w1, w2 = _mx_weights(g)
        w1v, w1s, w2v, w2s = w1.values, w1.scale_exponent, w2.values, w2.scale_exponent
        hs = torch.full((H // 32,), -5, dtype=torch.int8, device=DEV)
    else:
        in_scale = (act.float().abs().amax() / 127).reshape(())
        q1 = ops.quantize_int8(act, in_scale).values
        w1v, w1s = quant.weight_scales_and_values((torch.randn(H, C, generator=g) * C**-0.5).to(DEV))
        w2v, w2s = quant.weight_scales_and_values((torch.randn(C, H, generator=g) * H**-0.5).to(DEV))
        hs = torch.tensor(0.02, device=DEV)
    want = _two_convs(preset, q1, in_scale, w1v, w1s, b1, hs, w2v, w2s, b2, x)
    got = _gemm.refiner_mlp(q1, in_scale, w1v, w1s, b1, hs, w2v, w2s, b2, x)
    assert got.shape == want.shape == (b, h, w, C)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_block_semantics_match_oracle_composition():
    """The block semantics against the oracle's two convs (the bit-exact equality with this library's own two conv
    launches is tested above): relative L2 < 1e-2, as for the fused op."""
    g = torch.Generator().manual_seed(7)
    rows = 4096
    act = torch.randn(rows, C, generator=g).to(torch.bfloat16)
    in_scale = ref.calibrate_block32_exponent(act.float())
    q1 = ref.quantize_mxfp8(act, in_scale)
    w1 = quant.QuantizedWeight.from_float((torch.randn(H, C, generator=g) * 0.05).to(DEV))
    w2 = quant.QuantizedWeight.from_float((torch.randn(C, H, generator=g) * 0.05).to(DEV))
    b1 = (torch.randn(H, generator=g) * 0.1).to(torch.bfloat16)
    hs = ref.calibrate_block32_exponent(torch.nn.functional.gelu(torch.randn(64, H, generator=g) * 2))
    res = torch.randn(rows, C, generator=g).to(torch.bfloat16)
    got = _gemm.refiner_mlp(q1.to(DEV), in_scale.to(DEV), w1.values, w1.scale_exponent, b1.to(DEV), hs.to(DEV),
                            w2.values, w2.scale_exponent, None, res.to(DEV)).cpu()
    one = (1, 1, 1, 1, 0, 0, 1, 1)
    q2 = ref.mxfp8_conv2d(q1.view(1, 1, rows, C), in_scale, w1.values.cpu(), w1.scale_exponent.cpu(), b1, *one,
                          gelu=True, out_exponent=hs)
    want = ref.mxfp8_conv2d(q2, hs, w2.values.cpu(), w2.scale_exponent.cpu(), None, *one,
                            residual=res.view(1, 1, rows, C)).view(rows, C)
    assert _rel(got, want) < 1e-2


def test_unsupported_width_reports_99():
    from flashim_amd import _lib

    x = torch.zeros(8, 128, dtype=torch.uint8, device=DEV)
    code = _lib.load().fim_refiner_mlp(1, 0, x.data_ptr(), 8, 128, 512, x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                       None, 0, x.data_ptr(), x.data_ptr(), x.data_ptr(), None, 0, None, x.data_ptr(),
                                       _lib.stream_of(x))
    assert code == _lib.FIM_ERR_UNSUPPORTED
