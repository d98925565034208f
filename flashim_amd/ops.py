"""The ops of the quantized implicit-GEMM conv path, declared with FlashIM's names (``flashim/ops/conv.py``,
``flashim/ops/gemm.py``, ``flashim/ops/quantize.py``) on this package's dispatcher (:mod:`flashim_amd.dispatch`), with
this backend's impls registered for the ``"rocm"`` dispatch key and the gfx950 ISA features. Usage mirrors FlashIM:
``ops.int8_conv2d(...)`` dispatches, ``ops.int8_conv2d.get("hip")`` pins the HIP impl, ``ops.int8_conv2d.explain(...)``
says why an impl does or does not apply.

The declarations carry no torch implementation: a call no HIP impl accepts raises instead of computing elsewhere.
"""

from __future__ import annotations

from flashim_amd.backends.hip import conv as _conv
from flashim_amd.backends.hip import gemm as _gemm
from flashim_amd.backends.hip import quantize as _quantize
from flashim_amd.dispatch import (  # noqa: F401  (re-exported API)
    OPS, BoundOp, DeviceSpec, Op, call_counts, configure, reset_call_counts,
)
from flashim_amd.platforms import Feature

# declarations (FlashIM names)
quantize_mxfp8 = Op("quantize_mxfp8")
quantize_int8 = Op("quantize_int8")
quantize_int8_rows = Op("quantize_int8_rows")
gelu_quantize = Op("gelu_quantize")
gelu_quantize_int8 = Op("gelu_quantize_int8")
int8_conv2d = Op("int8_conv2d")
mxfp8_conv2d = Op("mxfp8_conv2d")
depthwise5x5_relu_mxfp8 = Op("depthwise5x5_relu_mxfp8")
depthwise5x5_relu_int8 = Op("depthwise5x5_relu_int8")
depthwise5x5_relu_pointwise = Op("depthwise5x5_relu_pointwise")
depthwise5x5_relu_pointwise_mxfp8 = Op("depthwise5x5_relu_pointwise_mxfp8")
depthwise5x5_relu_pointwise_int8 = Op("depthwise5x5_relu_pointwise_int8")
im2col_gather = Op("im2col_gather")
int8_conv2d_maxpool = Op("int8_conv2d_maxpool")
int8_linear = Op("int8_linear")
int8_linear_quantize = Op("int8_linear_quantize")
mxfp8_linear = Op("mxfp8_linear", weights=1)
mxfp8_scaled_mm = Op("mxfp8_scaled_mm")
mxfp8_gelu_mlp = Op("mxfp8_gelu_mlp")
conv2d_small_cin_quantize_int8 = Op("conv2d_small_cin_quantize_int8", weights=2)
bias_relu_quantize_int8 = Op("bias_relu_quantize_int8")
# this backend's refiner-block producer (folded BatchNorm + GELU)
depthwise5x5_gelu = Op("depthwise5x5_gelu")

ROCM = DeviceSpec("rocm")
HIP = "hip"
_MX = (Feature.HIP, Feature.MFMA_F8F6F4_SCALED)
_I8 = (Feature.HIP, Feature.MFMA_I8)

IMPLS = (
    # (op name, impl fn, required features, when)
    ("quantize_mxfp8", _quantize.quantize_mxfp8, (Feature.HIP, Feature.FP8_E4M3), _quantize.eligible_quantize_mxfp8),
    ("quantize_int8", _quantize.quantize_int8, (Feature.HIP,), _quantize.eligible_quantize_int8),
    ("quantize_int8_rows", _quantize.quantize_int8_rows, (Feature.HIP,), _quantize.eligible_quantize_int8_rows),
    ("gelu_quantize", _quantize.gelu_quantize, (Feature.HIP, Feature.FP8_E4M3), _quantize.eligible_gelu_quantize),
    ("gelu_quantize_int8", _quantize.gelu_quantize_int8, (Feature.HIP,), _quantize.eligible_gelu_quantize_int8),
    ("int8_conv2d", _conv.int8_conv2d, _I8, _conv.eligible_int8_conv2d),
    ("mxfp8_conv2d", _conv.mxfp8_conv2d, _MX, _conv.eligible_mxfp8_conv2d),
    ("depthwise5x5_relu_mxfp8", _conv.depthwise5x5_relu_mxfp8, (Feature.HIP, Feature.FP8_E4M3),
     _conv.eligible_depthwise),
    ("depthwise5x5_relu_int8", _conv.depthwise5x5_relu_int8, (Feature.HIP,), _conv.eligible_depthwise),
    ("depthwise5x5_gelu", _conv.depthwise5x5_gelu, (Feature.HIP,), _conv.eligible_depthwise),
    ("depthwise5x5_relu_pointwise", _conv.depthwise5x5_relu_pointwise, (Feature.HIP,), _conv.eligible_pointwise_bf16),
    ("depthwise5x5_relu_pointwise_mxfp8", _conv.depthwise5x5_relu_pointwise_mxfp8, _MX,
     _conv.eligible_pointwise_mxfp8),
    ("depthwise5x5_relu_pointwise_int8", _conv.depthwise5x5_relu_pointwise_int8, _I8, _conv.eligible_pointwise_int8),
    ("im2col_gather", _conv.im2col_gather, (Feature.HIP,), _conv.eligible_im2col),
    ("int8_conv2d_maxpool", _conv.int8_conv2d_maxpool, _I8, _conv.eligible_int8_conv2d_maxpool),
    ("int8_linear", _gemm.int8_linear, _I8, _gemm.eligible_int8_linear),
    ("int8_linear_quantize", _gemm.int8_linear_quantize, _I8, _gemm.eligible_int8_linear_quantize),
    ("mxfp8_linear", _gemm.mxfp8_linear, _MX, _gemm.eligible_mxfp8_linear),
    ("mxfp8_scaled_mm", _gemm.mxfp8_scaled_mm, _MX, _gemm.eligible_mxfp8_scaled_mm),
    ("mxfp8_gelu_mlp", _gemm.mxfp8_gelu_mlp, _MX, _gemm.eligible_mxfp8_gelu_mlp),
    ("bias_relu_quantize_int8", _conv.bias_relu_quantize_int8, (Feature.HIP,), _conv.eligible_bias_relu_quantize),
)

for _name, _fn, _requires, _when in IMPLS:
    OPS[_name].register(HIP, device=ROCM, requires=_requires, priority=2, when=_when)(_fn)

# the stem conv packs its weights once per bind (FlashIM's prepare / accepts, flashim/backends/triton/conv.py:925-950)
conv2d_small_cin_quantize_int8.register(
    HIP, device=ROCM, requires=(Feature.HIP,), priority=2, when=_conv.eligible_small_cin,
    accepts=_conv.accepts_small_cin, prepare=_conv.small_cin_prepare,
)(_conv.conv2d_small_cin_quantize_int8)
