"""ctypes binding of ``libflashim_amd.so`` (the C ABI in ``include/flashim_amd.h``).

The library is loaded once, on first use. There is no fallback: a missing or unloadable library raises, so a GPU call
can never silently run anything but the HIP kernels. Launch helpers raise ``RuntimeError`` on a nonzero status, in
the form FlashIM's CUDA backend uses (``flashim/backends/cuda/conv.py:69-70``), and ``UnsupportedShape`` (a subclass)
for status 99, so a caller can tell "no kernel for this shape" from a launch failure.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

from flashim_amd._build import HOST_LIBRARY, LIBRARY, PROBE_LIBRARY

FIM_ERR_INVALID = 98
FIM_ERR_UNSUPPORTED = 99

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int

# symbol -> argtypes (all return int)
SIGNATURES: dict[str, list] = {
    "fim_version": [],
    "fim_quantize_int8": [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp],
    "fim_quantize_mxfp8": [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp],
    "fim_gelu_quantize_mxfp8": [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _i64,
                                _vp],
    "fim_gelu_quantize_int8": [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp],
    "fim_quantize_mxfp8_dynamic": [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp],
    "fim_quantize_int8_rows": [_vp, _i32, _i64, _i64, _i64, _i32, _vp, _vp, _vp],
    "fim_calibrate_block32": [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp],
    "fim_calibrate_block32_noalloc": [_vp, _i32, _i64, _i64, _i64, _vp, _vp],
    "fim_int8_conv2d": [
        _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
        _vp, _i32, _i64, _vp, _vp, _vp, _vp,
    ],
    "fim_mxfp8_conv2d": [
        _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
        _vp, _i32, _i64, _vp, _vp, _vp, _vp,
    ],
    "fim_int8_conv2d_maxpool": [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i32] + [_i32] * 9
    + [_vp, _vp, _vp, _vp],
    "fim_int8_linear": [
        _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _i64, _i64, _vp, _vp, _vp,
    ],
    "fim_int8_linear_quantize": [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _vp],
    "fim_mxfp8_scaled_mm": [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _i32, _vp, _i32, _vp, _vp],
    "fim_im2col_gather": [_vp, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp],
    "fim_refiner_mlp": [_i32, _i32, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _vp,
                        _vp],
    "fim_conv3x3_small_cin_quantize_int8": [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _vp, _vp],
    "fim_bias_relu_quantize_int8": [_vp, _i64, _i64, _i64, _i64, _vp, _i32, _vp, _vp, _vp],
    "fim_depthwise5x5": [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp],
    "fim_pointwise_bf16": [_vp, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _vp],
    "fim_depthwise5x5_relu_pointwise_mxfp8": [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _i64, _vp, _vp, _i32,
                                              _vp, _vp],
    "fim_depthwise5x5_relu_pointwise_int8": [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _i64, _vp, _vp,
                                             _i32, _vp, _vp],
}

# the probe library (csrc/probe.h): test and measurement hooks, not part of the product ABI
PROBE_SIGNATURES: dict[str, list] = {
    "fim_test_e4m3": [_vp, _i64, _vp, _vp],
    "fim_test_mx_exponent": [_vp, _i64, _vp, _vp],
    "fim_test_mfma_peak": [_i32, _i64, _i32, _vp, _vp],
    "fim_test_bf16": [_vp, _i64, _vp, _vp],
    "fim_test_gelu": [_vp, _i64, _vp, _vp],
}

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


class UnsupportedShape(RuntimeError):
    """The library has no kernel for this shape / layout (status 99)."""


_lock = threading.Lock()
_library: ctypes.CDLL | None = None
_probe: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIBRARY


def load() -> ctypes.CDLL:
    """The loaded HIP library; raises if it has not been built (``python -m flashim_amd._build``)."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is None:
            if not LIBRARY.is_file():
                raise RuntimeError(
                    f"flashim_amd HIP library missing at {LIBRARY}: build it with `python -m flashim_amd._build`"
                )
            lib = ctypes.CDLL(str(LIBRARY))
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int
            _library = lib
    return _library


def load_probe() -> ctypes.CDLL:
    """The device probe library (tests and the bench's peak measurement only)."""
    global _probe
    with _lock:
        if _probe is None:
            if not PROBE_LIBRARY.is_file():
                raise RuntimeError(f"{PROBE_LIBRARY} missing: build with `python -m flashim_amd._build`")
            lib = ctypes.CDLL(str(PROBE_LIBRARY))
            for name, argtypes in PROBE_SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int
            _probe = lib
    return _probe


def probe_call(name: str, *args, what: str | None = None) -> None:
    check(getattr(load_probe(), name)(*args), what or name)


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def load_host() -> ctypes.CDLL:
    """Host build of the scalar numerics (CPU tests only)."""
    if not HOST_LIBRARY.is_file():
        raise RuntimeError(f"{HOST_LIBRARY} missing: build with `python -m flashim_amd._build`")
    return ctypes.CDLL(str(HOST_LIBRARY))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def check(code: int, what: str) -> None:
    if code == 0:
        return
    if code == FIM_ERR_UNSUPPORTED:
        raise UnsupportedShape(f"{what}: no HIP kernel for this shape/layout (code 99)")
    raise RuntimeError(f"{what} launch failed (code {code})")


def call(name: str, *args, what: str | None = None) -> None:
    check(getattr(load(), name)(*args), what or name)
