"""Writes tests/golden/golden.npz: the known answers of FlashIM's own tests for this path plus small seeded oracle
vectors (inputs and outputs) for the conv/quantize ops. ``python -m tests.golden.make_golden`` regenerates it.

Known answers copied as values: tests/quant/test_mx_format.py:13-17 (exponent rule) and tests/quant/test_int8.py:26-29
(round-half-even INT8). FlashIM ships no binary golden vectors for these ops; the seeded vectors are the oracle's
(oracle/reference.py, torch CPU) and pin it against drift of torch's arithmetic across versions."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from oracle import reference as ref

PATH = Path(__file__).resolve().parent / "golden.npz"


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().astype(np.uint16)


def _u8(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).numpy()


def compute() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    out["ka_exponent_amax"] = np.array([0.0, 448.0, 449.0, 1.0, 1e-30], dtype=np.float32)
    out["ka_exponent"] = np.array([-127, 0, 1, -8, -108], dtype=np.int8)
    out["ka_int8_x"] = np.array([0.5, 1.5, 2.5, -0.5, 1000.0, -1000.0, 0.0], dtype=np.float32)
    out["ka_int8_q"] = np.array([0, 2, 2, 0, 127, -127, 0], dtype=np.int8)
    assert np.array_equal(ref.scale_exponent_from_amax(torch.from_numpy(out["ka_exponent_amax"])).numpy(),
                          out["ka_exponent"])
    assert np.array_equal(ref.quantize_int8_static(torch.from_numpy(out["ka_int8_x"]), torch.tensor(1.0)).numpy(),
                          out["ka_int8_q"])

    g = torch.Generator().manual_seed(1234)
    # INT8 3x3 conv, stride 1, pad 1: accumulators and the BF16 output with bias
    x = torch.randint(-127, 127, (1, 6, 7, 16), dtype=torch.int8, generator=g)
    w = torch.randint(-127, 127, (24, 9 * 16), dtype=torch.int8, generator=g)
    a_scale = torch.tensor(0.017)
    w_scale = torch.rand(24, generator=g) * 0.01 + 0.001
    bias = torch.randn(24, generator=g).to(torch.bfloat16)
    geo = (3, 3, 1, 1, 1, 1, 1, 1)
    out["int8conv_x"], out["int8conv_w"] = x.numpy(), w.numpy()
    out["int8conv_w_scale"], out["int8conv_bias"] = w_scale.numpy(), _u16(bias)
    out["int8conv_acc"] = ref.int8_conv2d_accumulators(x, w, *geo).numpy().astype(np.int32)
    out["int8conv_out"] = _u16(ref.int8_conv2d(x, w, a_scale, w_scale, bias, *geo))
    # static MXFP8 quantize (channels padded 40 -> 64)
    xq = (torch.randn(5, 40, generator=g) * 5).to(torch.bfloat16)
    e = ref.calibrate_block32_exponent(xq.float())
    out["mxq_x"], out["mxq_exponent"], out["mxq_out"] = _u16(xq), e.numpy(), _u8(ref.quantize_mxfp8(xq, e))
    # dynamic per-(row, 32) MXFP8 with the swizzled scales
    xd = torch.randn(7, 64, generator=g) * torch.rand(7, 1, generator=g) * 20
    qd, ed = ref.quantize_dynamic_2d(xd)
    out["mxdyn_x"], out["mxdyn_out"], out["mxdyn_exponent"] = xd.numpy(), _u8(qd), ed.numpy()
    out["mxdyn_swizzled"] = ref.swizzle_scales(ed).numpy()
    # MXFP8 3x3 conv
    xm = (torch.randn(1, 5, 6, 32, generator=g) * 3).to(torch.float8_e4m3fn)
    cem = torch.tensor([-3], dtype=torch.int8)
    wm = (torch.randn(16, 9 * 32, generator=g)).to(torch.float8_e4m3fn)
    wem = torch.randint(-8, -3, (16, 9), dtype=torch.int8, generator=g)
    out["mxconv_x"], out["mxconv_ce"], out["mxconv_w"], out["mxconv_we"] = _u8(xm), cem.numpy(), _u8(wm), wem.numpy()
    out["mxconv_out"] = _u16(ref.mxfp8_conv2d(xm, cem, wm, wem, None, *geo))
    # depthwise 5x5 + ReLU -> INT8
    xdw = torch.randn(1, 32, 6, 7, generator=g).to(torch.bfloat16)
    wdw = (torch.randn(25, 32, generator=g) * 0.3).to(torch.bfloat16)
    bdw = torch.randn(32, generator=g)
    out["dw_x"], out["dw_w"], out["dw_b"] = _u16(xdw), _u16(wdw), bdw.numpy()
    out["dw_int8"] = ref.depthwise5x5_relu_int8(xdw, wdw, bdw, torch.tensor(0.03)).numpy()
    return out


def main() -> None:
    np.savez_compressed(PATH, **compute())
    print(PATH, PATH.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
