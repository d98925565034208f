"""Benchmark of the MI355X quantized implicit-GEMM conv path (BASELINE.json's metric).

``python bench.py [--steps K] [--warmup W]`` prints ONE JSON line. The headline workload is BASELINE config 2 (the
MXFP8 1x1 conv, N=2, 100x100, 512 -> 512, fused bias + GELU, BF16 out): a "step" is one launch of the implicit-GEMM
conv on E4M3 activations already resident in HBM. ``value`` is its throughput in TOPS (dense MXFP8 operations:
2 * M * N * K per launch); ``roofline`` relates the same launch to the HBM roofline (config 2's arithmetic intensity,
338 FLOP/B, is below the MI355X ridge of 625 FLOP/B). ``configs`` reports every BASELINE config on the same run:
per-kernel ms, TOPS or GB/s and roofline fractions, and the refiner block / stack ms.

Timing: each measured launch sequence is captured once in a HIP graph and replayed; K replays are bracketed by
``torch.cuda.synchronize()`` and HIP events on the stream the kernels run on (torch's current stream); the
per-launch time is the event time divided by the launches. ``cpu_baseline`` times this repository's torch CPU oracle of
the same op (FlashIM's reference path restated) on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import torch

METRIC = "TOPS + % MFMA peak, MXFP8/INT8 implicit-GEMM conv; ms per refiner stack"
PEAK_MX_TFLOPS = 5000.0  # dense MXFP8 / FP8 MFMA, MI355X
PEAK_INT8_TOPS = 5000.0  # dense INT8 MFMA
PEAK_HBM_GBS = 8000.0
# HBM bytes per launch of the config-2 conv from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs (KiB per dispatch), each
# scaled by what the counter reads for a plain 64 MiB device copy (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0); the runs and the
# arithmetic are in profiles/conv_mxfp8_1x1_gelu_cfg2.md. Re-measured by hand when the kernel changes.
CFG2_TRAFFIC_BYTES = int((6244.0 * 2.0 + 20000.0 * 1.0) * 1024)  # the op's one launch (whole-K pointwise kernel)
# The config-4 block's algorithmic HBM bytes when fused (204.8 MB for 2 x 400 x 400 x 64: 10 bytes per
# element); GBps_own_launches divides instead the bytes this library's own launches of the block must move once.
CFG4_FUSED_BYTES = 204_800_000
# Vector-ALU issue floor of the GELU-bearing kernels: SQ_INSTS_VALU per launch (wave instructions) from rocprofv3
# --pmc runs (profiles/*.md), x 4 cycles per 64-lane instruction on a 16-lane SIMD / 1024 SIMDs / 2.4 GHz. These
# kernels are bound by that floor before HBM or MFMA; re-measured by hand when a kernel changes.
VALU_INSTS = {
    "cfg2_mxfp8_1x1_gelu": 2.92e6,          # conv_1x1_resident_kernel (GELU epilogue)
    "cfg3_mxfp8_3x3_bn_relu": 2.542e6,       # conv_patch_kernel
    "cfg4_depthwise_gelu_mxfp8": 9.10e6,    # dw5x5_mfma_kernel<GELU, static MXFP8>
}
CLOCK_GHZ, SIMDS = 2.4, 1024


def valu_floor_ms(name: str) -> float | None:
    n = VALU_INSTS.get(name)
    return None if n is None else n * 4 / SIMDS / (CLOCK_GHZ * 1e9) * 1e3


DEV = "cuda"


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--only", default=None, help="run one workload only (cfg1|cfg2|cfg3|cfg3q|dw|stem|dwpw|cfg4|cfg5int8|cfg5mxfp8|copy|peaks)"
                                                  " and print its line (profiling runs)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-stack", action="store_true", help="skip configs 4 and 5")
    return p.parse_args()


# -- timing ----------------------------------------------------------------------------------------------------


def time_graph(fn, steps: int, warmup: int, per_graph: int = 10) -> float:
    """Mean ms per call of ``fn``: ``per_graph`` back-to-back calls are captured in one HIP graph (so the time is the
    kernels', not the per-replay launch gap), the graph is replayed ``ceil(steps / per_graph)`` times between two HIP
    events on the stream the kernels run on, and the event time is divided by the calls."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            fn()
    replays = max(1, -(-steps // per_graph))
    for _ in range(max(1, -(-warmup // per_graph))):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * per_graph)


def time_graph_cold(fns, steps: int, warmup: int) -> float:
    """Mean ms per call with a cold working set: ``fns`` are the same op bound to distinct input buffers (together past
    the 256 MB Infinity Cache), captured back to back in one HIP graph with every output kept alive (so no call
    reuses another's output memory either), so each call reads and writes memory the previous calls did not touch."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for fn in fns:
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph, keep = torch.cuda.CUDAGraph(), []
    with torch.cuda.graph(graph):
        for fn in fns:
            keep.append(fn())
    replays = max(1, -(-steps // len(fns)))
    for _ in range(max(1, -(-warmup // len(fns)))):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * len(fns))


COLD_BYTES = 300 << 20  # a working set past the 256 MB Infinity Cache


def cold_sets(bytes_per_call: int) -> int:
    return max(2, -(-COLD_BYTES // bytes_per_call))


def time_cpu(fn, calls: int = 50, warmup: int = 10) -> float:
    """Median ms of ``fn`` over ``calls`` calls after ``warmup`` untimed ones."""
    for _ in range(warmup):
        fn()
    samples = []
    for _ in range(calls):
        t0 = time.perf_counter()
        fn()
        samples.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(samples)


# -- workloads -------------------------------------------------------------------------------------------------


def cfg1():
    """INT8 3x3 conv, NHWC N=1, 128x128, 64 -> 64, stride 1, pad 1; per-tensor activation scale, per-channel int8
    weights, fp32 bias."""
    from flashim_amd import ops, quant

    g = torch.Generator(device="cpu").manual_seed(1)
    act = torch.randn(1, 64, 128, 128, generator=g).to(DEV)
    a_scale = (act.abs().amax() / 127).float()
    x = ops.quantize_int8(act.permute(0, 2, 3, 1), a_scale).values
    w = (torch.randn(64, 64, 3, 3, generator=g) * 0.05).to(DEV)
    wq, w_scale = quant.weight_scales_and_values(w.permute(0, 2, 3, 1).reshape(64, -1))
    bias = torch.randn(64, generator=g).to(DEV)
    args = (x, wq, a_scale, w_scale, bias, 3, 3, 1, 1, 1, 1, 1, 1)
    fn = lambda: ops.int8_conv2d(*args)  # noqa: E731
    m, n, k = 128 * 128, 64, 576
    return fn, {"ops": 2 * m * n * k, "bytes": m * 64 + n * k + 4 * n + m * n * 2, "kind": "int8"}, args


def _mx_act(shape_nchw, g, outliers: bool):
    x = torch.randn(*shape_nchw, generator=g)
    if outliers:
        c = shape_nchw[1]
        factor = torch.exp(torch.empty(c).uniform_(math.log(0.1), math.log(10.0), generator=g))
        x = x * factor[None, :, None, None]
    return x.to(torch.bfloat16).to(DEV).permute(0, 2, 3, 1).contiguous()


def cfg2():
    """MXFP8 1x1 conv, NHWC N=2, 100x100, 512 -> 512; outlier-channel activations; bias + GELU; BF16 out."""
    from flashim_amd import ops, quant

    g = torch.Generator(device="cpu").manual_seed(2)
    x_bf16 = _mx_act((2, 512, 100, 100), g, outliers=True)
    exponent = quant.calibrate_block32_exponent(x_bf16)
    xq = ops.quantize_mxfp8(x_bf16, exponent).values
    w = quant.QuantizedWeight.from_float((torch.randn(512, 512, generator=g) * 0.05).to(DEV))
    bias = (torch.randn(512, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    args = (xq, exponent, w.values, w.scale_exponent, bias, 1, 1, 1, 1, 0, 0, 1, 1)
    fn = lambda: ops.mxfp8_conv2d(*args, gelu=True)  # noqa: E731
    m, n, k = 20000, 512, 512
    nbytes = m * k + n * k + n * k // 32 + 2 * n + m * n * 2
    return fn, {"ops": 2 * m * n * k, "bytes": nbytes, "kind": "mxfp8"}, args


def cfg3():
    """MXFP8 3x3 conv, NHWC N=2, 200x200, 128 -> 128, pad 1; weights N(0, 0.03) with a folded BatchNorm affine;
    bias + ReLU epilogue; BF16 out. Returns the conv and, separately, the activation quantizer."""
    from flashim_amd import ops, quant

    g = torch.Generator(device="cpu").manual_seed(3)
    x_bf16 = _mx_act((2, 128, 200, 200), g, outliers=False)
    exponent = quant.calibrate_block32_exponent(x_bf16)
    w = torch.randn(128, 128, 3, 3, generator=g) * 0.03
    gamma, beta = torch.rand(128, generator=g) + 0.5, torch.randn(128, generator=g) * 0.1
    mean, var = torch.randn(128, generator=g) * 0.1, torch.rand(128, generator=g) + 0.5
    inv = gamma / torch.sqrt(var + 1e-5)
    w_folded = w * inv[:, None, None, None]
    b_folded = beta - mean * inv
    wq = quant.QuantizedWeight.from_float(w_folded.permute(0, 2, 3, 1).reshape(128, -1).to(DEV))
    bias = b_folded.to(torch.bfloat16).to(DEV)
    xq = ops.quantize_mxfp8(x_bf16, exponent).values
    args = (xq, exponent, wq.values, wq.scale_exponent, bias, 3, 3, 1, 1, 1, 1, 1, 1)
    conv = lambda: ops.mxfp8_conv2d(*args, relu=True)  # noqa: E731
    quantize = lambda: ops.quantize_mxfp8(x_bf16, exponent)  # noqa: E731
    m, n, k = 80000, 128, 1152
    conv_bytes = m * 128 + n * k + n * k // 32 + 2 * n + m * n * 2
    q_bytes = m * 128 * 2 + m * 128
    return (conv, {"ops": 2 * m * n * k, "bytes": conv_bytes, "kind": "mxfp8"}, args), \
        (quantize, {"bytes": q_bytes}, (x_bf16, exponent))


def cfg4_depthwise():
    """The config-4 depthwise producer alone: 5x5 dwconv (folded BN) + GELU -> static MXFP8, NHWC 2x400x400x64."""
    from flashim_amd import ops

    g = torch.Generator(device="cpu").manual_seed(6)
    x = torch.randn(2, 400, 400, 64, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(25, 64, generator=g) * 0.2).to(torch.bfloat16).to(DEV)
    b = (torch.randn(64, generator=g) * 0.1).to(DEV)
    e = torch.full((2,), -6, dtype=torch.int8, device=DEV)
    fn = lambda: ops.depthwise5x5_gelu(x.permute(0, 3, 1, 2), w, b, exponent=e)  # noqa: E731
    pixels = 2 * 400 * 400
    bind = lambda xi: (lambda: ops.depthwise5x5_gelu(xi.permute(0, 3, 1, 2), w, b, exponent=e))  # noqa: E731
    return fn, {"bytes": pixels * 64 * 2 + pixels * 64}, (x, bind)


def stem():
    """The VGG stem (conv2d_small_cin_quantize_int8): 3 x 3 conv of a BF16 NCHW 1 x 3 x 896 x 1200 image, 3 -> 64,
    + bias + ReLU -> static INT8 NHWC (the image size FlashIM times its own kernel on, flashim/backends/triton/conv.py
    :916-917). HBM bytes: 2 per input element + 1 per output code."""
    from flashim_amd import ops

    g = torch.Generator(device="cpu").manual_seed(9)
    x = torch.randn(1, 3, 896, 1200, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(64, 3, 3, 3, generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    b = torch.randn(64, generator=g).to(torch.bfloat16).to(DEV)
    scale = torch.tensor(0.04, device=DEV)
    bound = ops.conv2d_small_cin_quantize_int8.bind(w, b)
    fn = lambda: bound(x, scale)  # noqa: E731
    pixels = 896 * 1200
    return fn, {"bytes": pixels * 3 * 2 + pixels * 64}


def dwpw_block():
    """The depthwise-then-pointwise refiner blocks at the shape FlashIM times its fused kernels on (2 x 128 x 400 x 400,
    flashim/backends/triton/conv.py:572-574): depthwise 5x5 + bias + ReLU -> BF16 / dynamic MXFP8 / static INT8 ->
    128 x 128 pointwise + bias -> BF16; the quantized blocks also as one kernel and as the two-launch composite. HBM
    bytes: BF16 in + BF16 out."""
    from flashim_amd import ops, quant
    from flashim_amd.backends.hip import conv as hip_conv

    g = torch.Generator(device="cpu").manual_seed(10)
    c = 128
    x = (torch.randn(2, c, 400, 400, generator=g) * 2).to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
    dw_w = (torch.randn(25, c, generator=g) * 0.3).to(torch.bfloat16)
    dw_b, pw_b = torch.randn(c, generator=g), torch.randn(c, generator=g)
    pw = quant.QuantizedWeight.from_float((torch.randn(c, c, generator=g) * 0.1).to(DEV))
    mx = [t.to(DEV) for t in (x, dw_w, dw_b, pw.values, quant.swizzle_scales(pw.scale_exponent),
                              quant.exponent_to_e8m0(pw.scale_exponent), pw_b)]
    i8 = [t.to(DEV) for t in (x, dw_w, dw_b, torch.randint(-127, 128, (c, c), dtype=torch.int8, generator=g),
                              torch.rand(c, generator=g) * 0.01 + 0.001, pw_b, torch.tensor(0.03))]
    bf = [t.to(DEV) for t in (x, dw_w, dw_b.to(torch.bfloat16),
                              (torch.randn(c, c, generator=g) * 0.1).to(torch.bfloat16), pw_b.to(torch.bfloat16))]
    nbytes = 2 * 400 * 400 * c * 2 * 2
    return {
        "bf16_op": lambda: ops.depthwise5x5_relu_pointwise(*bf),
        "mxfp8_op": lambda: ops.depthwise5x5_relu_pointwise_mxfp8(*mx),
        "mxfp8_one_kernel": lambda: hip_conv.pointwise_mxfp8_fused(*mx),
        "mxfp8_composite": lambda: hip_conv.pointwise_mxfp8_composite(*mx),
        "int8_op": lambda: ops.depthwise5x5_relu_pointwise_int8(*i8),
        "int8_one_kernel": lambda: hip_conv.pointwise_int8_fused(*i8),
        "int8_composite": lambda: hip_conv.pointwise_int8_composite(*i8),
    }, {"bytes": nbytes}


def copy_calibration():
    """A plain device copy of a known size (the PMC traffic calibration)."""
    src = torch.empty(64 << 20, device=DEV, dtype=torch.uint8).fill_(1)
    dst = torch.empty_like(src)
    return lambda: dst.copy_(src), src.numel()


def measured_peaks(steps: int, warmup: int) -> dict:
    """The box's own peaks, beside the datasheet ones: MFMA throughput from the register-only microbenchmark
    (``fim_test_mfma_peak``: 8 wavefronts per SIMD, back-to-back independent 16 x 16 MFMAs) and HBM bandwidth from a
    plain 64 MiB device copy (read + write)."""
    from flashim_amd import _lib

    blocks = 8 * torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(blocks * 256, device=DEV, dtype=torch.float32)
    iters = 400
    res = {}
    for kind, name, ops_each in ((0, "mfma_mxfp8_TFLOPs", 65536), (1, "mfma_int8_TOPs", 32768),
                                 (2, "mfma_int8_32x32x32_TOPs", 65536)):
        fn = lambda k=kind: _lib.probe_call("fim_test_mfma_peak", k, blocks, iters, out.data_ptr(),  # noqa: E731
                                      _lib.stream_of(out), what="mfma peak")
        ms = time_graph(fn, max(steps // 5, 3), 2, per_graph=1)
        res[name] = round(blocks * 4 * iters * 8 * ops_each / (ms * 1e-3) / 1e12, 1)
    fn, nbytes = copy_calibration()
    ms = time_graph(fn, steps, warmup)
    res["copy_GBps"] = round(2 * nbytes / (ms * 1e-3) / 1e9, 1)
    return res


# -- CPU baseline (oracle) ---------------------------------------------------------------------------------------


def _cpu_threads() -> int:
    cores = min(os.cpu_count() or 1, 16)  # the GPU box's CPU share is 16 threads, whatever os.cpu_count() reports
    torch.set_num_threads(cores)
    return cores


def cpu_baseline_cfg2(args) -> dict:
    """Config 2 through the torch CPU oracle, BASELINE.md's protocol: 10 warm-up calls, median of 50."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import reference as ref

    cores = _cpu_threads()
    cpu_args = [a.cpu() if isinstance(a, torch.Tensor) else a for a in args]
    ms = time_cpu(lambda: ref.mxfp8_conv2d(*cpu_args, gelu=True))
    ops = 2 * 20000 * 512 * 512
    return {
        "value": round(ops / (ms * 1e-3) / 1e12, 5), "unit": "TOPS", "cores": cores, "kind": "port",
        "ms": round(ms, 3),
        "sample": f"config 2 in full (M=20000, K=N=512, bias+GELU): oracle.reference.mxfp8_conv2d (torch CPU, "
                  f"FlashIM's reference path restated), 10 warm-up calls then the median of 50 "
                  f"(~{60 * ms / 1e3:.1f} s of CPU work), torch threads={cores}",
    }


def cpu_baseline_cfg1(args) -> dict:
    """Config 1 (FlashIM's own CPU-runnable case) through the torch CPU oracle, same protocol."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import reference as ref

    cores = _cpu_threads()
    cpu_args = [a.cpu() if isinstance(a, torch.Tensor) else a for a in args]
    ms = time_cpu(lambda: ref.int8_conv2d(*cpu_args))
    ops = 2 * 128 * 128 * 64 * 576
    return {
        "value": round(ops / (ms * 1e-3) / 1e12, 5), "unit": "TOPS", "cores": cores, "kind": "port", "ms": round(ms, 3),
        "sample": f"config 1 in full (INT8 3x3, 1x128x128, 64 -> 64): oracle.reference.int8_conv2d (torch CPU), "
                  f"10 warm-up calls then the median of 50, torch threads={cores}",
    }


# -- main --------------------------------------------------------------------------------------------------------


def main() -> int:
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {a.gpus}).",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.backends.cuda.matmul.allow_tf32 = False
    steps, warmup = a.steps, a.warmup

    if a.only == "copy":
        fn, nbytes = copy_calibration()
        ms = time_graph(fn, steps, warmup)
        print(json.dumps({"workload": "copy", "bytes": nbytes, "ms": ms, "GBps": 2 * nbytes / ms / 1e6}))
        return 0

    if a.only == "peaks":
        print(json.dumps({"workload": "peaks", "results": measured_peaks(steps, warmup)}))
        return 0

    results = {}

    def gemm_line(name, fn, info):
        ms = time_graph(fn, steps, warmup)
        peak = PEAK_INT8_TOPS if info["kind"] == "int8" else PEAK_MX_TFLOPS
        tops = info["ops"] / (ms * 1e-3) / 1e12
        gbs = info["bytes"] / (ms * 1e-3) / 1e9
        ai = info["ops"] / info["bytes"]
        attainable = min(peak, ai * PEAK_HBM_GBS / 1e3)
        results[name] = {
            "ms": round(ms, 5), "TOPS": round(tops, 2), "mfma_peak_frac": round(tops / peak, 4),
            "GBps": round(gbs, 1), "AI": round(ai, 1), "attainable_TOPS": round(attainable, 1),
            "roofline_frac": round(tops / attainable, 4), "bound": "mfma" if ai * PEAK_HBM_GBS / 1e3 >= peak else "hbm",
        }
        return ms

    def hbm_line(name, fn, info):
        ms = time_graph(fn, steps, warmup)
        gbs = info["bytes"] / (ms * 1e-3) / 1e9
        results[name] = {"ms": round(ms, 5), "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
        return ms

    def cold(name, x, bind, nbytes):
        """The cold-working-set variant of ``name``: the op over distinct copies of its input ``x``."""
        fns = [bind(x.clone()) for _ in range(cold_sets(nbytes))]
        ms = time_graph_cold(fns, steps, warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        results[name].update({"cold_ms": round(ms, 5), "cold_GBps": round(gbs, 1),
                              "cold_hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "cold_sets": len(fns)})

    only = a.only
    c2 = None
    if only in (None, "cfg1"):
        fn, info, _ = cfg1()
        gemm_line("cfg1_int8_3x3", fn, info)
    if only in (None, "cfg2"):
        fn, info, c2_args = cfg2()
        c2 = (fn, info, c2_args)
        gemm_line("cfg2_mxfp8_1x1_gelu", fn, info)
        from flashim_amd import ops as _ops
        cold("cfg2_mxfp8_1x1_gelu", c2_args[0],
             lambda xi: (lambda: _ops.mxfp8_conv2d(xi, *c2_args[1:], gelu=True)), info["bytes"])
    if only in (None, "cfg3", "cfg3q"):
        (conv, cinfo, _), (qfn, qinfo, qargs) = cfg3()
        if only in (None, "cfg3"):
            gemm_line("cfg3_mxfp8_3x3_bn_relu", conv, cinfo)
        if only in (None, "cfg3q"):
            hbm_line("cfg3q_quantize_mxfp8", qfn, qinfo)
            from flashim_amd import ops as _ops
            x_bf16, q_exp = qargs
            cold("cfg3q_quantize_mxfp8", x_bf16, lambda xi: (lambda: _ops.quantize_mxfp8(xi, q_exp).values),
                 qinfo["bytes"])
    if only in (None, "dw"):
        fn, info, (dw_x, dw_bind) = cfg4_depthwise()
        hbm_line("cfg4_depthwise_gelu_mxfp8", fn, info)
        cold("cfg4_depthwise_gelu_mxfp8", dw_x, dw_bind, info["bytes"])
    if only in (None, "stem"):
        fn, info = stem()
        hbm_line("stem_conv3x3_cin3_int8", fn, info)
    if only in (None, "dwpw"):
        fns, info = dwpw_block()
        for name, fn in fns.items():
            hbm_line(f"dwpw_2x128x400x400_{name}", fn, info)
    if not a.no_stack and only in (None, "cfg4", "cfg5int8", "cfg5mxfp8"):
        from flashim_amd import blocks

        if only in (None, "cfg4"):
            for preset in ("mxfp8", "int8"):
                fn, info = blocks.bench_block(preset, device=DEV)
                ms = time_graph(fn, steps, warmup, per_graph=2)
                fused_gbs = CFG4_FUSED_BYTES / (ms * 1e-3) / 1e9
                results[f"cfg4_block_{preset}"] = {
                    "ms": round(ms, 5), "GBps_fused_algorithmic": round(fused_gbs, 1),
                    "hbm_frac_fused_algorithmic": round(fused_gbs / PEAK_HBM_GBS, 4),
                    "GBps_own_launches": round(info["bytes"] / (ms * 1e-3) / 1e9, 1),
                    "TOPS": round(info["ops"] / (ms * 1e-3) / 1e12, 2),
                }
        for preset in ("int8", "mxfp8"):
            if only in (None, f"cfg5{preset}"):
                fn, info = blocks.bench_stack(preset, device=DEV)
                ms = time_graph(fn, 3, 1, per_graph=1)
                results[f"cfg5_stack_{preset}"] = {
                    "ms": round(ms, 4), "TOPS": round(info["ops"] / (ms * 1e-3) / 1e12, 2),
                    "blocks": info["blocks"], "pixels_per_scale": info["pixels"],
                }

    for name, r in results.items():
        floor = valu_floor_ms(name)
        if floor is not None:
            r.update({"valu_floor_ms": round(floor, 5), "valu_frac": round(floor / r["ms"], 4)})
    if only is not None:
        print(json.dumps({"workload": only, "results": results}))
        return 0

    head = results["cfg2_mxfp8_1x1_gelu"]
    fn, info, c2_args = c2
    ms = head["ms"]
    value = info["ops"] / (ms * 1e-3) / 1e12
    achieved_gbs = info["bytes"] / (ms * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TOPS", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp8_e4m3", "data": "synthetic (seeded N(0,1) x per-channel log-uniform [0.1, 10]; random-init weights)",
        "config": {"workload": "cfg2: MXFP8 1x1 conv + bias + GELU, NHWC N=2 H=W=100 Cin=Cout=512, BF16 out",
                   "M": 20000, "N": 512, "K": 512, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / PEAK_HBM_GBS, 4), "traffic": CFG2_TRAFFIC_BYTES,
                     "mfma_frac": round(value / PEAK_MX_TFLOPS, 4), "algorithmic_bytes": info["bytes"],
                     "valu_floor_ms": round(valu_floor_ms("cfg2_mxfp8_1x1_gelu"), 5),
                     "valu_frac": round(valu_floor_ms("cfg2_mxfp8_1x1_gelu") / ms, 4)},
        "configs": results,
    }
    peaks = measured_peaks(steps, warmup)
    line["measured_peaks"] = peaks
    line["roofline"]["frac_of_measured_copy"] = round(achieved_gbs / peaks["copy_GBps"], 4)
    line["roofline"]["mfma_frac_of_measured"] = round(value / peaks["mfma_mxfp8_TFLOPs"], 4)
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline_cfg2(c2_args)
        line["cpu_baseline_cfg1"] = cpu_baseline_cfg1(cfg1()[2])
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
