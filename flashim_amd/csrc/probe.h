/* Device probes of libflashim_amd_probe.so: test and measurement hooks, not part of the product ABI
 * (include/flashim_amd.h). Same conventions: device pointers, the HIP stream, 0 or an error code back. */
#ifndef FLASHIM_AMD_PROBE_H
#define FLASHIM_AMD_PROBE_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* E4M3 encodings of n floats with the hardware conversion the kernels use (out[i]) and with the software encoder
 * (out[n + i]); x must be pre-clamped to +-448. */
int fim_test_e4m3(const float* x, int64_t n, uint8_t* out, hipStream_t stream);

/* BF16 roundings of n floats with the hardware conversion the kernels use (out[i]) and with the software rule
 * (out[n + i]). */
int fim_test_bf16(const float* x, int64_t n, uint16_t* out, hipStream_t stream);

/* GELU (erf form) of n BF16 values as the kernels' epilogues evaluate it, BF16 out. */
int fim_test_gelu(const uint16_t* x, int64_t n, uint16_t* out, hipStream_t stream);

/* MX exponents of n FP32 amax values with the device rule (quant/formats/mx.py:22-26). */
int fim_test_mx_exponent(const float* amax, int64_t n, int8_t* out, hipStream_t stream);

/* MFMA throughput microbenchmark: `blocks` workgroups of 256 threads, each wavefront `iters` rounds of 8 independent
 * MFMAs on register operands. kind 0: scaled MXFP8 16x16x128 (65536 FLOP each), 1: INT8 16x16x64 (32768 OP each),
 * 2: INT8 32x32x32 (65536 OP each). out: FP32 [blocks * 256], one sum per thread. */
int fim_test_mfma_peak(int kind, int64_t blocks, int iters, float* out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHIM_AMD_PROBE_H */
