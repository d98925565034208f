// Device probes for the tests and the bench, built as their own library (libflashim_amd_probe.so) and kept out of
// the product library and its public header: the kernels' numerics helpers evaluated element by element (checked
// against torch on the GPU), and an MFMA throughput microbenchmark (the measured peaks the roofline fractions are also
// quoted against). Declarations: probe.h.
#include "common.h"
#include "probe.h"

namespace fim {

__global__ void test_e4m3_kernel(const float* x, int64_t n, uint8_t* out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = e4m3(x[i]);
  out[n + i] = f32_to_e4m3_sw(x[i]);
}

__global__ void test_bf16_kernel(const float* x, int64_t n, uint16_t* out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (uint16_t)(pack_bf16x2(x[i], 0.0f) & 0xffffu);
  out[n + i] = f32_to_bf16(x[i]);
}

__global__ void test_gelu_kernel(const uint16_t* x, int64_t n, uint16_t* out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f32_to_bf16(gelu_erf(bf16_to_f32(x[i])));
}

__global__ void test_mx_exponent_kernel(const float* amax, int64_t n, int8_t* out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (int8_t)mx_exponent_from_amax(amax[i]);
}

// MFMA throughput microbenchmark: every wavefront runs `iters` rounds of 8 independent 16 x 16 MFMAs on register
// operands (no memory traffic in the loop; the operands depend on the lane, the sum is written out so nothing is
// dropped). kind 0: v_mfma_scale_f32_16x16x128_f8f6f4 (MXFP8, 65536 FLOP each), 1: v_mfma_i32_16x16x64_i8 (32768 OP),
// 2: v_mfma_i32_32x32x32_i8 (65536 OP).
template <int KIND>
__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, float* out) {
  const int lane = threadIdx.x & 63;
  v8i a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = 0x30303030 + ((lane + i) & 15);  // bytes 0x30..0x3f and 0x28..0x37: finite E4M3 (no 0x7f / 0xff NaN
    b[i] = 0x28282828 + ((3 * lane + i) & 15);  // codes), small INT8
  }
  v4f accf[8];
  v4i acci[8];
  v16i acc32[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    accf[j] = v4f{0.f, 0.f, 0.f, 0.f};
    acci[j] = v4i{0, 0, 0, 0};
    acc32[j] = v16i{};
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (KIND == 0)
        accf[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, accf[j], 0, 0, 0, 127, 0, 127);
      else if constexpr (KIND == 1)
        acci[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(a, a, 0, 1, 2, 3),
                                                        __builtin_shufflevector(b, b, 0, 1, 2, 3), acci[j], 0, 0, 0);
      else
        acc32[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_shufflevector(a, a, 0, 1, 2, 3),
                                                         __builtin_shufflevector(b, b, 0, 1, 2, 3), acc32[j], 0, 0, 0);
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) sum += KIND == 0 ? accf[j][e] : KIND == 1 ? (float)acci[j][e] : (float)acc32[j][e];
  out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
}

}  // namespace fim

using namespace fim;

extern "C" {

int fim_test_e4m3(const float* x, int64_t n, uint8_t* out, hipStream_t stream) {
  if (x == nullptr || out == nullptr || n < 0) return FIM_ERR_INVALID;
  if (n == 0) return FIM_OK;
  test_e4m3_kernel<<<dim3((unsigned)cdiv(n, 256)), dim3(256), 0, stream>>>(x, n, out);
  return launch_status();
}

int fim_test_bf16(const float* x, int64_t n, uint16_t* out, hipStream_t stream) {
  if (x == nullptr || out == nullptr || n < 0) return FIM_ERR_INVALID;
  if (n == 0) return FIM_OK;
  test_bf16_kernel<<<dim3((unsigned)cdiv(n, 256)), dim3(256), 0, stream>>>(x, n, out);
  return launch_status();
}

int fim_test_gelu(const uint16_t* x, int64_t n, uint16_t* out, hipStream_t stream) {
  if (x == nullptr || out == nullptr || n < 0) return FIM_ERR_INVALID;
  if (n == 0) return FIM_OK;
  test_gelu_kernel<<<dim3((unsigned)cdiv(n, 256)), dim3(256), 0, stream>>>(x, n, out);
  return launch_status();
}

int fim_test_mx_exponent(const float* amax, int64_t n, int8_t* out, hipStream_t stream) {
  if (amax == nullptr || out == nullptr || n < 0) return FIM_ERR_INVALID;
  if (n == 0) return FIM_OK;
  test_mx_exponent_kernel<<<dim3((unsigned)cdiv(n, 256)), dim3(256), 0, stream>>>(amax, n, out);
  return launch_status();
}

int fim_test_mfma_peak(int kind, int64_t blocks, int iters, float* out, hipStream_t stream) {
  if (out == nullptr || blocks <= 0 || blocks > (1 << 20) || iters <= 0 || kind < 0 || kind > 2)
    return FIM_ERR_INVALID;
  if (kind == 0)
    mfma_peak_kernel<0><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(iters, out);
  else if (kind == 1)
    mfma_peak_kernel<1><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(iters, out);
  else
    mfma_peak_kernel<2><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(iters, out);
  return launch_status();
}

}  // extern "C"
