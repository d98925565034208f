// Library version and the device test hooks declared in include/flashim_amd.h.
#include "common.h"

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

}  // namespace fim

using namespace fim;

extern "C" {

int fim_version(void) { return 100; }

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

}  // extern "C"
