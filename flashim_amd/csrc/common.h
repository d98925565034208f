// Device-side helpers shared by the HIP kernels: vector types, element loads of the activation dtypes, the C-ABI
// status codes and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "numerics.h"

#define FIM_OK 0
#define FIM_ERR_INVALID 98      // a null pointer or an inconsistent size
#define FIM_ERR_UNSUPPORTED 99  // a shape / layout this library has no kernel for (the caller takes another impl)

// dtype codes of floating activations crossing the C-ABI
#define FIM_F32 0
#define FIM_BF16 1
#define FIM_F16 2

namespace fim {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i);

template <>
__device__ __forceinline__ float load_elem<FIM_F32>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <>
__device__ __forceinline__ float load_elem<FIM_BF16>(const void* p, int64_t i) {
  return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <>
__device__ __forceinline__ float load_elem<FIM_F16>(const void* p, int64_t i) {
  return (float)static_cast<const _Float16*>(p)[i];
}

// Hardware FP32 -> E4M3 (gfx950 v_cvt_pk_fp8_f32 is OCP E4M3, round to nearest even). The GPU tests check it
// byte for byte against the software encoder in numerics.h over every BF16 value and random FP32 values.
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
#ifdef FIM_SOFTWARE_E4M3
  return (uint32_t)f32_to_e4m3_sw(a) | ((uint32_t)f32_to_e4m3_sw(b) << 8) | ((uint32_t)f32_to_e4m3_sw(c) << 16) |
         ((uint32_t)f32_to_e4m3_sw(d) << 24);
#else
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  int both = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
  return (uint32_t)both;
#endif
}

__device__ __forceinline__ uint8_t e4m3(float a) {
#ifdef FIM_SOFTWARE_E4M3
  return f32_to_e4m3_sw(a);
#else
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(a, a, 0, false) & 0xff);
#endif
}

inline int launch_status() {
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? FIM_OK : (int)err;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace fim
