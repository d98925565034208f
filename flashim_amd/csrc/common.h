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
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// Two floats -> packed BF16 (low = a), round to nearest even: one v_cvt_pk_bf16_f32 on gfx950. The GPU tests check it
// against the software rounding of numerics.h (f32_to_bf16) and torch over every BF16 neighbourhood class.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  v2f v = {a, b};
  v2bf p = __builtin_convertvector(v, v2bf);
  return __builtin_bit_cast(uint32_t, p);
}

// x rounded to BF16 and widened back (torch's `.to(torch.bfloat16).float()`): one v_cvt_pk_bf16_f32 with a zero low
// half, whose 32-bit result is the rounded value itself (no unpacking).
__device__ __forceinline__ float round_bf16_hw(float x) { return u2f(pack_bf16x2(0.0f, x)); }

// a and b rounded to BF16 and widened back: two conversions (cheaper than one packed conversion and two unpacks).
__device__ __forceinline__ void round_bf16x2(float& a, float& b) {
  a = round_bf16_hw(a);
  b = round_bf16_hw(b);
}

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
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  int both = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
  return (uint32_t)both;
}

// E4M3 codes of BF16(a..d) * 2^-e for values already within +-448 * 2^e (scale = 2^e): the pack rounds to BF16 and
// v_cvt_scalef32_pk_fp8_bf16 divides by the scale and converts (RNE). Out-of-range values become NaN codes (the
// conversion does not saturate), so callers clamp first.
__device__ __forceinline__ uint32_t e4m3x4_of_bf16_inrange(float a, float b, float c, float d, float scale) {
  typedef short v2s_t __attribute__((ext_vector_type(2)));
  typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));
  const v2s_t lo = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(v2s_t{0, 0}, __builtin_bit_cast(v2bf_t, pack_bf16x2(a, b)),
                                                             scale, false);
  const v2s_t both = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(lo, __builtin_bit_cast(v2bf_t, pack_bf16x2(c, d)),
                                                               scale, true);
  return __builtin_bit_cast(uint32_t, both);
}

// E4M3 codes of BF16(a..d) * 2^-e, clamped to +-448: the BF16 rounding then static MXFP8 quantize of the references
// (a BF16 activation quantized with quant/tensor.py:97-121). scale = 2^e, bound = 448 * 2^e. The clamp commutes with
// the BF16 rounding (bound is a BF16 value and rounding is monotonic), so the values are clamped in FP32 (IEEE
// minimum / maximum: NaN stays NaN), rounded to BF16 by the pack, and v_cvt_scalef32_pk_fp8_bf16 divides by the scale
// and converts: 2 operations per value fewer than unpacking, multiplying and converting from FP32, and byte for byte
// the same codes (measured on the GPU over every BF16 input, NaN and infinities included, at exponents -10..10).
__device__ __forceinline__ uint32_t e4m3x4_of_bf16(float a, float b, float c, float d, float scale, float bound) {
  a = __builtin_elementwise_maximum(__builtin_elementwise_minimum(a, bound), -bound);
  b = __builtin_elementwise_maximum(__builtin_elementwise_minimum(b, bound), -bound);
  c = __builtin_elementwise_maximum(__builtin_elementwise_minimum(c, bound), -bound);
  d = __builtin_elementwise_maximum(__builtin_elementwise_minimum(d, bound), -bound);
  return e4m3x4_of_bf16_inrange(a, b, c, d, scale);
}

__device__ __forceinline__ uint8_t e4m3(float a) {
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(a, a, 0, false) & 0xff);
}

// mx_exponent_from_amax for a finite amax >= 0 in wave-uniform control flow: the division-free mx_exponent_fast, and
// the exact path behind one wave-uniform branch for the lanes it declines (all-zero blocks, quotients near a power of
// two).
__device__ __forceinline__ int mx_exponent_wave(float amax) {
  int e = 0;
  const bool fast = mx_exponent_fast(amax, e);
  if (__builtin_amdgcn_ballot_w64(!fast) != 0) {
    if (!fast) e = mx_exponent_from_amax(amax);
  }
  return e;
}

// GELU, erf form: 0.5 x erfc(-x / sqrt 2) = max(x, 0) - |x| E with E = erfc(|x| / sqrt 2) / 2 (x >= 0: x - x E;
// x < 0: x E). With z = |x| / sqrt 2 and t = 2 z / 4.1 - 1, log2 E is the degree-7 polynomial P(t) below (a near-minimax
// fit of log2(erfc(z) / 2) on [0, 4.1], this repository's own, max error 4.7e-6 in log2 units, i.e. 3.3e-6 relative in
// E), so E = 2^P(t): one v_exp_f32, 7 FMAs, no division, and the last step is one FMA, fma(-|x|, E, max(x, -0)). The
// polynomial needs no clamp outside the fit: its leading coefficient is negative and P decreases monotonically for
// t > 1 (P = -28.2 at the fit's end, below -900 at |x| = 40, -inf once its leading term overflows), so the large-|x|
// limits come out right by themselves: x - 0 = x for large positive x, and -0 (fma(-|x|, 0, -0)) once 2^P underflows for
// large negative x. Between x = -5.53 (where torch's FP32 1 + erf(x / sqrt 2) becomes exactly 0, so torch returns -0)
// and about x = -12 the result is the true tiny GELU value (< 1e-7 in magnitude) instead of -0. Against torch's BF16
// GELU it differs by one BF16 step in about 1% of the finite BF16 inputs (torch's own erf rounding moves values across
// BF16 rounding boundaries too); in torch's cancelling negative tail (x < -3) both are within 2^-12 of each other.
// Signed zeros follow torch: GELU(+0) = +0, GELU(-0) = -0. A degree-5 fit (two FMAs fewer, 5e-5 relative) was measured
// too: the same fraction of one-step differences over all BF16 inputs, but true values within 5e-5 of a BF16 rounding
// midpoint then round to the other side of it far more often (7.7% of one INT8 linear's GELU outputs against torch),
// so the more accurate fit stays.
// Evaluated in the rescaled variable u = s t, s = |c7|^(1/7) = 0.43911893, where the polynomial is monic up to sign
// (coefficients c_k / s^k): its first Horner step is one subtraction with one literal, and u = |x| s sqrt(2) / 4.1 - s
// is one FMA.
constexpr float kGeluS = 0.43911893f, kGeluU = 0.15146535f;  // s, s sqrt(2) / 4.1
constexpr float kGeluC0 = 2.019375f;                         // c6 / s^6 (the first Horner step: kGeluC0 - u)
constexpr float kGeluC[6] = {-2.2946658f, 2.3185021f, -2.3095699f, -29.120948f, -30.379971f,
                             -9.0620125f};  // c5 / s^5 .. c0 (c0 includes the -1 of the factor 1/2)
__device__ __forceinline__ float gelu_erf(float x) {
  const float u = fmaf(fabsf(x), kGeluU, -kGeluS);
  float p = kGeluC0 - u;  // -u^7 + (c6 / s^6) u^6: the first Horner step
#pragma unroll
  for (int k = 0; k < 6; ++k) p = fmaf(p, u, kGeluC[k]);
  return fmaf(-fabsf(x), __builtin_amdgcn_exp2f(p), __builtin_elementwise_maximum(x, -0.0f));
}

// GELU, tanh form (F.gelu(approximate="tanh")): 0.5 x (1 + tanh(y)), y = sqrt(2 / pi) (x + 0.044715 x^3), written
// as x / (1 + e^(-2 y)) (1 + tanh y = 2 / (1 + e^(-2 y))): one v_exp_f32 and a correctly rounded division, no
// cancellation in the negative tail (torch's 1 + tanh loses the low bits there; the two agree within |x| 2^-23 in
// absolute terms). Limits: e -> inf gives x / inf = -0 for large negative x (torch: 0.5 x (1 - 1) = -0), e -> 0 gives
// x; GELU(+-0) = +-0 and NaN stays NaN.
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float kTwoK = 2.0f * 0.79788456080286535588f * 1.44269504088896340736f;  // 2 sqrt(2/pi) log2(e)
  const float x2 = x * x;
  const float t = -kTwoK * fmaf(0.044715f * x2, x, x);
  return __fdiv_rn(x, 1.0f + __builtin_amdgcn_exp2f(t));
}

// gelu_erf over N independent values, written step by step (each Horner step over all N values before the next), so
// the N dependent chains interleave: the compiler otherwise schedules a value's whole chain before the next value's,
// two at a time, and the VALU waits on the chain latency. Same arithmetic per value as gelu_erf.
template <int N>
__device__ __forceinline__ void gelu_erf_n(float (&x)[N]) {
  float u[N], p[N];
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = fmaf(fabsf(x[i]), kGeluU, -kGeluS);
#pragma unroll
  for (int i = 0; i < N; ++i) p[i] = kGeluC0 - u[i];
#pragma unroll
  for (int k = 0; k < 6; ++k)
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = fmaf(p[i], u[i], kGeluC[k]);
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] = fmaf(-fabsf(x[i]), __builtin_amdgcn_exp2f(p[i]), __builtin_elementwise_maximum(x[i], -0.0f));
}

// Workgroup barrier for LDS hand-offs that leaves global loads in flight: waits only for this wave's LDS operations
// (lgkmcnt), unlike __syncthreads(), whose workgroup-scope fence also drains every outstanding global load (vmcnt) and
// so serializes prefetches with the MFMAs. The "memory" clobber keeps the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

inline int launch_status() {
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? FIM_OK : (int)err;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (cached per device; 256, MI355X's count, if the query fails).
inline int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cached[dev];
}

}  // namespace fim
