// Scalar numerics shared by every kernel of the quantized conv path: BF16 rounding, OCP E4M3 encoding, the MX
// block-exponent rule and the symmetric INT8 rounding. Each function states the torch expression it reproduces bit for
// bit, because the parity target is FlashIM's torch reference path:
//   flashim/quant/formats/mx.py:22-38   (scale_exponent_from_amax, quantize_blocks)
//   flashim/quant/formats/int8.py:24-27 (quantize_symmetric)
// Everything here is __host__ __device__ so the CPU test library can check it exhaustively against torch.
#pragma once

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define FIM_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#define FIM_HD static inline
#endif

namespace fim {

FIM_HD uint32_t f2u(float f) {
#ifdef __HIP_DEVICE_COMPILE__
  return __float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}

FIM_HD float u2f(uint32_t u) {
#ifdef __HIP_DEVICE_COMPILE__
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

// float -> bfloat16 bits, round to nearest even; NaN stays a quiet NaN (torch's c10::BFloat16 rounding).
FIM_HD uint16_t f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

FIM_HD float bf16_to_f32(uint16_t h) { return u2f(((uint32_t)h) << 16); }

// x rounded to BF16 and widened back: torch's `.to(torch.bfloat16).float()`.
FIM_HD float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// 2^e for an int8 MX exponent e in [-127, 127], exactly (2^-127 is an FP32 subnormal): torch.exp2(e.float()).
FIM_HD float exp2_int(int e) {
  if (e >= -126) return u2f((uint32_t)(e + 127) << 23);
  return u2f(0x00400000u);  // e == -127
}

// FP32 -> OCP E4M3 (float8_e4m3fn), round to nearest even, for |x| <= 448 (callers clamp first, as
// quantize_blocks does). Sign is kept, so negative values that round to zero give -0 (0x80) as torch does.
FIM_HD uint8_t f32_to_e4m3_sw(float x) {
  uint32_t u = f2u(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  uint32_t code;
  if (a >= 0x3c800000u) {  // |x| >= 2^-6: normal E4M3; round 23 mantissa bits to 3 (carry may bump the exponent)
    uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    code = (r >> 20) - (120u << 3);
  } else {  // subnormal E4M3: multiples of 2^-9; |x| * 2^9 is exact, then round half to even to an integer 0..8
    float q = u2f(a) * 512.0f;
#ifdef __HIP_DEVICE_COMPILE__
    code = (uint32_t)__builtin_rintf(q);
#else
    code = (uint32_t)rintf(q);
#endif
  }
  return (uint8_t)(sign | code);
}

// OCP E4M3 byte -> float (exact).
FIM_HD float e4m3_to_f32(uint8_t c) {
  uint32_t sign = (uint32_t)(c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  float mag;
  if (e == 0)
    mag = (float)m * (1.0f / 512.0f);
  else if (e == 15 && m == 7)
    mag = u2f(0x7fc00000u);
  else
    mag = u2f(((e + 120u) << 23) | (m << 20));
  return u2f(f2u(mag) | sign);
}

// MX block exponent of an FP32 block amax (flashim/quant/formats/mx.py:22-26):
//   e = ceil(log2(amax / 448)); e = -127 where amax == 0; clamp(-127, 127).
// torch evaluates amax / 448 with an IEEE FP32 division and log2 correctly rounded to FP32 (checked against torch's
// CPU log2 at every power-of-two boundary by the CPU tests). So q = amax / 448 is formed exactly as torch does, then
// ceil(RN_f32(log2 q)) is decided from q's bits: a power of two 2^k gives k; q = 2^k (1 + j 2^-23) gives k unless the
// FP32 rounding of k + log2(1 + j 2^-23) already lands on k, i.e. j <= ties_to_k(k). The thresholds below are the
// largest such j.
FIM_HD int mx_ties_to_k(int k) {
  // largest j >= 0 with RN_f32(k + log2(1 + j*2^-23)) == k. Spacing of FP32 just above |k| (k > 0) or just below |k|
  // (k < 0, the sum moves toward zero) decides it: j_max = floor(ln2 * 2^23 * half_spacing) (never a tie).
  if (k == 0) return 0;
  int ak = k > 0 ? k : -k;
  int msb = 31 - __builtin_clz((unsigned)ak);  // 2^msb <= |k| < 2^(msb+1)
  // spacing above |k| is 2^(msb-23); below |k| it is the same unless |k| is a power of two (then half of it)
  int sp_exp = msb - 23;
  if (k < 0 && (ak & (ak - 1)) == 0) sp_exp -= 1;
  // half spacing in units of 2^-23 of the mantissa: log2(1 + j 2^-23) ~= j 2^-23 / ln 2 < 2^(sp_exp - 1)
  // -> j < ln2 * 2^(sp_exp - 1 + 23)
  int p = sp_exp - 1 + 23;
  if (p < 0) return 0;
  // floor(ln2 * 2^p) for p = 0..6 (|k| <= 149 keeps p <= 6): 0, 1, 2, 5, 11, 22, 44; the FP32 product is exact in
  // its integer part (ln2 is 0.693 and the fraction parts stay 0.07 or more away from the next integer)
  return (int)(0.69314718f * (float)(1 << (p > 6 ? 6 : p)));
}

FIM_HD int mx_exponent_from_amax(float amax) {
  if (amax == 0.0f) return -127;
#ifdef __HIP_DEVICE_COMPILE__
  float q = __fdiv_rn(amax, 448.0f);
#else
  volatile float den = 448.0f;
  float q = amax / den;
#endif
  uint32_t u = f2u(q) & 0x7fffffffu;
  if (u >= 0x7f800000u) return 127;  // inf (NaN is not a valid amax here)
  if (u == 0) return -127;           // amax / 448 underflowed: log2(0) = -inf, clamped
  int k;
  uint32_t frac;
  if (u >= 0x00800000u) {
    k = (int)(u >> 23) - 127;
    frac = u & 0x7fffffu;
  } else {  // subnormal q: normalise
    int lz = __builtin_clz(u) - 8;  // shifts to bring the leading one to bit 23
    k = -126 - lz;
    frac = (u << lz) & 0x7fffffu;
  }
  int e;
  if (frac == 0)
    e = k;
  else
    e = ((int)frac <= mx_ties_to_k(k)) ? k : k + 1;
  if (e < -127) e = -127;
  if (e > 127) e = 127;
  return e;
}

// The same exponent without the division, for a finite amax >= 0, when it can be decided from q' = amax * RN(1/448):
// q' is within 2 units in the last place of q = RN(amax / 448) (two roundings of relative size 2^-24 each), so when
// q' is normal and its 23 fraction bits lie in [48, 2^23 - 4], q has the same exponent k and a fraction above every
// ties_to_k threshold (at most 44) and below the next power of two: e = k + 1. Returns false (e untouched) otherwise:
// zero, subnormal or non-finite q', or q' within a few units of a power of two, where mx_exponent_from_amax decides.
FIM_HD bool mx_exponent_fast(float amax, int& e) {
  const uint32_t u = f2u(amax * (1.0f / 448.0f));
  const uint32_t frac = u & 0x7fffffu;
  if (u < 0x00800000u || u >= 0x7f800000u || frac - 48u > 0x7fffffu - 3u - 48u) return false;
  e = (int)(u >> 23) - 126;
  return true;
}

// round(x / scale) half to even, saturated to +-127 (flashim/quant/formats/int8.py:24-27), IEEE FP32 division.
FIM_HD int8_t quantize_int8_value(float x, float scale) {
#ifdef __HIP_DEVICE_COMPILE__
  float q = __builtin_rintf(__fdiv_rn(x, scale));
#else
  volatile float s = scale;
  float q = rintf(x / s);
#endif
  q = q > 127.0f ? 127.0f : q;
  q = q < -127.0f ? -127.0f : q;
  return (int8_t)(int)q;
}

#ifdef __HIPCC__
// quantize_int8_value with the division replaced by a multiply by inv = 1 / scale (correctly rounded), falling back
// to the IEEE division only where it can matter: x * inv is within a few ulps of the exact quotient, so both round to
// the same integer unless the quotient sits within 2^-15 of a half-integer; beyond |q| = 127 both saturate. The
// rounding is one FMA with M = 1.5 * 2^23: fma(x, inv, M) rounds x * inv + M once, to the nearest integer (ties to
// even) on the grid of unit spacing where M sits, so its low mantissa bits hold rint(x * inv) and its low byte is the
// INT8 code in two's complement; r = f - M (exact) is the rounded quotient and fma(x, inv, -r) the exact residual, and
// |residual| >= 0.5 - 2^-15 marks a near-tie. The fallback sits behind one wave-uniform branch for all N values (taken
// when any lane is near a tie), so it neither runs per element nor splits the code that produces the inputs. The
// saturation is one v_med3_f32 between M - 127 and M + 127 (LO = 0 folds a preceding ReLU in: relu then quantize
// equals clamping the rounded quotient at 0), so no conversion to an integer is needed: q[i] holds the clamped value's
// bit pattern, whose low byte is the code (callers keep that byte). 5 VALU operations per value (FMA, subtraction,
// residual FMA, running maximum, med3), none on the scalar unit. Checked on the host
// against round(x / s) on 20M cases including exact ties and their neighbours, with and without the ReLU, and on the
// GPU byte for byte against the torch references of every INT8 producer.
template <int N, int LO = -127>
__device__ __forceinline__ void quantize_int8_fast_n(const float (&x)[N], float scale, float inv, int (&q)[N]) {
  constexpr float M = 12582912.0f;  // 1.5 * 2^23
  constexpr float NEAR = 0.5f - 0x1p-15f;
  float f[N];
  // the largest residual of the lane's values, one maximum each (a per-value compare would put each result in a
  // scalar register pair and OR them on the scalar unit, a dependent chain that cost more than the rest together)
  float worst = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    f[i] = fmaf(x[i], inv, M);
    worst = fmaxf(worst, fabsf(fmaf(x[i], inv, -(f[i] - M))));
  }
  if (__builtin_amdgcn_ballot_w64(worst >= NEAR) != 0) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (fabsf(fmaf(x[i], inv, -(f[i] - M))) >= NEAR) f[i] = __builtin_rintf(__fdiv_rn(x[i], scale)) + M;
  }
#pragma unroll
  for (int i = 0; i < N; ++i) q[i] = __builtin_bit_cast(int, __builtin_amdgcn_fmed3f(f[i], M + (float)LO, M + 127.0f));
}

__device__ __forceinline__ int8_t quantize_int8_fast(float x, float scale, float inv) {
  const float xs[1] = {x};
  int q[1];
  quantize_int8_fast_n<1>(xs, scale, inv, q);
  return (int8_t)q[0];
}
#endif

// One element of quantize_blocks + .to(float8_e4m3fn): clamp(x / 2^e, +-448) -> E4M3. Division by an exact power of
// two equals multiplication by its exact reciprocal (one rounding of the same real), so multiply.
FIM_HD float mx_scale_clamp(float x, float inv_scale) {
  float q = x * inv_scale;
#ifdef __HIP_DEVICE_COMPILE__
  // IEEE 754-2019 minimum / maximum (v_minimum3_f32, v_maximum3_f32 on gfx950): NaN stays NaN as in torch's clamp,
  // +-inf saturate, and no compare-select pair on VCC.
  return __builtin_elementwise_maximum(__builtin_elementwise_minimum(q, 448.0f), -448.0f);
#else
  q = q > 448.0f ? 448.0f : q;
  q = q < -448.0f ? -448.0f : q;
  return q;
#endif
}

}  // namespace fim
