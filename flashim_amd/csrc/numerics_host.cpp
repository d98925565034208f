// Host build of numerics.h (the scalar rules every kernel uses), exported over arrays so the CPU test suite can check
// them against torch exhaustively without a GPU. Not part of the device library.
#include "numerics.h"

extern "C" {

void fim_host_e4m3(const float* x, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = fim::f32_to_e4m3_sw(x[i]);
}

void fim_host_e4m3_decode(const uint8_t* c, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = fim::e4m3_to_f32(c[i]);
}

void fim_host_mx_exponent(const float* amax, int64_t n, int8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = (int8_t)fim::mx_exponent_from_amax(amax[i]);
}

// mx_exponent_fast where it decides, else mx_exponent_from_amax; decided[i] = 1 where the fast path decided.
void fim_host_mx_exponent_fast(const float* amax, int64_t n, int8_t* out, uint8_t* decided) {
  for (int64_t i = 0; i < n; ++i) {
    int e = 0;
    decided[i] = fim::mx_exponent_fast(amax[i], e) ? 1 : 0;
    out[i] = (int8_t)(decided[i] ? e : fim::mx_exponent_from_amax(amax[i]));
  }
}

void fim_host_bf16(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = fim::f32_to_bf16(x[i]);
}

void fim_host_quantize_int8(const float* x, int64_t n, float scale, int8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = fim::quantize_int8_value(x[i], scale);
}

}  // extern "C"
