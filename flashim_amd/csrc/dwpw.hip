// Depthwise 5x5 + bias + ReLU -> quantize -> pointwise GEMM + bias in one kernel, the fused MXFP8 refiner block of
// flashim/backends/triton/conv.py:310-420 (op flashim/ops/conv.py:93-117, depthwise5x5_relu_pointwise_mxfp8):
// relu(dwconv + bias) in FP32 -> dynamic per-(pixel, 32-channel) MXFP8 -> block-scaled GEMM with the weight's E8M0
// bytes (+ bias) -> BF16, for C = 128 input channels and a 128 x 128 pointwise weight (the reference's fused shape).
// The quantized activations never leave the CU: the result is, bit for bit, the two-launch composite (depthwise
// producer, then fim_mxfp8_scaled_mm) with the same MFMA per 16 x 16 output block. (The INT8 block runs as that
// two-launch composite: its intermediate is 1 byte per element, and the composite measured faster than a fused kernel.)
//
// Tile: 32 columns x 8 rows of one image, all 128 channels, per 256-lane workgroup (2 per CU by LDS):
//   depthwise, per 32-channel slice: the 12 x 36-pixel input window is staged channel-planar in LDS and the taps run
//   on v_mfma_f32_4x4x4_16b_bf16 exactly as in depthwise.hip (Toeplitz weight rows, 10 MFMAs per 16 channels x 4 x 4
//   outputs); the activated FP32 values go through LDS in two 4-row halves and a per-pixel pass (8 channels per lane,
//   4 lanes per pixel) quantizes them into the workgroup's activation tile [256 pixels][128 B] (XOR-swizzled 16-byte
//   slots, as the conv kernels' stages) with the MX exponents beside it;
//   pointwise: wave w takes pixels [64 w, 64 w + 64) x 128 output channels in two 64-channel passes, weights (staged
//   in LDS once) as the MFMA's A operand so each lane ends with 4 consecutive output channels of one pixel.
#include "common.h"

namespace fim {

constexpr int DP_TW = 32, DP_TH = 8, DP_C = 128, DP_CS = 32, DP_N = 128;
constexpr int DP_PX = DP_TW * DP_TH;                  // 256 pixels per tile
constexpr int DP_ROWSTR = 18;                         // dwords per staged input row (36 BF16 columns)
constexpr int DP_PLANE = (DP_TH + 4) * DP_ROWSTR + 2; // dwords per channel plane (218: 16 channels on distinct banks)
constexpr int DP_OROW = DP_TW * DP_CS + 16;           // dwords per staged FP32 output row (padded)
constexpr int DP_STAGE = DP_CS * DP_PLANE;            // 6976 dwords
static_assert(4 * DP_OROW <= DP_STAGE, "a 4-row output half fits in the input window's space");


struct DwPwArgs {
  const uint16_t* x;        // BF16 [B, H, W, 128]
  const uint16_t* dw_w;     // BF16 [25, 128]
  const float* dw_b;        // FP32 [128]
  const uint8_t* pw_w;      // E4M3 [128, 128]
  const uint8_t* pw_e8m0;   // [128, 4] E8M0 bytes
  const void* pw_b;         // [128] or null
  int pw_b_dtype;
  uint16_t* out;            // BF16 [B, H, W, 128]
  int B, H, W;
  int tiles_x, tiles_y;
  int64_t ntiles;           // tiles_x * tiles_y * B
};

typedef __bf16 v4bf16 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256, 2) void dw_pw_kernel(const DwPwArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t sm[DP_STAGE];           // input window / FP32 output half
  __shared__ __attribute__((aligned(16))) uint8_t act[DP_PX * DP_C];       // quantized activations [px][128 B]
  __shared__ __attribute__((aligned(16))) uint8_t wts[DP_N * DP_C];        // pointwise weight [n][128 B]
  __shared__ int8_t aexp[DP_PX * 4];                                        // MX exponents [px][32-channel block]
  __shared__ float pb[DP_N];                                                // pointwise bias
  __shared__ uint8_t pe[DP_N * 4];                                          // MX weight E8M0 [n][block]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware tile order (workgroup p runs on XCD p % 8): each XCD takes a contiguous run of tiles, column tiles
  // fastest, so a tile's row neighbours, which share 4 of its 12 input rows, read through the same L2 shortly after
  const int64_t L = (int64_t)(blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  if (L >= a.ntiles) return;
  const int x0 = (int)(L % a.tiles_x) * DP_TW;
  const int y0 = (int)((L / a.tiles_x) % a.tiles_y) * DP_TH;
  const int b = (int)(L / ((int64_t)a.tiles_x * a.tiles_y));
  const int rows = min(DP_TH, a.H - y0), cols = min(DP_TW, a.W - x0);

  // pointwise weight and per-channel operands, staged once (swizzle: 16-byte slot s of row n at s ^ ((n >> 1) & 7))
  for (int idx = tid; idx < DP_N * DP_C / 16; idx += 256) {
    const int n = idx >> 3, seg = idx & 7;
    *reinterpret_cast<uint4*>(&wts[n * DP_C + ((seg ^ ((n >> 1) & 7)) << 4)]) =
        *reinterpret_cast<const uint4*>(a.pw_w + n * DP_C + seg * 16);
  }
  if (tid < DP_N) {
    float bias = -0.0f;  // x + (-0) == x for every x: added unconditionally
    if (a.pw_b != nullptr)
      bias = a.pw_b_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.pw_b)[tid])
                                      : static_cast<const float*>(a.pw_b)[tid];
    pb[tid] = bias;
    *reinterpret_cast<uint32_t*>(&pe[4 * tid]) = reinterpret_cast<const uint32_t*>(a.pw_e8m0)[tid];
  }

  // ---- depthwise, one 32-channel slice at a time -------------------------------------------------------------------
  const int cg = wave & 1, rq = wave >> 1;  // 16-channel group of the slice; output row quad (rows 4 rq .. 4 rq + 3)
  const int bch = lane >> 2, r4 = lane & 3;
  const uint16_t* xb = a.x + (int64_t)b * a.H * a.W * DP_C;
  float* st = reinterpret_cast<float*>(sm);
  for (int s = 0; s < DP_C / DP_CS; ++s) {
    const int cbase = s * DP_CS;
    __syncthreads();  // the previous slice's output pass is done with sm
    // stage: unit (row r, 4-column group q, channel octet o): 4 pixels x 8 channels, transposed (v_perm) into 8
    // channel rows of 4 BF16; unconditional loads from clamped in-image addresses, zeros outside the image
    for (int u = tid; u < (DP_TH + 4) * 9 * 4; u += 256) {
      const int o = u & 3, rqq = u >> 2;
      const int r = rqq / 9, q = rqq - r * 9;
      const int iy = y0 - 2 + r;
      const bool row_ok = iy >= 0 && iy < a.H;
      const uint16_t* src_row = xb + (int64_t)min(max(iy, 0), a.H - 1) * a.W * DP_C + cbase + 8 * o;
      uint32_t P[4][4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int ix = x0 - 2 + 4 * q + k;
        const bool ok = row_ok && ix >= 0 && ix < a.W;
        const uint4 v = *reinterpret_cast<const uint4*>(src_row + (int64_t)min(max(ix, 0), a.W - 1) * DP_C);
        P[k][0] = ok ? v.x : 0u; P[k][1] = ok ? v.y : 0u; P[k][2] = ok ? v.z : 0u; P[k][3] = ok ? v.w : 0u;
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {  // dword m of a pixel = channels 8 o + 2 m (low half), + 1 (high half)
        const uint32_t lo01 = __builtin_amdgcn_perm(P[1][m], P[0][m], 0x05040100u);
        const uint32_t lo23 = __builtin_amdgcn_perm(P[3][m], P[2][m], 0x05040100u);
        const uint32_t hi01 = __builtin_amdgcn_perm(P[1][m], P[0][m], 0x07060302u);
        const uint32_t hi23 = __builtin_amdgcn_perm(P[3][m], P[2][m], 0x07060302u);
        const int c0 = 8 * o + 2 * m;
        *reinterpret_cast<uint2*>(&sm[c0 * DP_PLANE + r * DP_ROWSTR + 2 * q]) = make_uint2(lo01, lo23);
        *reinterpret_cast<uint2*>(&sm[(c0 + 1) * DP_PLANE + r * DP_ROWSTR + 2 * q]) = make_uint2(hi01, hi23);
      }
    }
    // this lane's channel and Toeplitz weight rows (segment 0: v shifted up by r4 BF16 elements, segment 1: u shifted
    // down by 3 - r4, with v = w[ky][0..3], u = w[ky][1..4] packed 16 bits apart)
    const int ch = cbase + 16 * cg + bch;
    v4bf16 wa[5][2];
#pragma unroll
    for (int ky = 0; ky < 5; ++ky) {
      uint64_t w5[5];
#pragma unroll
      for (int kx = 0; kx < 5; ++kx) w5[kx] = a.dw_w[(ky * 5 + kx) * DP_C + ch];
      const uint64_t v = w5[0] | (w5[1] << 16) | (w5[2] << 32) | (w5[3] << 48);
      const uint64_t u = w5[1] | (w5[2] << 16) | (w5[3] << 32) | (w5[4] << 48);
      wa[ky][0] = __builtin_bit_cast(v4bf16, v << (16 * r4));
      wa[ky][1] = __builtin_bit_cast(v4bf16, u >> (16 * (3 - r4)));
    }
    const float dbias = a.dw_b[ch];
    __syncthreads();  // window staged

    v4f acc[8];  // [column quad cq]: D[i = 0..3][j = r4] = output (row 4 rq + r4, column 4 cq + i)
#pragma unroll
    for (int cq = 0; cq < 8; ++cq) acc[cq] = v4f{dbias, dbias, dbias, dbias};  // the bias first, as depthwise.hip
    const uint32_t* plane = &sm[(16 * cg + bch) * DP_PLANE];
#pragma unroll
    for (int ky = 0; ky < 5; ++ky) {
      const uint32_t* rowp = plane + (4 * rq + r4 + ky) * DP_ROWSTR;
#pragma unroll
      for (int cq = 0; cq < 8; ++cq)
#pragma unroll
        for (int sg = 0; sg < 2; ++sg) {
          const uint2 raw = *reinterpret_cast<const uint2*>(rowp + 2 * cq + 2 * sg);
          acc[cq] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(wa[ky][sg], __builtin_bit_cast(v4bf16, raw), acc[cq], 0,
                                                           0, 0);
        }
    }
    float y[8][4];
#pragma unroll
    for (int cq = 0; cq < 8; ++cq)
#pragma unroll
      for (int i = 0; i < 4; ++i) y[cq][i] = fmaxf(acc[cq][i], 0.f);

#pragma unroll
    for (int half = 0; half < 2; ++half) {
      __syncthreads();  // half 0: the taps are done with the window; half 1: the previous pass is done
      if (rq == half) {
#pragma unroll
        for (int cq = 0; cq < 8; ++cq)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[r4 * DP_OROW + (4 * cq + i) * DP_CS + 16 * cg + bch] = y[cq][i];
      }
      __syncthreads();
      // per pixel: 4 rows x 32 columns x 4 parts of 8 channels; 4 consecutive lanes share a pixel
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int unit = tid + 256 * it;
        const int part = unit & 3, pxh = unit >> 2;
        const int rl = pxh >> 5, col = pxh & 31;
        const float4 va = *reinterpret_cast<const float4*>(&st[rl * DP_OROW + col * DP_CS + 8 * part]);
        const float4 vb = *reinterpret_cast<const float4*>(&st[rl * DP_OROW + col * DP_CS + 8 * part + 4]);
        float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
        uint2 codes;
        const int p = (4 * half + rl) * DP_TW + col;  // tile pixel
        // the values are >= 0 (ReLU): the amax is a plain max and the clamp is one-sided
        float amax = fmaxf(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])), fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
        amax = fmaxf(amax, __shfl_xor(amax, 1));
        amax = fmaxf(amax, __shfl_xor(amax, 2));
        const int ex = mx_exponent_wave(amax);
        const float inv = exp2_int(-ex);
        float q[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = __builtin_elementwise_minimum(v[e] * inv, 448.0f);
        codes = make_uint2(pack_e4m3x4(q[0], q[1], q[2], q[3]), pack_e4m3x4(q[4], q[5], q[6], q[7]));
        if (part == 0) aexp[p * 4 + s] = (int8_t)ex;
        const int seg = 2 * s + (part >> 1);  // 16-byte slot of channels [32 s + 8 part, + 8)
        *reinterpret_cast<uint2*>(&act[p * DP_C + ((seg ^ ((p >> 1) & 7)) << 4) + 8 * (part & 1)]) = codes;
      }
    }
  }
  __syncthreads();  // activation tile complete

  // ---- pointwise: wave w, pixels [64 w, 64 w + 64), output channels in two passes of 64 --------------------------
  const int g = lane >> 4, r16 = lane & 15;
  v8i xf[4];
  int sx[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int p = 64 * wave + 16 * j + r16;
    const v4i lo = *reinterpret_cast<const v4i*>(&act[p * DP_C + ((g ^ ((p >> 1) & 7)) << 4)]);
    const v4i hi = *reinterpret_cast<const v4i*>(&act[p * DP_C + (((g + 4) ^ ((p >> 1) & 7)) << 4)]);
    xf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    sx[j] = (int)aexp[p * 4 + g] + 127;  // lane group g scales K block g = channel slice g
  }
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    v4f acc_f[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 64 * pass + 16 * i + r16;
      const v4i wl = *reinterpret_cast<const v4i*>(&wts[n * DP_C + ((g ^ ((n >> 1) & 7)) << 4)]);
      const v4i wh = *reinterpret_cast<const v4i*>(&wts[n * DP_C + (((g + 4) ^ ((n >> 1) & 7)) << 4)]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v8i wf = __builtin_shufflevector(wl, wh, 0, 1, 2, 3, 4, 5, 6, 7);
        acc_f[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf, xf[j], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0,
                                                                       (int)pe[n * 4 + g], 0, sx[j]);
      }
    }
    // epilogue: + bias, BF16, 4 channels of one pixel per store
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = 64 * wave + 16 * j + r16;
      const int py = p >> 5, pxx = p & 31;
      const bool ok = py < rows && pxx < cols;
      uint16_t* dst = a.out + (((int64_t)b * a.H + y0 + py) * a.W + x0 + pxx) * DP_N;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n0 = 64 * pass + 16 * i + 4 * g;
        float yv[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          yv[v] = __fadd_rn(acc_f[i][j][v], pb[n0 + v]);
        }
        if (ok) *reinterpret_cast<uint2*>(dst + n0) = make_uint2(pack_bf16x2(yv[0], yv[1]), pack_bf16x2(yv[2], yv[3]));
      }
    }
  }
}

}  // namespace fim

using namespace fim;

static int dwpw_launch(const DwPwArgs& a, int64_t C, int64_t N, hipStream_t stream) {
  if (a.x == nullptr || a.dw_w == nullptr || a.dw_b == nullptr || a.pw_w == nullptr || a.out == nullptr)
    return FIM_ERR_INVALID;
  if (a.B < 0 || a.H < 0 || a.W < 0) return FIM_ERR_INVALID;
  if (C != DP_C || N != DP_N) return FIM_ERR_UNSUPPORTED;
  if (((uintptr_t)a.x % 16) != 0 || ((uintptr_t)a.pw_w % 16) != 0 || ((uintptr_t)a.out % 8) != 0 ||
      ((uintptr_t)a.dw_w % 2) != 0)
    return FIM_ERR_UNSUPPORTED;
  if ((int64_t)a.B * a.H * a.W == 0) return FIM_OK;
  DwPwArgs t = a;
  t.tiles_x = (int)cdiv(a.W, DP_TW);
  t.tiles_y = (int)cdiv(a.H, DP_TH);
  t.ntiles = (int64_t)t.tiles_x * t.tiles_y * a.B;
  if (t.ntiles > (1LL << 31) - 8) return FIM_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)(cdiv(t.ntiles, 8) * 8));  // a multiple of the 8 XCDs
  dw_pw_kernel<<<grid, dim3(256), 0, stream>>>(t);
  return launch_status();
}

extern "C" {

int fim_depthwise5x5_relu_pointwise_mxfp8(const uint16_t* x, int64_t B, int64_t H, int64_t W, int64_t C,
                                          const uint16_t* dw_weight, const float* dw_bias, const uint8_t* pw_weight,
                                          int64_t N, const uint8_t* pw_scale_e8m0, const void* pw_bias,
                                          int pw_bias_dtype, uint16_t* out, hipStream_t stream) {
  if (pw_scale_e8m0 == nullptr || ((uintptr_t)pw_scale_e8m0 % 4) != 0) return FIM_ERR_INVALID;
  if (B > 2147483647LL || H > 2147483647LL || W > 2147483647LL || B * H * W * C >= (1LL << 40))
    return FIM_ERR_UNSUPPORTED;
  DwPwArgs a{x, dw_weight, dw_bias, pw_weight, pw_scale_e8m0, pw_bias, pw_bias_dtype, out,
             (int)B, (int)H, (int)W, 0, 0, 0};
  return dwpw_launch(a, C, N, stream);
}

}  // extern "C"
