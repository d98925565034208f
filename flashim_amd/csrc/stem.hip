// The first convolution of a VGG encoder with its epilogue, and that epilogue on its own:
//   conv2d_small_cin_quantize_int8 (flashim/ops/conv.py:225-235): quantize_int8(relu(bf16(conv3x3(x)) + bias)),
//     x NCHW BF16 [B, Cin <= 8, H, W], stride 1, padding 1, INT8 NHWC [B, H, W, Cout] out;
//   bias_relu_quantize_int8 (flashim/ops/quantize.py:134-142): quantize_int8(relu(raw + bias)), raw NCHW BF16 (a
//     bias-free conv output), INT8 NHWC out.
// Rounding points as the references: the conv result is BF16 (cuDNN returns BF16; FP32 accumulation), the bias is
// added in the promoted dtype (BF16 + BF16 -> BF16: FP32 sum rounded to BF16; BF16 + FP32 -> FP32), ReLU, then
// round(v / scale) with torch's FP32 division, saturated to +-127.
//
// Stem conv: K = (c, ky, kx), 9 Cin taps, padded to KP = a multiple of 32 with zero weights; one
// v_mfma_f32_16x16x32_bf16 per 16 output channels and 32 taps (lane l supplies A[row l & 15][k 8 (l >> 4) + e] and
// B[k 8 (l >> 4) + e][col l & 15], e = 0..7, and gets D[row 4 (l >> 4) + r][col l & 15]; measured). Weights are A
// (rows = output channels), pixels are B, so a lane ends with 4 consecutive channels of one pixel. A workgroup takes a
// tile of 8 output rows x 64 columns: the Cin x 10 x 66 input patch is staged in LDS once, each wave owns a
// 16-column block and walks the 8 rows (tap offsets into the patch, bias and weights are per-lane registers set up
// once), and the INT8 codes of a row go through the wave's LDS slice so its 16 pixels x Cout bytes leave as one
// contiguous run of 16-byte stores. HBM-bound: 2 Cin bytes in and Cout bytes out per pixel.
#include <type_traits>

#include "common.h"

namespace fim {

constexpr int ST_SEG = 64;      // output columns per workgroup
constexpr int ST_TH = 8;        // output rows per workgroup
constexpr int ST_COLS = ST_SEG + 2;
constexpr int ST_MAX_CIN = 8;
constexpr int ST_MAX_COUT = 128;

typedef __bf16 v8bf16 __attribute__((ext_vector_type(8)));

struct StemArgs {
  const uint16_t* x;     // BF16 NCHW [B, Cin, H, W]
  const uint16_t* w;     // BF16 [Cout, KP]: tap k = 9 c + 3 ky + kx, zero for k >= 9 Cin
  const void* bias;      // [Cout] BF16 or FP32
  int bias_bf16;
  const float* scale;    // FP32 scalar
  int8_t* out;           // INT8 NHWC [B, H, W, Cout]
  int B, Cin, H, W, Cout, KP;
};

// v + bias: a BF16 bias adds in FP32 and rounds to BF16 (torch's BF16 + BF16); an FP32 bias keeps the FP32 sum (BF16 +
// FP32 promotes). The ReLU that follows is folded into the quantizer's saturation.
__device__ __forceinline__ float bias_add(float v, float b, bool bias_bf16) {
  const float t = __fadd_rn(v, b);
  return bias_bf16 ? round_bf16_hw(t) : t;
}

template <int NCH, int CHUNKS>  // Cout / 16; KP / 32
__global__ __launch_bounds__(256, (NCH <= 4 && CHUNKS == 1) ? 5 : 2) void stem_conv_kernel(const StemArgs a) {
  constexpr int COUT = NCH * 16;
  constexpr int PR = ST_TH + 2;  // staged input rows
  __shared__ uint16_t patch[ST_MAX_CIN * PR * ST_COLS + 1];         // [c][row][column], then one zero
  __shared__ __attribute__((aligned(16))) int8_t qs[4][16 * COUT];  // per wave: 16 pixels x Cout codes
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rows_per_image = (a.H + ST_TH - 1) / ST_TH;
  const int b = blockIdx.x / rows_per_image, oh0 = (blockIdx.x - b * rows_per_image) * ST_TH;
  const int ow0 = blockIdx.y * ST_SEG;

  // the input patch: rows oh0 - 1 .. oh0 + ST_TH, columns ow0 - 1 .. ow0 + 64 of every channel (zero outside);
  // 8 elements per thread per batch, loaded unconditionally from clamped in-image addresses, then selected
  const int n_patch = a.Cin * PR * ST_COLS;
  for (int i0 = 0; i0 < n_patch; i0 += 8 * 256) {
    uint16_t v[8];
    bool ok[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = min(i0 + tid + 256 * j, n_patch - 1);
      const int c = i / (PR * ST_COLS), r = i - c * (PR * ST_COLS);
      const int pr = r / ST_COLS, col = r - pr * ST_COLS;
      const int ih = oh0 + pr - 1, iw = ow0 + col - 1;
      ok[j] = ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
      v[j] = a.x[(((int64_t)b * a.Cin + c) * a.H + min(max(ih, 0), a.H - 1)) * a.W + min(max(iw, 0), a.W - 1)];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (i0 + tid + 256 * j < n_patch) patch[i0 + tid + 256 * j] = ok[j] ? v[j] : (uint16_t)0;
  }
  constexpr int ZERO = ST_MAX_CIN * PR * ST_COLS;  // padding taps (k >= 9 Cin) read this element
  if (tid == 0) patch[ZERO] = 0;
  // per lane: the patch offsets of its 8 taps per 32-tap chunk (relative to output row 0, column px), -1 for padding
  // taps; the bias of its 4 x NCH channels
  const int taps = 9 * a.Cin;
  int toff[CHUNKS][8];
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = 32 * ch + 8 * g + e;
      const int c = k / 9, r = k - 9 * c, ky = r / 3, kx = r - 3 * ky;
      toff[ch][e] = k < taps ? (c * PR + ky) * ST_COLS + kx : -1;  // -1: the zero element
    }
  // (all bias loads issued under one uniform branch; nothing waits on them before the first row's epilogue)
  float bias[NCH][4];
  if (a.bias_bf16) {
    uint2 raw[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) raw[i] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.bias) + 16 * i + 4 * g);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      bias[i][0] = u2f(raw[i].x << 16); bias[i][1] = u2f(raw[i].x & 0xffff0000u);
      bias[i][2] = u2f(raw[i].y << 16); bias[i][3] = u2f(raw[i].y & 0xffff0000u);
    }
  } else {
    float4 raw[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) raw[i] = *reinterpret_cast<const float4*>(static_cast<const float*>(a.bias) + 16 * i + 4 * g);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      bias[i][0] = raw[i].x; bias[i][1] = raw[i].y; bias[i][2] = raw[i].z; bias[i][3] = raw[i].w;
    }
  }
  v8bf16 wop[NCH][CHUNKS];  // weights (A): row 16 i + (lane & 15), taps [32 ch + 8 g, + 8)
#pragma unroll
  for (int i = 0; i < NCH; ++i)
#pragma unroll
    for (int ch = 0; ch < CHUNKS; ++ch) {
      const int kk = 32 * ch + 8 * g;
      wop[i][ch] = __builtin_bit_cast(v8bf16, *reinterpret_cast<const uint4*>(a.w + (int64_t)(16 * i + (lane & 15)) * a.KP + kk));
    }
  const float scale = *a.scale, inv = __fdiv_rn(1.0f, scale);
  const bool bias_bf16 = a.bias_bf16 != 0;
  __syncthreads();

  const int px = wave * 16 + (lane & 15);  // this lane's pixel (B column) within the segment
  const int npx = min(16, a.W - (ow0 + wave * 16));  // valid pixels of this wave's block
  int8_t* q_lds = qs[wave];
  for (int rr = 0; rr < ST_TH && oh0 + rr < a.H; ++rr) {
    v4f acc[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ch = 0; ch < CHUNKS; ++ch) {
      v8bf16 bop;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int o = toff[ch][e];
        bop[e] = __builtin_bit_cast(__bf16, patch[o >= 0 ? o + rr * ST_COLS + px : ZERO]);
      }
#pragma unroll
      for (int i = 0; i < NCH; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wop[i][ch], bop, acc[i], 0, 0, 0);
    }
    // epilogue: channels 16 i + 4 g + r of pixel px: BF16 conv result, + bias, ReLU, INT8
    float y[NCH * 4];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      float v0 = acc[i][0], v1 = acc[i][1], v2 = acc[i][2], v3 = acc[i][3];
      round_bf16x2(v0, v1);
      round_bf16x2(v2, v3);
      const float v[4] = {v0, v1, v2, v3};
#pragma unroll
      for (int r = 0; r < 4; ++r) y[4 * i + r] = __fadd_rn(v[r], bias[i][r]);
      if (bias_bf16) {
        round_bf16x2(y[4 * i], y[4 * i + 1]);
        round_bf16x2(y[4 * i + 2], y[4 * i + 3]);
      }
    }
    int q[NCH * 4];
    quantize_int8_fast_n<NCH * 4, 0>(y, scale, inv, q);  // the ReLU folds into the saturation
#pragma unroll
    for (int i = 0; i < NCH; ++i)
      *reinterpret_cast<uint32_t*>(&q_lds[(lane & 15) * COUT + 16 * i + 4 * g]) =
          (uint32_t)(uint8_t)q[4 * i] | ((uint32_t)(uint8_t)q[4 * i + 1] << 8) |
          ((uint32_t)(uint8_t)q[4 * i + 2] << 16) | ((uint32_t)(uint8_t)q[4 * i + 3] << 24);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the block's 16 pixels x Cout codes are contiguous in the output row: 16-byte pieces, lane-consecutive
    int8_t* dst = a.out + (((int64_t)b * a.H + oh0 + rr) * a.W + ow0 + wave * 16) * COUT;
    for (int i = lane; i < npx * NCH; i += 64)
      *reinterpret_cast<uint4*>(dst + (int64_t)i * 16) = *reinterpret_cast<const uint4*>(&q_lds[i * 16]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// bias_relu_quantize_int8: a tile of 64 channels x 64 pixels of one image plane; reads along pixels (NCHW rows),
// writes along channels (NHWC) through an LDS transpose.
__global__ __launch_bounds__(256) void bias_relu_quantize_kernel(const uint16_t* __restrict__ raw, int64_t C,
                                                                 int64_t HW, const void* bias, int bias_bf16,
                                                                 const float* scale_ptr, int8_t* __restrict__ out) {
  __shared__ int8_t t[64][64 + 4];  // [pixel][channel], padded against bank conflicts
  const int tid = threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64, b = blockIdx.z;
  const float scale = *scale_ptr, inv = __fdiv_rn(1.0f, scale);
  // read: 4 pixels per lane (8 bytes), 16 lanes per channel row, 16 channel rows per pass, 4 passes
  const int pl = (tid & 15) * 4, cr = tid >> 4;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int cl = cr + 16 * pass;
    const int64_t c = c0 + cl;
    if (c >= C) continue;
    const float bv = bias_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(bias)[c]) : static_cast<const float*>(bias)[c];
    const uint16_t* src = raw + (b * C + c) * HW + p0 + pl;
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = p0 + pl + e < HW ? bf16_to_f32(src[e]) : 0.0f;
      y[e] = bias_add(v, bv, bias_bf16 != 0);
    }
    int q[4];
    quantize_int8_fast_n<4, 0>(y, scale, inv, q);  // ReLU folded in
#pragma unroll
    for (int e = 0; e < 4; ++e) t[pl + e][cl] = (int8_t)q[e];
  }
  __syncthreads();
  // write: each lane 4 channels of one pixel (4 bytes); 16 lanes per pixel row of 64 channels
  const int cw = (tid & 15) * 4;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int pl2 = (tid >> 4) + 16 * pass;
    const int64_t p = p0 + pl2;
    if (p >= HW) continue;
    int8_t* dst = out + (b * HW + p) * C + c0 + cw;
    if (c0 + cw + 4 <= C && (C % 4) == 0) {
      *reinterpret_cast<uint32_t*>(dst) = (uint32_t)(uint8_t)t[pl2][cw] | ((uint32_t)(uint8_t)t[pl2][cw + 1] << 8) |
                                         ((uint32_t)(uint8_t)t[pl2][cw + 2] << 16) |
                                         ((uint32_t)(uint8_t)t[pl2][cw + 3] << 24);
    } else {
      for (int e = 0; e < 4; ++e)
        if (c0 + cw + e < C) dst[e] = t[pl2][cw + e];
    }
  }
}

}  // namespace fim

using namespace fim;

extern "C" {

// conv2d_small_cin_quantize_int8: w_packed [Cout, KP] BF16 (KP = 32 ceil(9 Cin / 32), tap k = 9 c + 3 ky + kx, zero
// padded); bias [Cout] (bias_dtype FIM_BF16 or FIM_F32); scale FP32 scalar; out INT8 NHWC [B, H, W, Cout].
int fim_conv3x3_small_cin_quantize_int8(const uint16_t* x, int64_t B, int64_t Cin, int64_t H, int64_t W,
                                        const uint16_t* w_packed, int64_t Cout, const void* bias, int bias_dtype,
                                        const float* scale, int8_t* out, hipStream_t stream) {
  if (x == nullptr || w_packed == nullptr || bias == nullptr || scale == nullptr || out == nullptr) return FIM_ERR_INVALID;
  if (B < 0 || H < 0 || W < 0 || Cin <= 0 || Cout <= 0) return FIM_ERR_INVALID;
  if (bias_dtype != FIM_BF16 && bias_dtype != FIM_F32) return FIM_ERR_INVALID;
  if (Cin > ST_MAX_CIN || Cout > ST_MAX_COUT || (Cout & (Cout - 1)) != 0 || Cout < 16) return FIM_ERR_UNSUPPORTED;
  if (((uintptr_t)w_packed % 16) != 0 || ((uintptr_t)out % 16) != 0 || ((uintptr_t)bias % 16) != 0)
    return FIM_ERR_UNSUPPORTED;
  if (B * H * W == 0) return FIM_OK;
  if (B * cdiv(H, ST_TH) > 2147483647LL || cdiv(W, ST_SEG) > 65535) return FIM_ERR_UNSUPPORTED;
  StemArgs a;
  a.x = x; a.w = w_packed; a.bias = bias; a.bias_bf16 = bias_dtype == FIM_BF16; a.scale = scale; a.out = out;
  a.B = (int)B; a.Cin = (int)Cin; a.H = (int)H; a.W = (int)W; a.Cout = (int)Cout;
  a.KP = (int)cdiv(9 * Cin, 32) * 32;
  const dim3 grid((unsigned)(B * cdiv(H, ST_TH)), (unsigned)cdiv(W, ST_SEG));
  const int chunks = a.KP / 32;  // 1 (Cin <= 3), 2 (Cin <= 7) or 3
  auto go = [&](auto nch) {
    constexpr int N = decltype(nch)::value;
    if (chunks == 1)
      stem_conv_kernel<N, 1><<<grid, dim3(256), 0, stream>>>(a);
    else if (chunks == 2)
      stem_conv_kernel<N, 2><<<grid, dim3(256), 0, stream>>>(a);
    else
      stem_conv_kernel<N, 3><<<grid, dim3(256), 0, stream>>>(a);
  };
  switch (Cout) {
    case 16: go(std::integral_constant<int, 1>{}); break;
    case 32: go(std::integral_constant<int, 2>{}); break;
    case 64: go(std::integral_constant<int, 4>{}); break;
    default: go(std::integral_constant<int, 8>{}); break;
  }
  return launch_status();
}

// bias_relu_quantize_int8: raw BF16 NCHW [B, C, H, W] -> INT8 NHWC [B, H, W, C].
int fim_bias_relu_quantize_int8(const uint16_t* raw, int64_t B, int64_t C, int64_t H, int64_t W, const void* bias,
                                int bias_dtype, const float* scale, int8_t* out, hipStream_t stream) {
  if (raw == nullptr || bias == nullptr || scale == nullptr || out == nullptr) return FIM_ERR_INVALID;
  if (B < 0 || C <= 0 || H < 0 || W < 0) return FIM_ERR_INVALID;
  if (bias_dtype != FIM_BF16 && bias_dtype != FIM_F32) return FIM_ERR_INVALID;
  const int64_t HW = H * W;
  if (B * HW == 0) return FIM_OK;
  if (B > 65535 || cdiv(C, 64) > 65535 || cdiv(HW, 64) > 2147483647LL) return FIM_ERR_UNSUPPORTED;
  if (((uintptr_t)out % 4) != 0) return FIM_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)cdiv(HW, 64), (unsigned)cdiv(C, 64), (unsigned)B);
  bias_relu_quantize_kernel<<<grid, dim3(256), 0, stream>>>(raw, C, HW, bias, bias_dtype == FIM_BF16, scale, out);
  return launch_status();
}

}  // extern "C"
