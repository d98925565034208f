// Depthwise 5x5 (pad 2, stride 1) producers of the depthwise-then-pointwise refiner block:
//   ACT_RELU + OUT_MX_DYNAMIC  depthwise5x5_relu_mxfp8   flashim/ops/conv.py:30-44
//                              (relu(dwconv + bias) in FP32 -> per-(pixel, 32-channel) dynamic MXFP8, swizzled scales)
//   ACT_RELU + OUT_INT8        depthwise5x5_relu_int8    flashim/ops/conv.py:50-61
//                              (relu(dwconv + bias) -> BF16 -> static INT8)
//   ACT_GELU + OUT_{BF16, INT8, MX_STATIC}: the folded-BatchNorm + GELU step of the conv-refiner block
//                              (dwconv + bias -> BF16 -> GELU -> BF16 [-> static INT8 / static MXFP8]), the rounding
//                              points of a BF16 depthwise conv followed by nn.GELU and the consumer's quantize
//                              (flashim/ops/quantize.py:63-74, 91-100).
//
// Layout: input BF16 NHWC [B, H, W, C] (the channels-last memory of [B, C, H, W]); weight BF16 [25, C] (ky, kx major,
// flashim/quant/passes/separable_conv_block.py:52-55); bias FP32 [C]. Output row = pixel (b, y, x), C channels.
//
// Work split: see the tile and matrix-unit comments below (dw5x5_mfma_kernel).
#include <type_traits>

#include "common.h"

namespace fim {

enum { ACT_RELU = 0, ACT_GELU = 1 };
enum { DW_MX_DYNAMIC = 0, DW_INT8 = 1, DW_BF16 = 2, DW_MX_STATIC = 3 };

struct DwArgs {
  const uint16_t* x;
  const uint16_t* w;
  const float* bias;
  const float* scale;      // INT8
  const int8_t* expo;      // MX static [C / 32]
  void* out;
  uint8_t* swizzled;       // MX dynamic scales (cuBLAS 128x4 layout), may be null
  int8_t* expo_out;        // MX dynamic exponents [rows, C / 32], may be null
  int B, H, W, C;
  int tiles_x, tiles_y;    // column and row tiles per image
  int64_t ntiles;          // tiles_x * tiles_y * B * (C / 32)
};

// Tile: 32 output columns x 16 output rows x 32 channels per workgroup (a 1-D grid over (channel slice, column tile,
// row tile, image), XCD-aware), with the 2-pixel halo of the 5x5 window staged in LDS once.
constexpr int DW_TW = 32, DW_TH = 16, DW_CS = 32;  // output columns, output rows, channels per workgroup

// ---- The taps on the matrix unit ----------------------------------------------------------------------------
// v_mfma_f32_4x4x4_16b_bf16 runs 16 independent 4x4x4 products per instruction; each is one channel: D[i][j] (output
// columns 4 cq + i, output row 4 rq + j) += A[i][k] B[k][j] with A the Toeplitz matrix of one weight row, A[i][k] =
// w[ky][4 s + k - i] (zero outside 0..4), and B[k][j] = input (row 4 rq + j + ky, column 4 cq + 4 s + k) of the staged
// tile (origin y0 - 2, x0 - 2): 5 weight rows x 2 column segments s = 10 MFMAs per 16 channels x 4 x 4 outputs.
// Operand layout (measured): lane l = 4 b + r supplies A_b[r][0..3] and B_b[0..3][r] and gets D_b[0..3][r].
// The tile is staged channel-planar ([channel][row][column] BF16, 40 columns per row, planes 402 dwords apart so the
// 16 channels of an instruction fall on different banks) so each B operand is one 8-byte LDS read. After the taps the
// activated FP32 values go through LDS in two 8-row halves ([row][column][channel], rows padded by 16 dwords) and the
// output pass writes per pixel: 8 channels per lane, MX dynamic exponents from 4-lane amax shuffles.
constexpr int DWM_ROWSTR = 20;                      // dwords per staged row (40 columns, 36 used)
constexpr int DWM_PLANE = 20 * DWM_ROWSTR + 2;      // dwords per channel plane
constexpr int DWM_LDS = DW_CS * DWM_PLANE;          // 12864 dwords
constexpr int DWM_OROW = DW_TW * DW_CS + 16;        // dwords per staged output row (FP32, padded)
static_assert(8 * DWM_OROW <= DWM_LDS, "an 8-row output half fits in the input tile's space");

typedef __bf16 v4bf16 __attribute__((ext_vector_type(4)));

template <int ACT, int OUT>
__global__ __launch_bounds__(256, 3) void dw5x5_mfma_kernel(const DwArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t sm[DWM_LDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware tile order: workgroup p runs on XCD p % 8, so each XCD takes a contiguous run of tiles in (channel slice,
  // column tile, row tile, image) order, slice fastest: the slices of a pixel (which share its 128-byte input lines)
  // and neighbouring column tiles (which share halo columns) read through the same L2 at about the same time.
  // (One workgroup per tile in a 3-D grid read each input line from HBM about three times.)
  const int cslices = a.C / DW_CS;
  const int64_t L = (int64_t)(blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  if (L >= a.ntiles) return;
  const int cbase = (int)(L % cslices) * DW_CS;
  int64_t rest = L / cslices;
  const int x0 = (int)(rest % a.tiles_x) * DW_TW;
  rest /= a.tiles_x;
  const int y0 = (int)(rest % a.tiles_y) * DW_TH;
  const int b = (int)(rest / a.tiles_y);

  // stage: unit (row r, 4-column group q, channel octet o): 4 pixels x 8 channels, transposed (v_perm) into 8
  // channel rows of 4 BF16, one 8-byte LDS write each; loads unconditional from clamped in-image addresses
  for (int u = tid; u < 20 * 10 * 4; u += 256) {
    const int o = u & 3, rq = u >> 2;
    const int r = rq / 10, q = rq - r * 10;
    const int iy = y0 - 2 + r;
    const bool row_ok = iy >= 0 && iy < a.H;
    const uint16_t* src_row = a.x + ((int64_t)b * a.H + min(max(iy, 0), a.H - 1)) * a.W * a.C + cbase + 8 * o;
    uint32_t P[4][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int ix = x0 - 2 + 4 * q + k;
      const bool ok = row_ok && ix >= 0 && ix < a.W;
      const uint4 v = *reinterpret_cast<const uint4*>(src_row + (int64_t)min(max(ix, 0), a.W - 1) * a.C);
      P[k][0] = ok ? v.x : 0u; P[k][1] = ok ? v.y : 0u; P[k][2] = ok ? v.z : 0u; P[k][3] = ok ? v.w : 0u;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {  // dword m of a pixel = channels 8 o + 2 m (low half), + 1 (high half)
      const uint32_t lo01 = __builtin_amdgcn_perm(P[1][m], P[0][m], 0x05040100u);
      const uint32_t lo23 = __builtin_amdgcn_perm(P[3][m], P[2][m], 0x05040100u);
      const uint32_t hi01 = __builtin_amdgcn_perm(P[1][m], P[0][m], 0x07060302u);
      const uint32_t hi23 = __builtin_amdgcn_perm(P[3][m], P[2][m], 0x07060302u);
      const int c0 = 8 * o + 2 * m;
      *reinterpret_cast<uint2*>(&sm[c0 * DWM_PLANE + r * DWM_ROWSTR + 2 * q]) = make_uint2(lo01, lo23);
      *reinterpret_cast<uint2*>(&sm[(c0 + 1) * DWM_PLANE + r * DWM_ROWSTR + 2 * q]) = make_uint2(hi01, hi23);
    }
  }

  // this lane's channel (block b of the wave's 16-channel group) and row/column index r4 within the 4 x 4 blocks
  const int cg = wave & 1, rh = wave >> 1;  // channel group; row half (row quads 2 rh, 2 rh + 1)
  const int bch = lane >> 2, r4 = lane & 3;
  const int ch = cbase + 16 * cg + bch;
  // A operands: row r4 of the Toeplitz matrix of weight row ky, column segment s. With v = (w0, w1, w2, w3) and
  // u = (w1, w2, w3, w4) as 64-bit vectors of BF16 (element k in bits 16 k), segment 0 is v shifted up by r4 elements
  // (zeros enter below) and segment 1 is u shifted down by 3 - r4 elements.
  v4bf16 wa[5][2];
#pragma unroll
  for (int ky = 0; ky < 5; ++ky) {
    uint64_t w5[5];
#pragma unroll
    for (int kx = 0; kx < 5; ++kx) w5[kx] = a.w[(ky * 5 + kx) * a.C + ch];
    const uint64_t v = w5[0] | (w5[1] << 16) | (w5[2] << 32) | (w5[3] << 48);
    const uint64_t u = w5[1] | (w5[2] << 16) | (w5[3] << 32) | (w5[4] << 48);
    wa[ky][0] = __builtin_bit_cast(v4bf16, v << (16 * r4));
    wa[ky][1] = __builtin_bit_cast(v4bf16, u >> (16 * (3 - r4)));
  }
  const float bias = a.bias[ch];
  __syncthreads();

  v4f acc[2][8];  // [row quad 2 rh + t][column quad cq]: D[i = 0..3][j = r4]
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int cq = 0; cq < 8; ++cq) acc[t][cq] = v4f{0.f, 0.f, 0.f, 0.f};
  const uint32_t* plane = &sm[(16 * cg + bch) * DWM_PLANE];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int ky = 0; ky < 5; ++ky) {
      const uint32_t* rowp = plane + (4 * (2 * rh + t) + r4 + ky) * DWM_ROWSTR;
#pragma unroll
      for (int cq = 0; cq < 8; ++cq)
#pragma unroll
        for (int sg = 0; sg < 2; ++sg) {
          const uint2 raw = *reinterpret_cast<const uint2*>(rowp + 2 * cq + 2 * sg);
          acc[t][cq] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(wa[ky][sg], __builtin_bit_cast(v4bf16, raw), acc[t][cq],
                                                              0, 0, 0);
        }
    }

  // activation in registers (bias; ReLU, or BF16 rounding + GELU + rounding), for all 64 values of the lane
  float y[2][8][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int cq = 0; cq < 8; ++cq)
#pragma unroll
      for (int i = 0; i < 4; ++i) y[t][cq][i] = acc[t][cq][i] + bias;
  if (ACT == ACT_RELU) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int cq = 0; cq < 8; ++cq)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[t][cq][i] = fmaxf(y[t][cq][i], 0.f);
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int cq = 0; cq < 8; ++cq) {
        float* v = y[t][cq];
        round_bf16x2(v[0], v[1]);
        round_bf16x2(v[2], v[3]);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gelu_erf(v[i]);
        if (OUT != DW_MX_STATIC) {  // static MXFP8 rounds to BF16 in its conversion (e4m3x4_of_bf16)
          round_bf16x2(v[0], v[1]);
          round_bf16x2(v[2], v[3]);
        }
      }
  }

  float oscale = 0.f, oinv8 = 1.f, oinv = 1.f;
  if (OUT == DW_INT8) {
    oscale = *a.scale;
    oinv8 = __fdiv_rn(1.0f, oscale);
  }
  float osc = 1.f;
  if (OUT == DW_MX_STATIC) {
    oinv = exp2_int(-(int)a.expo[cbase >> 5]);
    osc = exp2_int((int)a.expo[cbase >> 5]);
  }
  const int64_t groups = a.C >> 5;
  const int64_t tiles_k = (groups + 3) >> 2;
  const int rows = min(DW_TH, a.H - y0), cols = min(DW_TW, a.W - x0);
  float* st = reinterpret_cast<float*>(sm);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    __syncthreads();  // half 0: the taps are done with the input tile; half 1: the previous output pass is done
    if (rh == half) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int cq = 0; cq < 8; ++cq)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            st[(4 * t + r4) * DWM_OROW + (4 * cq + i) * DW_CS + 16 * cg + bch] = y[t][cq][i];
    }
    __syncthreads();
    // output pass: 8 rows x 32 columns x 4 parts of 8 channels; 4 consecutive lanes share a pixel
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int unit = tid + 256 * it;
      const int part = unit & 3, px = unit >> 2;  // px: 8 rows x 32 columns
      const int rl = px >> 5, col = px & 31;
      const int oy = 8 * half + rl;
      const float4 va = *reinterpret_cast<const float4*>(&st[rl * DWM_OROW + col * DW_CS + 8 * part]);
      const float4 vb = *reinterpret_cast<const float4*>(&st[rl * DWM_OROW + col * DW_CS + 8 * part + 4]);
      float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
      const bool ok = oy < rows && col < cols;
      const int64_t row = ((int64_t)b * a.H + y0 + oy) * a.W + x0 + col;
      const int c = cbase + 8 * part;
      if (OUT == DW_MX_DYNAMIC) {
        float amax = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
        amax = fmaxf(amax, __shfl_xor(amax, 1));
        amax = fmaxf(amax, __shfl_xor(amax, 2));
        const int ex = mx_exponent_from_amax(amax);
        const float inv = exp2_int(-ex);
        if (ok) {
          *reinterpret_cast<uint2*>(static_cast<uint8_t*>(a.out) + row * a.C + c) =
              make_uint2(pack_e4m3x4(mx_scale_clamp(v[0], inv), mx_scale_clamp(v[1], inv), mx_scale_clamp(v[2], inv),
                                     mx_scale_clamp(v[3], inv)),
                         pack_e4m3x4(mx_scale_clamp(v[4], inv), mx_scale_clamp(v[5], inv), mx_scale_clamp(v[6], inv),
                                     mx_scale_clamp(v[7], inv)));
          if (part == 0) {
            const int64_t gi = cbase >> 5;
            if (a.expo_out != nullptr) a.expo_out[row * groups + gi] = (int8_t)ex;
            if (a.swizzled != nullptr) {
              const int64_t rt = row & 127;
              a.swizzled[(((row >> 7) * tiles_k + (gi >> 2)) << 9) + (rt & 31) * 16 + (rt >> 5) * 4 + (gi & 3)] =
                  (uint8_t)(ex + 127);
            }
          }
        }
      } else if (OUT == DW_INT8) {
        if (ACT == ACT_RELU) {
#pragma unroll
          for (int e = 0; e < 8; e += 2) round_bf16x2(v[e], v[e + 1]);
        }
        int qi[8];
        quantize_int8_fast_n<8>(v, oscale, oinv8, qi);
        if (ok) {
          uint32_t q0 = 0, q1 = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            q0 |= (uint32_t)(uint8_t)qi[e] << (8 * e);
            q1 |= (uint32_t)(uint8_t)qi[4 + e] << (8 * e);
          }
          *reinterpret_cast<uint2*>(static_cast<uint8_t*>(a.out) + row * a.C + c) = make_uint2(q0, q1);
        }
      } else if (OUT == DW_MX_STATIC) {
        uint2 codes;
        if (ACT == ACT_GELU) {  // BF16 rounding and static E4M3 in one step (the values arrive unrounded)
          codes = make_uint2(e4m3x4_of_bf16(v[0], v[1], v[2], v[3], osc, 448.0f * osc),
                             e4m3x4_of_bf16(v[4], v[5], v[6], v[7], osc, 448.0f * osc));
        } else {
          codes = make_uint2(pack_e4m3x4(mx_scale_clamp(v[0], oinv), mx_scale_clamp(v[1], oinv),
                                         mx_scale_clamp(v[2], oinv), mx_scale_clamp(v[3], oinv)),
                             pack_e4m3x4(mx_scale_clamp(v[4], oinv), mx_scale_clamp(v[5], oinv),
                                         mx_scale_clamp(v[6], oinv), mx_scale_clamp(v[7], oinv)));
        }
        if (ok) *reinterpret_cast<uint2*>(static_cast<uint8_t*>(a.out) + row * a.C + c) = codes;
      } else {
        if (ok)
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + row * a.C + c) =
              make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                         pack_bf16x2(v[6], v[7]));
      }
    }
  }
}

template <int ACT>
static void dw_launch_out(const DwArgs& a, int out_mode, dim3 grid, hipStream_t s) {
  switch (out_mode) {
    case DW_MX_DYNAMIC: dw5x5_mfma_kernel<ACT, DW_MX_DYNAMIC><<<grid, dim3(256), 0, s>>>(a); break;
    case DW_INT8: dw5x5_mfma_kernel<ACT, DW_INT8><<<grid, dim3(256), 0, s>>>(a); break;
    case DW_BF16: dw5x5_mfma_kernel<ACT, DW_BF16><<<grid, dim3(256), 0, s>>>(a); break;
    default: dw5x5_mfma_kernel<ACT, DW_MX_STATIC><<<grid, dim3(256), 0, s>>>(a); break;
  }
}

}  // namespace fim

using namespace fim;

extern "C" {

// act: 0 ReLU, 1 GELU. out_mode: 0 MXFP8 dynamic (e4m3 out + exponents / swizzled scales), 1 INT8 (scale),
// 2 BF16, 3 MXFP8 static (exponent [C/32]).
int fim_depthwise5x5(const uint16_t* x, int64_t B, int64_t H, int64_t W, int64_t C, const uint16_t* weight,
                     const float* bias, int act, int out_mode, const float* scale, const int8_t* exponent, void* out,
                     int8_t* exponent_out, uint8_t* swizzled, hipStream_t stream) {
  if (x == nullptr || weight == nullptr || bias == nullptr || out == nullptr) return FIM_ERR_INVALID;
  if (B < 0 || H < 0 || W < 0 || C <= 0) return FIM_ERR_INVALID;
  if (out_mode < 0 || out_mode > 3 || act < 0 || act > 1) return FIM_ERR_INVALID;
  if (out_mode == DW_INT8 && scale == nullptr) return FIM_ERR_INVALID;
  if (out_mode == DW_MX_STATIC && exponent == nullptr) return FIM_ERR_INVALID;
  if (C % 32 != 0) return FIM_ERR_UNSUPPORTED;
  if (((uintptr_t)x % 8) != 0 || ((uintptr_t)weight % 8) != 0 || ((uintptr_t)out % 8) != 0) return FIM_ERR_UNSUPPORTED;
  if (B * H * W == 0) return FIM_OK;
  if (H > 2147483647LL || W > 2147483647LL) return FIM_ERR_UNSUPPORTED;
  // 32-bit channel and weight indices ((ky * 5 + kx) * C + c) and 40-bit element offsets
  if (C > 2147483647LL / 25 || B * H * W > (1LL << 40) / C) return FIM_ERR_UNSUPPORTED;
  if (((uintptr_t)x % 16) != 0) return FIM_ERR_UNSUPPORTED;
  const int64_t tx = cdiv(W, DW_TW), ty = cdiv(H, DW_TH);
  const int64_t ntiles = tx * ty * B * (C / DW_CS);
  if (ntiles > (1LL << 31) - 8) return FIM_ERR_UNSUPPORTED;
  DwArgs a{x, weight, bias, scale, exponent, out, swizzled, exponent_out, (int)B, (int)H, (int)W, (int)C,
           (int)tx, (int)ty, ntiles};
  dim3 grid((unsigned)(cdiv(ntiles, 8) * 8));  // a multiple of the 8 XCDs: the kernel maps pids to tiles per XCD
  if (act == ACT_RELU)
    dw_launch_out<ACT_RELU>(a, out_mode, grid, stream);
  else
    dw_launch_out<ACT_GELU>(a, out_mode, grid, stream);
  return launch_status();
}

}  // extern "C"
