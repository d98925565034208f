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
// Work split: see the tile comment at dw5x5_kernel. The weights of a lane's 4 channels live in VGPRs as 60 BF16 pairs.
#include <type_traits>

#include "common.h"

namespace fim {

enum { ACT_RELU = 0, ACT_GELU = 1 };
enum { DW_MX_DYNAMIC = 0, DW_INT8 = 1, DW_BF16 = 2, DW_MX_STATIC = 3 };

__device__ __forceinline__ void load4_bf16(const uint16_t* p, float* v) {
  uint2 q = *reinterpret_cast<const uint2*>(p);
  v[0] = u2f(q.x << 16);
  v[1] = u2f(q.x & 0xffff0000u);
  v[2] = u2f(q.y << 16);
  v[3] = u2f(q.y & 0xffff0000u);
}

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
};

// Tile: 32 output columns x 16 output rows x 32 channels per workgroup. The (16 + 4) x (32 + 4) input pixels of the
// 32-channel slice are staged in LDS once, with adjacent columns interleaved per channel: dword (row, column pair p,
// channel c) holds the BF16 values of columns 2p and 2p + 1, so two horizontal taps of one channel are one
// v_dot2_f32_bf16 operand (two products, FP32 accumulate). A lane owns 4 channels of one output column x and covers its
// 5 taps of a row with 3 dot2 steps: columns (x, x+1), (x+2, x+3), (x+4, x+5) with weight pairs (w0, w1), (w2, w3),
// (w4, 0) when x is even; (x-1, x), (x+1, x+2), (x+3, x+4) with (0, w0), (w1, w2), (w3, w4) when x is odd. The lane
// walks the 20 input rows; row s feeds output rows s - ky for the 5 ky, held in a ring of 5 accumulators indexed at
// compile time (the row loop is unrolled by 5), and output row s - 4 is complete after row s. The FP32 sums are those
// of a direct 25-tap loop in another order (per ky: the dot2 pairs, then the rows).
constexpr int DW_TW = 32, DW_TH = 16, DW_CS = 32;  // output columns, output rows, channels per workgroup
constexpr int DW_IW = DW_TW + 4, DW_IH = DW_TH + 4;
constexpr int DW_PAIRS = DW_IW / 2;                // 18 column pairs per staged row

typedef __bf16 v2bf16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v2bf16 as_bf2(uint32_t u) { return __builtin_bit_cast(v2bf16, u); }

template <int ACT, int OUT>
__global__ __launch_bounds__(256) void dw5x5_kernel(const DwArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t tile[DW_IH * DW_PAIRS * DW_CS];  // [row][pair][32 ch], 46 KB
  const int tid = threadIdx.x;
  const int x0 = blockIdx.x * DW_TW;
  const int y0 = blockIdx.y * DW_TH;
  const int cslices = a.C / DW_CS;
  const int b = blockIdx.z / cslices;
  const int cbase = (blockIdx.z % cslices) * DW_CS;

  // stage: 20 rows x 18 column pairs x 4 segments of 8 channels; each item loads the 8 channels of both columns
  // (zero outside the image) and interleaves them (v_perm) into 8 dwords
  for (int i = tid; i < DW_IH * DW_PAIRS * 4; i += 256) {
    const int segi = i & 3, rp = i >> 2;
    const int r = rp / DW_PAIRS, p = rp - r * DW_PAIRS;
    const int iy = y0 - 2 + r, ix = x0 - 2 + 2 * p;
    uint4 va = make_uint4(0, 0, 0, 0), vb = make_uint4(0, 0, 0, 0);
    const bool row_ok = iy >= 0 && iy < a.H;
    const uint16_t* src = a.x + (((int64_t)b * a.H + (row_ok ? iy : 0)) * a.W) * a.C + cbase + segi * 8;
    if (row_ok && ix >= 0 && ix < a.W) va = *reinterpret_cast<const uint4*>(src + (int64_t)ix * a.C);
    if (row_ok && ix + 1 >= 0 && ix + 1 < a.W) vb = *reinterpret_cast<const uint4*>(src + (int64_t)(ix + 1) * a.C);
    const uint32_t A[4] = {va.x, va.y, va.z, va.w}, B[4] = {vb.x, vb.y, vb.z, vb.w};
    uint32_t o[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = __builtin_amdgcn_perm(B[k], A[k], 0x05040100u);      // channel 2k: (col 2p, col 2p + 1)
      o[2 * k + 1] = __builtin_amdgcn_perm(B[k], A[k], 0x07060302u);  // channel 2k + 1
    }
    uint32_t* dst = &tile[(r * DW_PAIRS + p) * DW_CS + segi * 8];
    *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4*>(dst + 4) = make_uint4(o[4], o[5], o[6], o[7]);
  }

  const int lane = tid & 63, wave = tid >> 6;
  const int cq = lane & 7;                   // channel quad within the 32-channel slice
  const int xl = wave * 8 + (lane >> 3);     // output column within the tile
  const int x = x0 + xl;
  const int c = cbase + cq * 4;
  const bool x_ok = x < a.W;
  const bool odd = (xl & 1) != 0;
  const int pb = xl >> 1;                    // first column pair of this lane's taps

  // weight pairs per (ky, dot2 step k, channel): (w[ky][2k], w[ky][2k+1]) for even columns, shifted by one for odd
  uint32_t wp[5][3][4];
#pragma unroll
  for (int ky = 0; ky < 5; ++ky) {
    uint32_t w5[5][4];  // BF16 bits of w[ky][kx] for the lane's 4 channels
#pragma unroll
    for (int kx = 0; kx < 5; ++kx) {
      const uint2 q = *reinterpret_cast<const uint2*>(a.w + (ky * 5 + kx) * a.C + c);
      w5[kx][0] = q.x & 0xffffu; w5[kx][1] = q.x >> 16; w5[kx][2] = q.y & 0xffffu; w5[kx][3] = q.y >> 16;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t e0 = w5[0][i] | (w5[1][i] << 16), e1 = w5[2][i] | (w5[3][i] << 16), e2 = w5[4][i];
      const uint32_t o0 = w5[0][i] << 16, o1 = w5[1][i] | (w5[2][i] << 16), o2 = w5[3][i] | (w5[4][i] << 16);
      wp[ky][0][i] = odd ? o0 : e0;
      wp[ky][1][i] = odd ? o1 : e1;
      wp[ky][2][i] = odd ? o2 : e2;
    }
  }
  float bias[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bias[i] = a.bias[c + i];
  float oscale = 0.f, oinv = 1.f;
  float oinv8 = 1.f;
  if (OUT == DW_INT8) {
    oscale = *a.scale;
    oinv8 = __fdiv_rn(1.0f, oscale);
  }
  if (OUT == DW_MX_STATIC) oinv = exp2_int(-(int)a.expo[c >> 5]);
  const int64_t groups = a.C >> 5;
  const int64_t tiles_k = (groups + 3) >> 2;

  __syncthreads();

  float acc[5][4];  // ring: output row o accumulates in acc[o % 5]
#pragma unroll
  for (int k = 0; k < 5; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[k][i] = 0.f;

  auto finish = [&](int oy, float (&sum)[4]) {
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = sum[i] + bias[i];
    if (ACT == ACT_RELU) {
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = fmaxf(y[i], 0.f);
    } else {
      round_bf16x2(y[0], y[1]);
      round_bf16x2(y[2], y[3]);
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = gelu_erf(y[i]);
      round_bf16x2(y[0], y[1]);
      round_bf16x2(y[2], y[3]);
    }
    const int64_t row = ((int64_t)b * a.H + oy) * a.W + x;
    if (OUT == DW_MX_DYNAMIC) {
      float amax = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      amax = fmaxf(amax, __shfl_xor(amax, 4));
      const int e = mx_exponent_from_amax(amax);
      const float inv = exp2_int(-e);
      if (x_ok) {
        const uint32_t q = pack_e4m3x4(mx_scale_clamp(y[0], inv), mx_scale_clamp(y[1], inv),
                                       mx_scale_clamp(y[2], inv), mx_scale_clamp(y[3], inv));
        *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.out) + row * a.C + c) = q;
        if (cq == 0) {
          const int64_t gi = c >> 5;
          if (a.expo_out != nullptr) a.expo_out[row * groups + gi] = (int8_t)e;
          if (a.swizzled != nullptr) {
            const int64_t rt = row & 127;
            a.swizzled[(((row >> 7) * tiles_k + (gi >> 2)) << 9) + (rt & 31) * 16 + (rt >> 5) * 4 + (gi & 3)] =
                (uint8_t)(e + 127);
          }
        }
      }
    } else if (x_ok) {
      if (OUT == DW_INT8) {
        if (ACT == ACT_RELU) {
          round_bf16x2(y[0], y[1]);
          round_bf16x2(y[2], y[3]);
        }
        int qi[4];
        quantize_int8_fast_n<4>(y, oscale, oinv8, qi);
        uint32_t q = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) q |= (uint32_t)(uint8_t)qi[i] << (8 * i);
        *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.out) + row * a.C + c) = q;
      } else if (OUT == DW_MX_STATIC) {
        const uint32_t q = pack_e4m3x4(mx_scale_clamp(y[0], oinv), mx_scale_clamp(y[1], oinv),
                                       mx_scale_clamp(y[2], oinv), mx_scale_clamp(y[3], oinv));
        *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.out) + row * a.C + c) = q;
      } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + row * a.C + c) =
            make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
      }
    }
  };

  // one input row s (u = s mod 5, compile time): 3 pair reads, 60 dot2 into the ring, then output row s - 4
  const int rows = min(DW_TH, a.H - y0);  // output rows of this tile
  auto row_step = [&](int s, auto uc) {
    constexpr int U = decltype(uc)::value;
    const uint32_t* rp = &tile[(s * DW_PAIRS + pb) * DW_CS + cq * 4];
    uint4 v[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = *reinterpret_cast<const uint4*>(rp + k * DW_CS);
#pragma unroll
    for (int ky = 0; ky < 5; ++ky) {
      float* r = acc[(U - ky + 5) % 5];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const uint32_t xv[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(xv[i]), as_bf2(wp[ky][k][i]), r[i], false);
      }
    }
    // row s - 4 (ring slot (U + 1) % 5) has all its taps: emit it (rows above the tile, s < 4, only collected the
    // taps of the zero padding), then clear the slot for row s + 1
    float* o = acc[(U + 1) % 5];
    if (s >= 4) {
      float sum[4] = {o[0], o[1], o[2], o[3]};
      finish(y0 + s - 4, sum);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = 0.f;
  };
  for (int s = 0; s < rows + 4; s += 5) {
    row_step(s, std::integral_constant<int, 0>{});
    if (s + 1 < rows + 4) row_step(s + 1, std::integral_constant<int, 1>{});
    if (s + 2 < rows + 4) row_step(s + 2, std::integral_constant<int, 2>{});
    if (s + 3 < rows + 4) row_step(s + 3, std::integral_constant<int, 3>{});
    if (s + 4 < rows + 4) row_step(s + 4, std::integral_constant<int, 4>{});
  }
}

template <int ACT>
static void dw_launch_out(const DwArgs& a, int out_mode, dim3 grid, hipStream_t s) {
  switch (out_mode) {
    case DW_MX_DYNAMIC: dw5x5_kernel<ACT, DW_MX_DYNAMIC><<<grid, dim3(256), 0, s>>>(a); break;
    case DW_INT8: dw5x5_kernel<ACT, DW_INT8><<<grid, dim3(256), 0, s>>>(a); break;
    case DW_BF16: dw5x5_kernel<ACT, DW_BF16><<<grid, dim3(256), 0, s>>>(a); break;
    default: dw5x5_kernel<ACT, DW_MX_STATIC><<<grid, dim3(256), 0, s>>>(a); break;
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
  if (((uintptr_t)x % 16) != 0) return FIM_ERR_UNSUPPORTED;
  DwArgs a{x, weight, bias, scale, exponent, out, swizzled, exponent_out, (int)B, (int)H, (int)W, (int)C};
  const int64_t gz = B * (C / DW_CS);
  const int64_t gy = cdiv(H, DW_TH);
  if (gz > 65535 || gy > 65535) return FIM_ERR_UNSUPPORTED;
  dim3 grid((unsigned)cdiv(W, DW_TW), (unsigned)gy, (unsigned)gz);
  if (act == ACT_RELU)
    dw_launch_out<ACT_RELU>(a, out_mode, grid, stream);
  else
    dw_launch_out<ACT_GELU>(a, out_mode, grid, stream);
  return launch_status();
}

}  // extern "C"
