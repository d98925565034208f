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
// Work split: see the tile comment at dw5x5_kernel. The 25 x 4 weights of a lane's channels live in VGPRs.
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
// 32-channel slice (64 B each) are staged in LDS once; a lane then owns 4 channels of one column and walks the 20 input
// rows with row rolling: each row's 5 horizontal taps are read from LDS once and accumulated into the 5 output rows
// that use them, FP32 FMA in ky-major, kx-minor order (the order of a direct 25-tap loop). Lane l of a wavefront reads
// channel quad l % 8 of column l / 8, so a tap read is 64 lanes x 8 contiguous bytes: no LDS bank conflicts.
constexpr int DW_TW = 32, DW_TH = 16, DW_CS = 32;  // output columns, output rows, channels per workgroup
constexpr int DW_IW = DW_TW + 4, DW_IH = DW_TH + 4;

template <int ACT, int OUT>
__global__ __launch_bounds__(256) void dw5x5_kernel(const DwArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[DW_IH * DW_IW * DW_CS];  // [row][col][32 ch] BF16, 46 KB
  const int tid = threadIdx.x;
  const int x0 = blockIdx.x * DW_TW;
  const int y0 = blockIdx.y * DW_TH;
  const int cslices = a.C / DW_CS;
  const int b = blockIdx.z / cslices;
  const int cbase = (blockIdx.z % cslices) * DW_CS;

  // stage the input tile: 20 x 36 pixels x 4 segments of 16 B (8 channels), zero outside the image
  for (int i = tid; i < DW_IH * DW_IW * 4; i += 256) {
    const int segi = i & 3, pix = i >> 2;
    const int r = pix / DW_IW, cidx = pix - r * DW_IW;
    const int iy = y0 - 2 + r, ix = x0 - 2 + cidx;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (iy >= 0 && iy < a.H && ix >= 0 && ix < a.W)
      v = *reinterpret_cast<const uint4*>(a.x + (((int64_t)b * a.H + iy) * a.W + ix) * a.C + cbase + segi * 8);
    *reinterpret_cast<uint4*>(&tile[pix * DW_CS + segi * 8]) = v;
  }

  const int lane = tid & 63, wave = tid >> 6;
  const int cq = lane & 7;                   // channel quad within the 32-channel slice
  const int xl = wave * 8 + (lane >> 3);     // output column within the tile
  const int x = x0 + xl;
  const int c = cbase + cq * 4;
  const bool x_ok = x < a.W;

  float wt[25][4];
#pragma unroll
  for (int t = 0; t < 25; ++t) load4_bf16(a.w + t * a.C + c, wt[t]);
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

  float acc[5][4];
#pragma unroll
  for (int k = 0; k < 5; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[k][i] = 0.f;

  const int rows = min(DW_TH, a.H - y0);  // output rows of this tile
#pragma unroll 2
  for (int s = 0; s < rows + 4; ++s) {
    const uint16_t* rp = &tile[(s * DW_IW + xl) * DW_CS + cq * 4];
    float v[5][4];
#pragma unroll
    for (int kx = 0; kx < 5; ++kx) load4_bf16(rp + kx * DW_CS, v[kx]);
    // output row (s - 2) + 2 - ky of the tile receives tap row ky: acc[4 - ky]
#pragma unroll
    for (int ky = 0; ky < 5; ++ky)
#pragma unroll
      for (int kx = 0; kx < 5; ++kx)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[4 - ky][i] = fmaf(v[kx][i], wt[ky * 5 + kx][i], acc[4 - ky][i]);

    if (s >= 4) {  // acc[0] holds all 25 taps of tile row s - 4
      const int oy = y0 + s - 4;
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = acc[0][i] + bias[i];
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
          uint32_t q = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) q |= (uint32_t)(uint8_t)quantize_int8_fast(y[i], oscale, oinv8) << (8 * i);
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
    }
    // roll
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[k][i] = acc[k + 1][i];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[4][i] = 0.f;
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
