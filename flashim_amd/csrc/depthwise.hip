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
// flashim/quant/passes/separable_conv_block.py:52-55); bias FP32 or BF16 [C]. Output row = pixel (b, y, x), C channels.
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
  const void* bias;        // FP32 or BF16 [C]
  int bias_bf16;
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
// Output columns, output rows, channels per workgroup. 16 columns (a 25.3 KB LDS tile, 74-80 VGPRs: six workgroups per
// CU) measured faster than 24 (four per CU), 32 (three) and 8 (eight, with 1.5x the halo): config 4 22.9 / 24.8 / 26.8 /
// 25.0 us, the depthwise-pointwise composites 3-7% faster than at 32.
constexpr int DW_TW = 16, DW_TH = 16, DW_CS = 32;
constexpr int DW_CQ = DW_TW / 4;    // 4-column output quads per tile row
constexpr int DW_SEGS = DW_CQ + 1;  // 4-column staged segments per row (the 2-column halos on both sides)

// ---- The taps on the matrix unit ----------------------------------------------------------------------------
// v_mfma_f32_4x4x4_16b_bf16 runs 16 independent 4x4x4 products per instruction; each is one channel: D[i][j] (output
// columns 4 cq + i, output row 4 rq + j) += A[i][k] B[k][j] with A the Toeplitz matrix of one weight row, A[i][k] =
// w[ky][4 s + k - i] (zero outside 0..4), and B[k][j] = input (row 4 rq + j + ky, column 4 cq + 4 s + k) of the staged
// tile (origin y0 - 2, x0 - 2): 5 weight rows x 2 column segments s = 10 MFMAs per 16 channels x 4 x 4 outputs; the
// first MFMA of each output block takes the bias as its accumulator input.
// Operand layout (measured): lane l = 4 b + r supplies A_b[r][0..3] and B_b[0..3][r] and gets D_b[0..3][r].
// The tile is staged channel-planar ([channel][row][column] BF16, 20 columns per row, planes 200 dwords apart plus 16
// dwords per channel octet) so each B operand is one 8-byte LDS read. With 64 four-byte banks and a 64-bit access
// served 32 lanes at a time, the B reads of 8 channels x 4 rows (plane steps of 8 banks, row steps of 10: the 4 rows
// in distinct residues mod 8, the 8 channels apart within each) and the staging writes (4 octets apart by the octet
// padding, consecutive 4-column groups of a row 2 banks apart) are conflict-free.
// After the taps each lane activates and quantizes its 32 values in registers (one channel, 4 columns x 4 column
// quads x 2 rows);
// static outputs (INT8, static MXFP8, BF16) then go through LDS as finished codes in [row][column][channel] order
// (byte or 16-bit writes with immediate offsets) and leave as 16-byte stores of 16 (8) channels of one pixel. Dynamic
// MXFP8 needs the per-(pixel, 32-channel) amax first, so its FP32 values go through LDS in two 8-row halves and a
// per-pixel pass (8 channels per lane, exponents from 4-lane amax shuffles) quantizes and stores.
constexpr int DWM_ROWSTR = 2 * DW_SEGS;              // dwords per staged row (DW_TW + 4 columns)
constexpr int DWM_PLANE = 20 * DWM_ROWSTR;          // dwords per channel plane
constexpr int DWM_OCTPAD = 16;                      // extra dwords per channel octet
constexpr int DWM_LDS = DW_CS * DWM_PLANE + 4 * DWM_OCTPAD;  // 11584 dwords
__device__ __forceinline__ constexpr int dw_plane(int c) { return c * DWM_PLANE + (c >> 3) * DWM_OCTPAD; }
constexpr int DWM_UNITS = 20 * DW_SEGS * 4;         // staging units: 20 rows x column quads x 4 channel octets
constexpr int DWM_OROW = DW_TW * DW_CS + 16;        // dwords per staged FP32 output row (dynamic MXFP8, padded)
constexpr int DWO_ROW8 = DW_TW * DW_CS + 16;        // bytes per staged 8-bit output row (padded: rows 4 banks apart)
constexpr int DWO_ROW16 = DW_TW * DW_CS * 2 + 16;   // bytes per staged BF16 output row
static_assert(8 * DWM_OROW <= DWM_LDS, "an 8-row FP32 output half fits in the input tile's space");
static_assert(DW_TH * DWO_ROW16 <= 4 * DWM_LDS, "the staged BF16 output tile fits in the input tile's space");

typedef __bf16 v4bf16 __attribute__((ext_vector_type(4)));

// One staging unit: 4 pixels (columns 4 q .. 4 q + 3 of staged row r) x 8 channels (octet o), transposed (v_perm) into
// 8 channel rows of 4 BF16, one 8-byte LDS write each.
__device__ __forceinline__ void dw_stage_unit(uint32_t* sm, int o, int r, int q, const uint4 (&v)[4]) {
  const uint32_t P[4][4] = {{v[0].x, v[0].y, v[0].z, v[0].w}, {v[1].x, v[1].y, v[1].z, v[1].w},
                            {v[2].x, v[2].y, v[2].z, v[2].w}, {v[3].x, v[3].y, v[3].z, v[3].w}};
  uint32_t* base = &sm[dw_plane(8 * o) + r * DWM_ROWSTR + 2 * q];
#pragma unroll
  for (int m = 0; m < 4; ++m) {  // dword m of a pixel = channels 8 o + 2 m (low half), + 1 (high half)
    const uint32_t lo01 = __builtin_amdgcn_perm(P[1][m], P[0][m], 0x05040100u);
    const uint32_t lo23 = __builtin_amdgcn_perm(P[3][m], P[2][m], 0x05040100u);
    const uint32_t hi01 = __builtin_amdgcn_perm(P[1][m], P[0][m], 0x07060302u);
    const uint32_t hi23 = __builtin_amdgcn_perm(P[3][m], P[2][m], 0x07060302u);
    *reinterpret_cast<uint2*>(base + 2 * m * DWM_PLANE) = make_uint2(lo01, lo23);
    *reinterpret_cast<uint2*>(base + (2 * m + 1) * DWM_PLANE) = make_uint2(hi01, hi23);
  }
}

template <int ACT, int OUT>
__global__ __launch_bounds__(256, 6) void dw5x5_mfma_kernel(const DwArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t sm[DWM_LDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware tile order: workgroup p runs on XCD p % 8, so each XCD takes a contiguous run of tiles in (channel slice,
  // column tile, row tile, image) order, slice fastest: the slices of a pixel (which share its 128-byte input lines)
  // and neighbouring column tiles (which share halo columns) read through the same L2 at about the same time.
  const int cslices = a.C / DW_CS;
  const int64_t L = (int64_t)(blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  if (L >= a.ntiles) return;
  const int cbase = (int)(L % cslices) * DW_CS;
  int64_t rest = L / cslices;
  const int x0 = (int)(rest % a.tiles_x) * DW_TW;
  rest /= a.tiles_x;
  const int y0 = (int)(rest % a.tiles_y) * DW_TH;
  const int b = (int)(rest / a.tiles_y);
  // interior tile: the whole halo is inside the image (no masking, no partial rows or columns)
  const bool interior = y0 >= 2 && y0 + DW_TH + 2 <= a.H && x0 >= 2 && x0 + DW_TW + 2 <= a.W;

  // (weights first: their loads are in flight with the tile's)
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
  const float bias = a.bias_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(a.bias)[ch])
                                 : static_cast<const float*>(a.bias)[ch];
  const v4f biasv = {bias, bias, bias, bias};

  // stage the (DW_TH + 4) x (DW_TW + 4) x 32 halo tile: every load of the thread's units is issued before the first
  // LDS write, so the HBM latency is paid once per tile, not once per unit. Buffer loads from the first in-image halo
  // row; a pixel outside the image gets an offset past the buffer's range, which the hardware returns as zeros.
  constexpr int NU = (DWM_UNITS + 255) / 256;
  uint4 v[NU][4];
  {
    const int ybase = max(y0 - 2, 0);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.x + ((int64_t)b * a.H + ybase) * a.W * a.C + cbase), (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      const int u = min(tid + 256 * j, DWM_UNITS - 1);  // a repeated unit past the end is loaded, not written
      const int o = u & 3, rq = u >> 2;
      const int r = rq / DW_SEGS, q = rq - r * DW_SEGS;
      const int iy = y0 - 2 + r;
      const bool row_ok = iy >= 0 && iy < a.H;
      // byte offsets below 2^31 (the host bounds 40 W C)
      const uint32_t row_off = (uint32_t)(((iy - ybase) * a.W + x0 - 2 + 4 * q) * a.C + 8 * o) * 2u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int ix = x0 - 2 + 4 * q + k;
        const bool ok = interior || (row_ok && ix >= 0 && ix < a.W);
        const uint32_t off = ok ? row_off + (uint32_t)(k * a.C * 2) : 0x80000000u;
        v[j][k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NU; ++j) {
    const int u = tid + 256 * j;
    if (j < NU - 1 || u < DWM_UNITS) {
      const int o = u & 3, rq = u >> 2;
      const int r = rq / DW_SEGS, q = rq - r * DW_SEGS;
      dw_stage_unit(sm, o, r, q, v[j]);
    }
  }

  __syncthreads();

  // The taps row by row: staged row 8 rh + r4 + rr (rr = 4 t + ky) feeds weight row ky of row quad t; its DW_SEGS column
  // segments (4 columns each) are read once and reused by the DW_CQ column quads x 2 segments, and the next row's
  // segments are read while this row's MFMAs run.
  v4f acc[2][DW_CQ];  // [row quad 2 rh + t][column quad cq]: D[i = 0..3][j = r4]
  const uint32_t* plane = &sm[dw_plane(16 * cg + bch) + (8 * rh + r4) * DWM_ROWSTR];
  uint2 seg[2][DW_SEGS];
#pragma unroll
  for (int g = 0; g < DW_SEGS; ++g) seg[0][g] = *reinterpret_cast<const uint2*>(plane + 2 * g);
#pragma unroll
  for (int rr = 0; rr < 9; ++rr) {
    if (rr < 8) {
#pragma unroll
      for (int g = 0; g < DW_SEGS; ++g)
        seg[(rr + 1) & 1][g] = *reinterpret_cast<const uint2*>(plane + (rr + 1) * DWM_ROWSTR + 2 * g);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int ky = rr - 4 * t;
      if (ky < 0 || ky > 4) continue;
#pragma unroll
      for (int sg = 0; sg < 2; ++sg)
#pragma unroll
        for (int cq = 0; cq < DW_CQ; ++cq)
          acc[t][cq] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(wa[ky][sg], __builtin_bit_cast(v4bf16, seg[rr & 1][cq + sg]),
                                                              (ky == 0 && sg == 0) ? biasv : acc[t][cq], 0, 0, 0);
    }
  }

  const int rows = min(DW_TH, a.H - y0), cols = min(DW_TW, a.W - x0);
  uint8_t* sm8 = reinterpret_cast<uint8_t*>(sm);

  if (OUT == DW_MX_DYNAMIC) {
    // ReLU in registers, FP32 values through LDS in two 8-row halves, per-pixel dynamic quantize
    float y[2][DW_CQ][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int cq = 0; cq < DW_CQ; ++cq)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[t][cq][i] = fmaxf(acc[t][cq][i], 0.f);
    const int64_t groups = a.C >> 5;
    const int64_t tiles_k = (groups + 3) >> 2;
    const int64_t gi = cbase >> 5;
    float* st = reinterpret_cast<float*>(sm);
    // output pass lanes: 4 consecutive lanes share a pixel (part = 8-channel quarter of the slice); unit tid + 256 it
    // is pixel (tid >> 2) + 64 it of the half (row-major over DW_TW columns); addresses from the tile's first pixel
    const int part = tid & 3;
    const int64_t rowt = ((int64_t)b * a.H + y0) * a.W + x0;  // the tile's first output pixel
    uint8_t* const out0 = static_cast<uint8_t*>(a.out) + rowt * a.C + cbase + 8 * part;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      __syncthreads();  // half 0: the taps are done with the input tile; half 1: the previous output pass is done
      if (rh == half) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int cq = 0; cq < DW_CQ; ++cq)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              st[(4 * t + r4) * DWM_OROW + (4 * cq + i) * DW_CS + 16 * cg + bch] = y[t][cq][i];
      }
      __syncthreads();
      // output pass: 8 rows x DW_TW columns x 4 parts of 8 channels
#pragma unroll
      for (int it = 0; it < 8 * DW_TW * 4 / 256; ++it) {
        const int pxh = (tid >> 2) + 64 * it;
        const int rl = pxh / DW_TW, col = pxh - rl * DW_TW;
        const int oy = 8 * half + rl;
        const float4 va = *reinterpret_cast<const float4*>(&st[rl * DWM_OROW + col * DW_CS + 8 * part]);
        const float4 vb = *reinterpret_cast<const float4*>(&st[rl * DWM_OROW + col * DW_CS + 8 * part + 4]);
        const float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
        // the values are >= 0 (ReLU): the amax is a plain max and the clamp is one-sided
        float amax = fmaxf(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])), fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
        amax = fmaxf(amax, __shfl_xor(amax, 1));
        amax = fmaxf(amax, __shfl_xor(amax, 2));
        const int ex = mx_exponent_wave(amax);
        const float inv = exp2_int(-ex);
        float q[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = __builtin_elementwise_minimum(v[e] * inv, 448.0f);
        const bool ok = interior || (oy < rows && col < cols);
        if (ok) {
          const int64_t step = (int64_t)oy * a.W + col;  // pixels from the tile's first
          *reinterpret_cast<uint2*>(out0 + step * a.C) =
              make_uint2(pack_e4m3x4(q[0], q[1], q[2], q[3]), pack_e4m3x4(q[4], q[5], q[6], q[7]));
          if (part == 0) {
            const int64_t row = rowt + step;
            if (a.expo_out != nullptr) a.expo_out[row * groups + gi] = (int8_t)ex;
            if (a.swizzled != nullptr) {
              const int64_t rt = row & 127;
              a.swizzled[(((row >> 7) * tiles_k + (gi >> 2)) << 9) + (rt & 31) * 16 + (rt >> 5) * 4 + (gi & 3)] =
                  (uint8_t)(ex + 127);
            }
          }
        }
      }
    }
    return;
  }

  // static outputs: activate and quantize in registers, then the finished codes go through LDS
  // (lane's LDS byte offset of its channel at tile row 8 rh + r4, column 0)
  const int ob8 = (8 * rh + r4) * DWO_ROW8 + 16 * cg + bch;
  const int ob16 = (8 * rh + r4) * DWO_ROW16 + 2 * (16 * cg + bch);
  uint32_t code[2][DW_CQ][2];  // 8-bit: [t][cq][0] = 4 codes (columns 4 cq + i); BF16: two packed pairs
  float oscale = 0.f, oinv8 = 1.f, osc = 1.f, obound = 448.f;
  bool low_clamp = false;
  if (OUT == DW_INT8) {
    oscale = *a.scale;
    oinv8 = __fdiv_rn(1.0f, oscale);
  }
  if (OUT == DW_MX_STATIC) {
    const int e = (int)a.expo[cbase >> 5];
    osc = exp2_int(e);
    obound = 448.0f * osc;
    low_clamp = e < -11;  // GELU >= -0.17 > -bound unless the bound is below 0.17
  }
  // (the lower clamp as a wave-uniform choice of loop, not a per-value select)
  auto activate_quantize = [&](auto lowc) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int cq = 0; cq < DW_CQ; ++cq) {
        float v[4] = {acc[t][cq][0], acc[t][cq][1], acc[t][cq][2], acc[t][cq][3]};
        if (ACT == ACT_RELU) {
          if (OUT != DW_INT8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
          }
        } else {
          round_bf16x2(v[0], v[1]);
          round_bf16x2(v[2], v[3]);
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = gelu_erf(v[i]);
        }
        if (OUT == DW_INT8) {
          round_bf16x2(v[0], v[1]);
          round_bf16x2(v[2], v[3]);
          int qi[4];
          if (ACT == ACT_RELU)
            quantize_int8_fast_n<4, 0>(v, oscale, oinv8, qi);  // the ReLU folded into the saturation
          else
            quantize_int8_fast_n<4>(v, oscale, oinv8, qi);
          code[t][cq][0] = (uint32_t)(qi[0] & 0xff) | ((uint32_t)(qi[1] & 0xff) << 8) | ((uint32_t)(qi[2] & 0xff) << 16) |
                           ((uint32_t)qi[3] << 24);
        } else if (OUT == DW_MX_STATIC) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[i] = __builtin_elementwise_minimum(v[i], obound);
            if (decltype(lowc)::value) v[i] = __builtin_elementwise_maximum(v[i], -obound);
          }
          code[t][cq][0] = e4m3x4_of_bf16_inrange(v[0], v[1], v[2], v[3], osc);
        } else {
          code[t][cq][0] = pack_bf16x2(v[0], v[1]);
          code[t][cq][1] = pack_bf16x2(v[2], v[3]);
        }
      }
  };
  if (OUT == DW_MX_STATIC && low_clamp)
    activate_quantize(std::true_type{});
  else
    activate_quantize(std::false_type{});
  __syncthreads();  // every wave is done with the input tile
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int cq = 0; cq < DW_CQ; ++cq) {
      if (OUT == DW_BF16) {
        uint8_t* p = sm8 + ob16 + 4 * t * DWO_ROW16 + 4 * cq * (2 * DW_CS);
        *reinterpret_cast<uint16_t*>(p) = (uint16_t)code[t][cq][0];
        *reinterpret_cast<uint16_t*>(p + 2 * DW_CS) = (uint16_t)(code[t][cq][0] >> 16);
        *reinterpret_cast<uint16_t*>(p + 4 * DW_CS) = (uint16_t)code[t][cq][1];
        *reinterpret_cast<uint16_t*>(p + 6 * DW_CS) = (uint16_t)(code[t][cq][1] >> 16);
      } else {
        uint8_t* p = sm8 + ob8 + 4 * t * DWO_ROW8 + 4 * cq * DW_CS;
        const uint32_t c4 = code[t][cq][0];
        p[0] = (uint8_t)c4;
        p[DW_CS] = (uint8_t)(c4 >> 8);
        p[2 * DW_CS] = (uint8_t)(c4 >> 16);
        p[3 * DW_CS] = (uint8_t)(c4 >> 24);
      }
    }
  __syncthreads();
  // 16-byte chunks: 8-bit, 2 per pixel (16 channels each); BF16, 4 per pixel (8 channels each)
  constexpr int CPP = OUT == DW_BF16 ? 4 : 2;
  constexpr int ROWB = OUT == DW_BF16 ? DWO_ROW16 : DWO_ROW8;
  constexpr int ESZ = OUT == DW_BF16 ? 2 : 1;
#pragma unroll
  for (int it = 0; it < DW_TH * DW_TW * CPP / 256; ++it) {
    const int k = tid + 256 * it;
    const int part = k % CPP, px = k / CPP;
    const int R = px / DW_TW, X = px - R * DW_TW;
    const uint4 val = *reinterpret_cast<const uint4*>(sm8 + R * ROWB + X * (DW_CS * ESZ) + 16 * part);
    if (interior || (R < rows && X < cols)) {
      const int64_t row = ((int64_t)b * a.H + y0 + R) * a.W + x0 + X;
      *reinterpret_cast<uint4*>(static_cast<uint8_t*>(a.out) + (row * a.C + cbase) * ESZ + 16 * part) = val;
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
                     const void* bias, int bias_dtype, int act, int out_mode, const float* scale,
                     const int8_t* exponent, void* out, int8_t* exponent_out, uint8_t* swizzled, hipStream_t stream) {
  if (x == nullptr || weight == nullptr || bias == nullptr || out == nullptr) return FIM_ERR_INVALID;
  if (bias_dtype != FIM_F32 && bias_dtype != FIM_BF16) return FIM_ERR_INVALID;
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
  if (out_mode != DW_MX_DYNAMIC && ((uintptr_t)out % 16) != 0) return FIM_ERR_UNSUPPORTED;  // 16-byte code stores
  if (40 * W * C > 2147483647LL) return FIM_ERR_UNSUPPORTED;  // 31-bit byte offsets within a staged tile
  const int64_t tx = cdiv(W, DW_TW), ty = cdiv(H, DW_TH);
  const int64_t ntiles = tx * ty * B * (C / DW_CS);
  if (ntiles > (1LL << 31) - 8) return FIM_ERR_UNSUPPORTED;
  DwArgs a{x, weight, bias, bias_dtype == FIM_BF16, scale, exponent, out, swizzled, exponent_out, (int)B, (int)H, (int)W, (int)C,
           (int)tx, (int)ty, ntiles};
  dim3 grid((unsigned)(cdiv(ntiles, 8) * 8));  // a multiple of the 8 XCDs: the kernel maps pids to tiles per XCD
  if (act == ACT_RELU)
    dw_launch_out<ACT_RELU>(a, out_mode, grid, stream);
  else
    dw_launch_out<ACT_GELU>(a, out_mode, grid, stream);
  return launch_status();
}

}  // extern "C"
