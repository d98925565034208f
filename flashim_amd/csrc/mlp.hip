// Fused refiner MLP on one CU: expand C -> H, GELU, static quantize, contract H -> C (+ bias, + residual), with the
// quantized hidden layer kept in LDS. Two epilogue semantics:
//   MLP_BLOCK      the conv-refiner block's pointwise pair, exactly the two conv launches it replaces:
//                  int8_conv2d / mxfp8_conv2d 1x1 (bias, GELU, quantized output) then 1x1 (bias, + residual)
//                  (flashim/ops/conv.py:174-206, 309-342; chained quantized output quant/methods/conv2d.py:102-125;
//                  residual epilogue ops/conv.py:198-203);
//   MLP_REFERENCE  ops.mxfp8_gelu_mlp (flashim/ops/gemm.py:146-157): hidden = bf16(x W1^T); gelu(hidden + b1) in
//                  FP32 -> BF16; static MXFP8 quantize; out = bf16(q W2^T) (no second bias, no residual).
// Shape: C = 64 channels, H = 256 hidden (the fine-scale refiner width). Both weight matrices (32 KB), their
// exponents / scales and the biases are loaded into LDS once per workgroup; the workgroup then walks 64-pixel tiles
// (grid-stride), prefetching the next tile's activations into registers while it computes the current one.
//
// MFMA operands: A = weight rows, B = pixel rows, so each lane ends with 4 consecutive output channels of one pixel.
// The expand epilogue packs the 4 quantized hidden codes of a lane into one 32-bit LDS store at the place the contract
// reads them from: hidden row px holds 256 bytes in 16 slots of 16 B, slot s stored at s ^ (px & 15), so both the
// 4-byte writes and the 16-byte fragment reads of 16 consecutive rows are conflict-free. Rows of 64 bytes (input
// tile, W1) swizzle their 4 slots with (row >> 2) & 3.
#include "common.h"

namespace fim {

enum { MLP_INT8 = 0, MLP_MX = 1 };
enum { MLP_BLOCK = 0, MLP_REFERENCE = 1 };

constexpr int MLP_C = 64, MLP_H = 256, MLP_BM = 64;


struct MlpArgs {
  const uint8_t* x;        // [P, C] int8 / E4M3
  const uint8_t* w1;       // [H, C]
  const uint8_t* w2;       // [C, H]
  const void* x_scale;     // MX: int8 [C / 32]; INT8: FP32 scalar
  const void* w1_scale;    // MX: int8 [H, C / 32]; INT8: FP32 [H]
  const void* h_scale;     // MX: int8 [H / 32]; INT8: FP32 scalar (the hidden layer's static scale)
  const void* w2_scale;    // MX: int8 [C, H / 32]; INT8: FP32 [C]
  const void* b1;          // [H] or null
  int b1_dtype;
  const void* b2;          // [C] or null
  int b2_dtype;
  const uint16_t* residual;  // [P, C] BF16 or null
  uint16_t* out;           // [P, C] BF16
  int P;
  int ntiles;
};

__device__ __forceinline__ float load_bias(const void* b, int dtype, int i) {
  if (b == nullptr) return 0.0f;
  return dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(b)[i]) : static_cast<const float*>(b)[i];
}

// Workgroups per CU: three (51.5 KB of LDS each, the input tile sharing the hidden tile's space) when the kernel fits
// 168 VGPRs, else two.
template <int KIND, int SEM>
constexpr int mlp_wgs_per_cu() { return KIND == MLP_MX && SEM == MLP_REFERENCE ? 2 : 3; }  // (the latter spills at 3)
// MXFP8 (182 VGPRs with all four accumulator blocks live) computes and drains one hidden block at a time
template <int KIND>
constexpr bool mlp_split_expand() { return KIND == MLP_MX; }

template <int KIND, int SEM>
__global__ __launch_bounds__(256, (mlp_wgs_per_cu<KIND, SEM>())) void refiner_mlp_kernel(const MlpArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t w1s[MLP_H * MLP_C];  // [h][64 B]
  __shared__ __attribute__((aligned(16))) uint8_t w2s[MLP_C * MLP_H];  // [c][256 B]
  __shared__ __attribute__((aligned(16))) uint8_t hs[MLP_BM * MLP_H];  // [px][256 B]
  // the input tile [px][64 B] lives in the hidden tile's first 4 KB: read into registers at the start of the expand,
  // before any hidden value is written (a barrier between), and written again after the contract's reads (a barrier
  // before)
  uint8_t* const xs = hs;
  __shared__ float b1s[MLP_H], b2s[MLP_C], s1[MLP_H], s2[MLP_C];
  __shared__ int8_t e1s[MLP_H * (MLP_C / 32)], e2s[MLP_C * (MLP_H / 32)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int r16 = lane & 15;

  // ---- once per workgroup: weights, exponents / scales, biases -------------------------------------------------
  for (int idx = tid; idx < MLP_H * MLP_C / 16; idx += 256) {  // W1: 1024 segments of 16 B
    const int row = idx >> 2, seg = idx & 3;
    *reinterpret_cast<uint4*>(&w1s[row * MLP_C + ((seg ^ ((row >> 2) & 3)) << 4)]) =
        *reinterpret_cast<const uint4*>(a.w1 + row * MLP_C + seg * 16);
  }
  for (int idx = tid; idx < MLP_C * MLP_H / 16; idx += 256) {  // W2: 1024 segments of 16 B
    const int row = idx >> 4, seg = idx & 15;
    *reinterpret_cast<uint4*>(&w2s[row * MLP_H + ((seg ^ (row & 15)) << 4)]) =
        *reinterpret_cast<const uint4*>(a.w2 + row * MLP_H + seg * 16);
  }
  {
    const int h = tid;  // 256 threads = H
    b1s[h] = load_bias(a.b1, a.b1_dtype, h);
    if (KIND == MLP_INT8) {
      s1[h] = *static_cast<const float*>(a.x_scale) * static_cast<const float*>(a.w1_scale)[h];
    } else {
      e1s[2 * h] = static_cast<const int8_t*>(a.w1_scale)[2 * h];
      e1s[2 * h + 1] = static_cast<const int8_t*>(a.w1_scale)[2 * h + 1];
    }
    if (h < MLP_C) {
      b2s[h] = load_bias(a.b2, a.b2_dtype, h);
      if (KIND == MLP_INT8) {
        s2[h] = *static_cast<const float*>(a.h_scale) * static_cast<const float*>(a.w2_scale)[h];
      } else {
#pragma unroll
        for (int b = 0; b < MLP_H / 32; ++b) e2s[h * (MLP_H / 32) + b] = static_cast<const int8_t*>(a.w2_scale)[h * (MLP_H / 32) + b];
      }
    }
  }
  // activation exponents of the expand input (2 blocks of 32 channels) and of the hidden layer (8 blocks)
  int xe[2] = {0, 0};
  float hq_scale = 1.0f, hq_inv = 1.0f;
  if (KIND == MLP_MX) {
    xe[0] = static_cast<const int8_t*>(a.x_scale)[0];
    xe[1] = static_cast<const int8_t*>(a.x_scale)[1];
  } else {
    hq_scale = *static_cast<const float*>(a.h_scale);
    hq_inv = __fdiv_rn(1.0f, hq_scale);
  }
  const int8_t* hexp = static_cast<const int8_t*>(a.h_scale);
  // MX: the scales 2^e of this wave's two 32-channel hidden blocks (2 wave, 2 wave + 1)
  float hsc_w[2] = {1.0f, 1.0f};
  // MX: the contract's activation scales (E8M0) of the lane's K blocks 4 s + g, read once here: read in the tile loop
  // (the output stores may alias them, so the compiler reloads them per tile), their wait also drained the next tile's
  // prefetch
  int hsx[MLP_H / 128];
#pragma unroll
  for (int s = 0; s < MLP_H / 128; ++s) hsx[s] = 127;
  if (KIND == MLP_MX) {
    hsc_w[0] = exp2_int((int)hexp[2 * __builtin_amdgcn_readfirstlane(wave)]);
    hsc_w[1] = exp2_int((int)hexp[2 * __builtin_amdgcn_readfirstlane(wave) + 1]);
#pragma unroll
    for (int s = 0; s < MLP_H / 128; ++s) hsx[s] = (int)hexp[4 * s + g] + 127;
  }

  // per-lane pieces of the tile loop
  const int ld_px = tid >> 2, ld_seg = tid & 3;  // the input segment this lane stages
  const int ld_dst = ld_px * MLP_C + ((ld_seg ^ ((ld_px >> 2) & 3)) << 4);
  auto load_tile = [&](int t) -> uint4 {
    const int px = t * MLP_BM + ld_px;
    if (t < a.ntiles && px < a.P) return *reinterpret_cast<const uint4*>(a.x + (int64_t)px * MLP_C + ld_seg * 16);
    return make_uint4(0, 0, 0, 0);
  };
  // the residual of a tile, prefetched with its input: lane (wave, r16, g) adds pixel 16 wave + r16, channels
  // 16 i + 4 g .. + 3
  auto load_res = [&](int t, uint2 (&r)[4]) {
    const int px = t * MLP_BM + 16 * wave + r16;
    const bool ok = a.residual != nullptr && t < a.ntiles && px < a.P;
    const uint16_t* src = a.residual + (int64_t)(ok ? px : 0) * MLP_C + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint2 v = ok ? *reinterpret_cast<const uint2*>(src + 16 * i) : make_uint2(0, 0);
      r[i] = v;
    }
  };
  // the output as a buffer (P x C BF16 < 2 GiB: checked by the host), its descriptor from uniform operands
  const uint64_t out_addr = (uint64_t)a.out;
  const uint64_t out_u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(out_addr >> 32)) << 32) |
                         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)out_addr);
  const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(out_u), (short)0, __builtin_amdgcn_readfirstlane((int)((uint32_t)a.P * MLP_C * 2u)),
      0x00020000);
  uint4 cur = load_tile(blockIdx.x);
  uint2 res_cur[4], res_nxt[4];
  load_res(blockIdx.x, res_cur);
  __syncthreads();  // weights and tables staged

  for (int t = blockIdx.x; t < a.ntiles; t += gridDim.x) {
    const int px0 = t * MLP_BM;
    __syncthreads();  // the previous tile's contract is done reading the hidden tile (the input tile's space)
    *reinterpret_cast<uint4*>(&xs[ld_dst]) = cur;
    __syncthreads();  // input tile staged
    cur = load_tile(t + gridDim.x);  // prefetch the next tile's input and residual
    load_res(t + gridDim.x, res_nxt);

    // ---- expand: wave w computes hidden channels [64 w, 64 w + 64) x all 64 pixels ----------------------------
    // 32 x 32 MFMA blocks (2 hidden x 2 pixel blocks per wave): MXFP8 v_mfma_scale_f32_32x32x64_f8f6f4 takes the
    // whole K = 64 in one instruction (no zero-padded K half), INT8 two v_mfma_i32_32x32x32_i8. Operand layout
    // (measured on gfx950): lane l supplies row l % 32; for the scaled MFMA, bytes 0-15 are K [16 h, 16 h + 16) and
    // bytes 16-31 are K [32 + 16 h, +16) with h = l / 32, and the scale of lane i + 32 kb covers K block kb of row i;
    // the INT8 products are exact, so any K order shared by both operands gives the same int32 sums. Output: register r
    // of lane l is row 8 (r / 4) + 4 h + r % 4, column l % 32: a lane holds 4 groups of 4 consecutive hidden channels
    // of one pixel, all in one 32-channel scale block. All MFMAs first (their latency hides behind each other), the
    // VALU-heavy epilogues after.
    {
      const int l32 = lane & 31, h2 = lane >> 5;
      v4i xlo[2], xhi[2];  // pixel rows 32 jb + l32: 16-byte slots h2 and 2 + h2
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const int row = 32 * jb + l32;
        xlo[jb] = *reinterpret_cast<const v4i*>(&xs[row * MLP_C + ((h2 ^ ((row >> 2) & 3)) << 4)]);
        xhi[jb] = *reinterpret_cast<const v4i*>(&xs[row * MLP_C + (((2 + h2) ^ ((row >> 2) & 3)) << 4)]);
      }
      if constexpr (mlp_split_expand<KIND>()) {
        // one hidden block's MFMAs, then its epilogue: half the accumulators are live at a time, which fits the
        // registers of three workgroups per CU (the other workgroups' waves cover the MFMA latency)
        v16i acc_i[2][2];
        v16f acc_f[2][2];
        __syncthreads();  // every wave holds its input fragments: the hidden tile may be written over the input tile
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
          const int h = 64 * wave + 32 * ib + l32;
          const v4i wlo = *reinterpret_cast<const v4i*>(&w1s[h * MLP_C + ((h2 ^ ((h >> 2) & 3)) << 4)]);
          const v4i whi = *reinterpret_cast<const v4i*>(&w1s[h * MLP_C + (((2 + h2) ^ ((h >> 2) & 3)) << 4)]);
          const int sw = (int)e1s[2 * h + h2] + 127;
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            if (KIND == MLP_INT8) {
              v16i c = {};
              c = __builtin_amdgcn_mfma_i32_32x32x32_i8(wlo, xlo[jb], c, 0, 0, 0);
              acc_i[ib][jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(whi, xhi[jb], c, 0, 0, 0);
            } else {
              const v8i wa = __builtin_shufflevector(wlo, whi, 0, 1, 2, 3, 4, 5, 6, 7);
              const v8i xb = __builtin_shufflevector(xlo[jb], xhi[jb], 0, 1, 2, 3, 4, 5, 6, 7);
              acc_f[ib][jb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wa, xb, v16f{}, 0, 0, 0, sw, 0,
                                                                              xe[h2] + 127);
            }
          }

          const int hb = 64 * wave + 32 * ib + 4 * h2;  // hidden channel of register 0; register r adds 8 (r / 4) + r % 4
          // MXFP8: the block's scale; GELU outputs are >= -0.1700 (BF16), so the lower clamp at -448 * 2^e is a no-op
          // for every scale >= 2^-11 (wave-uniform: the wave's 32 channels share one scale block)
          const float sc = hsc_w[ib], bound = 448.0f * sc;
          const bool two_sided = __builtin_amdgcn_readfirstlane((int)(sc < 0x1p-11f)) != 0;
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            float yb[16];  // the block's 16 values, all computed before any is quantized (one INT8 tie test)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int hh = hb + 8 * (r >> 2) + (r & 3);
              float y;
              if (KIND == MLP_INT8) {
                y = __fadd_rn(__fmul_rn((float)acc_i[ib][jb][r], s1[hh]), b1s[hh]);
              } else if (SEM == MLP_REFERENCE) {  // bf16(x W1^T), + b1 in FP32, GELU of the FP32 sum
                y = __fadd_rn(round_bf16_hw(acc_f[ib][jb][r]), b1s[hh]);
              } else {
                y = __fadd_rn(acc_f[ib][jb][r], b1s[hh]);
              }
              yb[r] = SEM == MLP_BLOCK ? round_bf16_hw(y) : y;  // the conv epilogue: BF16 rounding before the GELU
            }
            gelu_erf_n<16>(yb);  // the block's 16 GELU chains interleaved
            uint32_t qw[4];
            if (KIND == MLP_MX) {  // BF16 rounding and static E4M3 in one step
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                float q[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) q[v] = __builtin_elementwise_minimum(yb[4 * k + v], bound);
                if (two_sided) {
#pragma unroll
                  for (int v = 0; v < 4; ++v) q[v] = __builtin_elementwise_maximum(q[v], -bound);
                }
                qw[k] = e4m3x4_of_bf16_inrange(q[0], q[1], q[2], q[3], sc);
              }
            } else {
#pragma unroll
              for (int r = 0; r < 16; ++r) yb[r] = round_bf16_hw(yb[r]);
              int qi[16];
              quantize_int8_fast_n<16>(yb, hq_scale, hq_inv, qi);
#pragma unroll
              for (int k = 0; k < 4; ++k)
                qw[k] = (uint32_t)(uint8_t)qi[4 * k] | ((uint32_t)(uint8_t)qi[4 * k + 1] << 8) |
                        ((uint32_t)(uint8_t)qi[4 * k + 2] << 16) | ((uint32_t)(uint8_t)qi[4 * k + 3] << 24);
            }
            const int px = 32 * jb + l32;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const int h0 = hb + 8 * k;
              *reinterpret_cast<uint32_t*>(&hs[px * MLP_H + ((((h0 >> 4)) ^ (px & 15)) << 4) + (h0 & 15)]) = qw[k];
            }
          }

        }
      } else {
        v16i acc_i[2][2];
        v16f acc_f[2][2];
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
          const int h = 64 * wave + 32 * ib + l32;
          const v4i wlo = *reinterpret_cast<const v4i*>(&w1s[h * MLP_C + ((h2 ^ ((h >> 2) & 3)) << 4)]);
          const v4i whi = *reinterpret_cast<const v4i*>(&w1s[h * MLP_C + (((2 + h2) ^ ((h >> 2) & 3)) << 4)]);
          const int sw = (int)e1s[2 * h + h2] + 127;
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            if (KIND == MLP_INT8) {
              v16i c = {};
              c = __builtin_amdgcn_mfma_i32_32x32x32_i8(wlo, xlo[jb], c, 0, 0, 0);
              acc_i[ib][jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(whi, xhi[jb], c, 0, 0, 0);
            } else {
              const v8i wa = __builtin_shufflevector(wlo, whi, 0, 1, 2, 3, 4, 5, 6, 7);
              const v8i xb = __builtin_shufflevector(xlo[jb], xhi[jb], 0, 1, 2, 3, 4, 5, 6, 7);
              acc_f[ib][jb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wa, xb, v16f{}, 0, 0, 0, sw, 0,
                                                                              xe[h2] + 127);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // every wave holds its input fragments: the hidden tile may be written over the input tile
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
          const int hb = 64 * wave + 32 * ib + 4 * h2;  // hidden channel of register 0; register r adds 8 (r / 4) + r % 4
          // MXFP8: the block's scale; GELU outputs are >= -0.1700 (BF16), so the lower clamp at -448 * 2^e is a no-op
          // for every scale >= 2^-11 (wave-uniform: the wave's 32 channels share one scale block)
          const float sc = hsc_w[ib], bound = 448.0f * sc;
          const bool two_sided = __builtin_amdgcn_readfirstlane((int)(sc < 0x1p-11f)) != 0;
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            float yb[16];  // the block's 16 values, all computed before any is quantized (one INT8 tie test)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int hh = hb + 8 * (r >> 2) + (r & 3);
              float y;
              if (KIND == MLP_INT8) {
                y = __fadd_rn(__fmul_rn((float)acc_i[ib][jb][r], s1[hh]), b1s[hh]);
              } else if (SEM == MLP_REFERENCE) {  // bf16(x W1^T), + b1 in FP32, GELU of the FP32 sum
                y = __fadd_rn(round_bf16_hw(acc_f[ib][jb][r]), b1s[hh]);
              } else {
                y = __fadd_rn(acc_f[ib][jb][r], b1s[hh]);
              }
              yb[r] = SEM == MLP_BLOCK ? round_bf16_hw(y) : y;  // the conv epilogue: BF16 rounding before the GELU
            }
            gelu_erf_n<16>(yb);  // the block's 16 GELU chains interleaved
            uint32_t qw[4];
            if (KIND == MLP_MX) {  // BF16 rounding and static E4M3 in one step
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                float q[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) q[v] = __builtin_elementwise_minimum(yb[4 * k + v], bound);
                if (two_sided) {
#pragma unroll
                  for (int v = 0; v < 4; ++v) q[v] = __builtin_elementwise_maximum(q[v], -bound);
                }
                qw[k] = e4m3x4_of_bf16_inrange(q[0], q[1], q[2], q[3], sc);
              }
            } else {
#pragma unroll
              for (int r = 0; r < 16; ++r) yb[r] = round_bf16_hw(yb[r]);
              int qi[16];
              quantize_int8_fast_n<16>(yb, hq_scale, hq_inv, qi);
#pragma unroll
              for (int k = 0; k < 4; ++k)
                qw[k] = (uint32_t)(uint8_t)qi[4 * k] | ((uint32_t)(uint8_t)qi[4 * k + 1] << 8) |
                        ((uint32_t)(uint8_t)qi[4 * k + 2] << 16) | ((uint32_t)(uint8_t)qi[4 * k + 3] << 24);
            }
            const int px = 32 * jb + l32;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const int h0 = hb + 8 * k;
              *reinterpret_cast<uint32_t*>(&hs[px * MLP_H + ((((h0 >> 4)) ^ (px & 15)) << 4) + (h0 & 15)]) = qw[k];
            }
          }
        }
      }
    }
    __syncthreads();  // hidden tile complete

    // ---- contract: wave w computes pixels [16 w, 16 w + 16) x all 64 channels ---------------------------------
    {
      const int prow = 16 * wave + r16;  // the hidden row this lane's B fragments come from
      const int px = px0 + prow;         // and the output pixel of this lane's results
      const bool pok = px < a.P;
      const uint2 (&res)[4] = res_cur;
      v4i acc_i[4] = {};
      v4f acc_f[4] = {};
      if (KIND == MLP_INT8) {
#pragma unroll
        for (int q = 0; q < MLP_H / 64; ++q) {  // K chunks of 64 bytes: lane reads slot 4 q + g
          const int slot = 4 * q + g;
          const v4i hf = *reinterpret_cast<const v4i*>(&hs[prow * MLP_H + ((slot ^ (prow & 15)) << 4)]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int c = 16 * i + r16;
            const v4i wf = *reinterpret_cast<const v4i*>(&w2s[c * MLP_H + ((slot ^ (c & 15)) << 4)]);
            acc_i[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, hf, acc_i[i], 0, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int s = 0; s < MLP_H / 128; ++s) {  // K steps of 128 bytes: lo slot 8 s + g, hi slot 8 s + 4 + g
          const int sl = 8 * s + g, sh = 8 * s + 4 + g;
          const v4i hl = *reinterpret_cast<const v4i*>(&hs[prow * MLP_H + ((sl ^ (prow & 15)) << 4)]);
          const v4i hh = *reinterpret_cast<const v4i*>(&hs[prow * MLP_H + ((sh ^ (prow & 15)) << 4)]);
          const v8i hf = v8i{hl[0], hl[1], hl[2], hl[3], hh[0], hh[1], hh[2], hh[3]};
          const int sx = hsx[s];  // lane group g scales K block 4 s + g
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int c = 16 * i + r16;
            const v4i wl = *reinterpret_cast<const v4i*>(&w2s[c * MLP_H + ((sl ^ (c & 15)) << 4)]);
            const v4i wh = *reinterpret_cast<const v4i*>(&w2s[c * MLP_H + ((sh ^ (c & 15)) << 4)]);
            const v8i wf = v8i{wl[0], wl[1], wl[2], wl[3], wh[0], wh[1], wh[2], wh[3]};
            const int sw = (int)e2s[c * (MLP_H / 32) + 4 * s + g] + 127;
            acc_f[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf, hf, acc_f[i], 0, 0, 0, sw, 0, sx);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c0 = 16 * i + 4 * g;
        float y[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          y[v] = KIND == MLP_INT8 ? __fmul_rn((float)acc_i[i][v], s2[c0 + v]) : acc_f[i][v];
          if (a.b2 != nullptr) y[v] = __fadd_rn(y[v], b2s[c0 + v]);
        }
        round_bf16x2(y[0], y[1]);
        round_bf16x2(y[2], y[3]);
        if (a.residual != nullptr) {
          y[0] = __fadd_rn(y[0], u2f(res[i].x << 16));
          y[1] = __fadd_rn(y[1], u2f(res[i].x & 0xffff0000u));
          y[2] = __fadd_rn(y[2], u2f(res[i].y << 16));
          y[3] = __fadd_rn(y[3], u2f(res[i].y & 0xffff0000u));
        }
        // an unconditional buffer store (pixels past P at an offset past the buffer's end): the compiler then counts
        // the stores exactly, and the next tile's wait for its prefetched input does not wait for them
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const uint32_t off = pok ? (uint32_t)(px * MLP_C + c0) * 2u : 0x80000000u;
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])}, orsrc, (int)off, 0,
                                              0);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) res_cur[i] = res_nxt[i];
  }
}

}  // namespace fim

using namespace fim;

// kind 0: INT8 (scales FP32), 1: MXFP8 (exponents int8). semantics 0: the refiner block's pointwise pair,
// 1: ops.mxfp8_gelu_mlp (MXFP8 only; b2 and residual must be null).
extern "C" int fim_refiner_mlp(int kind, int semantics, const uint8_t* x, int64_t P, int64_t C, int64_t H,
                               const void* x_scale, const uint8_t* w1, const void* w1_scale, const void* b1,
                               int b1_dtype, const void* h_scale, const uint8_t* w2, const void* w2_scale,
                               const void* b2, int b2_dtype, const uint16_t* residual, uint16_t* out,
                               hipStream_t stream) {
  if (x == nullptr || x_scale == nullptr || w1 == nullptr || w1_scale == nullptr || h_scale == nullptr ||
      w2 == nullptr || w2_scale == nullptr || out == nullptr || P < 0 || (kind != MLP_INT8 && kind != MLP_MX) ||
      (semantics != MLP_BLOCK && semantics != MLP_REFERENCE))
    return FIM_ERR_INVALID;
  if (semantics == MLP_REFERENCE && (kind != MLP_MX || b2 != nullptr || residual != nullptr)) return FIM_ERR_INVALID;
  if (C != MLP_C || H != MLP_H) return FIM_ERR_UNSUPPORTED;
  if (P * MLP_H >= (1LL << 31)) return FIM_ERR_UNSUPPORTED;
  if (((uintptr_t)x | (uintptr_t)w1 | (uintptr_t)w2) % 16 != 0 || ((uintptr_t)out | (uintptr_t)residual) % 8 != 0)
    return FIM_ERR_UNSUPPORTED;
  if (P == 0) return FIM_OK;
  MlpArgs a{x, w1, w2, x_scale, w1_scale, h_scale, w2_scale, b1, b1_dtype, b2, b2_dtype, residual, out, (int)P, 0};
  a.ntiles = (int)cdiv(P, MLP_BM);
  // grid-stride over the tiles with as many workgroups as fit on the GPU at once
  const int slots = device_cus() * (kind == MLP_INT8         ? mlp_wgs_per_cu<MLP_INT8, MLP_BLOCK>()
                                    : semantics == MLP_BLOCK ? mlp_wgs_per_cu<MLP_MX, MLP_BLOCK>()
                                                             : mlp_wgs_per_cu<MLP_MX, MLP_REFERENCE>());
  const int grid = a.ntiles < slots ? a.ntiles : slots;
  if (kind == MLP_INT8)
    refiner_mlp_kernel<MLP_INT8, MLP_BLOCK><<<dim3(grid), dim3(256), 0, stream>>>(a);
  else if (semantics == MLP_BLOCK)
    refiner_mlp_kernel<MLP_MX, MLP_BLOCK><<<dim3(grid), dim3(256), 0, stream>>>(a);
  else
    refiner_mlp_kernel<MLP_MX, MLP_REFERENCE><<<dim3(grid), dim3(256), 0, stream>>>(a);
  return launch_status();
}
