// Implicit-GEMM NHWC convolution on CDNA4 MFMA, for the two quantized conv ops:
//   fim_int8_conv2d   flashim/ops/conv.py:174-206 (reference: im2col_gather -> int8_linear, flashim/ops/gemm.py:78-101)
//   fim_mxfp8_conv2d  flashim/ops/conv.py:309-342 (reference: im2col_gather -> mxfp8_linear, flashim/ops/gemm.py:58-72)
//
// GEMM view: M = B*Ho*Wo output pixels, N = Cout, K = taps * Cin in (ky, kx, c) order. Both operands are K-contiguous
// (NHWC activations, [Cout, taps*Cin] weights), so each lane of an MFMA reads 32 consecutive bytes of one row.
// The K loop walks (tap, 128-channel chunk) steps; each step gathers a BM x 128-byte activation tile straight from x
// (the tap's spatial offset folded into the address, padding and channel tails zero-filled) and a BN x 128-byte weight
// tile, both staged through LDS with double buffering (one barrier per step, the next step's global loads in flight
// during the current step's MFMAs).
//
// MFMA per 16x16 output block and 128-byte K step:
//   INT8  : two v_mfma_i32_16x16x64_i8 (a lane's 32 bytes split in two halves, the same split on both operands,
//           so the int32 dot product is exact and independent of the hardware's K order);
//   MXFP8 : one v_mfma_scale_f32_16x16x128_f8f6f4 with E8M0 scales. Operand layout (measured on gfx950): lane l,
//           g = l / 16, supplies row l % 16 with K bytes [16g, 16g + 16) in VGPRs 0-3 and [64 + 16g, 64 + 16g + 16)
//           in VGPRs 4-7; the scale operand of lane i + 16 kb is the E8M0 of row i's K block kb ([32 kb, 32 kb + 32)).
//           So a lane reads two 16-byte pieces of its row from LDS and passes the scale of block g:
//           channel_exponent[block] + 127 (activations) or weight_exponent[n, block] + 127 (weights).
// The workgroup is 4 wavefronts (2 x 2) over a 128 x BN tile; each wavefront owns 64 x BN/2 of it.
//
// Epilogue (per element, in the reference's rounding order):
//   INT8 : y = float(acc) * (a_scale * w_scale[n]); y = y + bias[n]  (two roundings, no FMA: ops/gemm.py:88-90)
//   MXFP8: y = acc + bias[n]
//   ReLU (before the BF16 rounding when there is no residual), BF16 rounding, optional GELU (erf form, rounded to BF16:
//   ops/gemm.py:94-95), optional residual relu(y + r) in FP32 then BF16 (ops/conv.py:198-203), then the store as
//   BF16, or quantized for the next layer: INT8 with out_scale (quant/tensor.py:148-151) or E4M3 with out_exponent
//   (quant/tensor.py:97-121).
#include <type_traits>

#include "common.h"

namespace fim {

enum { KIND_INT8 = 0, KIND_MX = 1 };
enum { OUT_BF16 = 0, OUT_INT8 = 1, OUT_E4M3 = 2 };

struct ConvArgs {
  const uint8_t* x;        // [B, H, W, Cin] int8 / e4m3
  const uint8_t* w;        // [Cout, T*Cin]
  const int8_t* x_expo;    // MX: [Cin / 32]
  const int8_t* w_expo;    // MX: [Cout, T*Cin / 32]
  int w_expo_e8m0;         // MX: w_expo holds E8M0 bytes (exponent + 127) instead of signed exponents
  const uint8_t* x_swz;    // MX, per-row scales (XS = 1): E8M0 bytes of x in the 128x4 swizzled layout
  int x_swz_tiles_k;       //   ceil((Cin / 32) / 4)
  const float* a_scale_rows;  // INT8: per-row activation scales [M] (null: the per-tensor a_scale)
  const float* a_scale;    // INT8: scalar
  const float* w_scale;    // INT8: [Cout]
  const void* bias;        // [Cout] or null
  int bias_dtype;          // FIM_F32 / FIM_BF16
  const void* residual;    // [B, Ho, Wo, res_channels] with strides, or null
  int res_dtype;
  int64_t res_channels, rs_b, rs_h, rs_w, rs_c;
  const float* out_scale;  // OUT_INT8
  const int8_t* out_expo;  // OUT_E4M3: [Cout / 32]
  void* out;               // [B, Ho, Wo, Cout]: pixel rows out_ld elements apart (out_ld >= Cout)
  int64_t out_ld;
  int8_t* pool_out;        // POOL: [B, Ho/2, Wo/2, Cout] int8, the 2x2 max pool of out quantized with out_scale
  int out_mode, relu_pre, relu_post, gelu;  // ReLU before the BF16 rounding / after the residual add
  int B, H, W, Cin, Ho, Wo, Cout;
  int kh, kw, sh, sw, ph, pw, dh, dw;
  int M;                   // output pixels (< 2^31)
  int kchunks;             // ceil(Cin / 128)
  int tps;                 // taps per 128-byte K step of the packed-tap kernels (PACK): 128 / Cin for Cin 16, 32, 64
  int n_tiles, m_tiles;
  int m_base;              // first GEMM row of this launch (a split launch runs its last rows as a second launch)
};

// The MFMA scale byte (E8M0: exponent + 127) of a weight exponent entry read as int8: signed exponents get + 127,
// E8M0 bytes pass through; (v + add) & 0xff covers both (an E8M0 byte above 127 reads as v - 256).
__device__ __forceinline__ int w_scale_byte(const ConvArgs& a, int v) { return (v + (a.w_expo_e8m0 ? 0 : 127)) & 0xff; }


constexpr int BM_MAIN = 128;  // pixel rows per tile (the tail of a launch may use 64-row tiles)
constexpr int KC = 128;          // bytes of K per step


// 16 bytes of one row segment, channel-masked. LW = widest load the layout allows (16: Cin % 16 == 0; else 1).
// 16 zero bytes in device memory: masked lanes (padding pixels, channel tails, rows past the tile) load from here, so
// every 16-byte segment load is unconditional and branch-free.
__device__ __attribute__((aligned(16))) uint4 fim_zero_segment[1];

template <int LW>
__device__ __forceinline__ uint4 load_seg(const uint8_t* p, bool row_ok, int cvalid) {
  if (LW == 16) {
    const uint8_t* src = (row_ok && cvalid > 0) ? p : reinterpret_cast<const uint8_t*>(fim_zero_segment);
    return *reinterpret_cast<const uint4*>(src);
  }
  uint4 v = make_uint4(0, 0, 0, 0);
  if (!row_ok || cvalid <= 0) return v;
  if (LW == 4) {
    uint32_t t[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * i < cvalid) t[i] = reinterpret_cast<const uint32_t*>(p)[i];
    v = make_uint4(t[0], t[1], t[2], t[3]);
  } else {
    uint32_t t[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i < cvalid) t[i >> 2] |= (uint32_t)p[i] << (8 * (i & 3));
    v = make_uint4(t[0], t[1], t[2], t[3]);
  }
  return v;
}

// GEMM row m -> output pixel index (img * Ho + oh) * Wo + ow. Plain order is the identity; the pool order (POOL, Ho and
// Wo even) puts the 4 pixels of each 2x2 pool window on 4 consecutive rows, windows in (img, oh / 2, ow / 2) order:
// m = 4 * window + 2 * dy + dx.
template <int POOL>
__device__ __forceinline__ int pixel_of_row(const ConvArgs& a, int m, int& img, int& oh, int& ow) {
  if (POOL) {
    const int wo2 = a.Wo >> 1, ho2 = a.Ho >> 1;
    const int win = m >> 2;
    const int q = win / wo2;
    ow = 2 * (win - q * wo2) + (m & 1);
    img = q / ho2;
    oh = 2 * (q - img * ho2) + ((m >> 1) & 1);
    return (img * a.Ho + oh) * a.Wo + ow;
  }
  ow = m % a.Wo;
  const int q = m / a.Wo;
  img = q / a.Ho;
  oh = q - img * a.Ho;
  return m;
}

// Epilogue of one wavefront's MB x NB blocks of 16 x 16 outputs, straight from the accumulators: D[n][m] with
// lane = pixel (lane & 15) of a 16-pixel block and 4 consecutive channels 4 (lane >> 4) + v of a 16-channel block, so
// each store writes 4 channels of one pixel. mrow[j]: this lane's GEMM row in block j (M or more: no output);
// n_tile0: the tile's first channel; nl0:
// the wave's first channel within the tile (index into the per-channel operands ep_* staged in LDS).
// Branch-free epilogue for the common case (no residual, no pooling, Cout % 16 == 0, output below 2 GiB): per
// 16-pixel row block, all NB x 4 values of the lane are computed (their chains, GELU's above all, interleave) and then
// stored, so the stores stream out while the next block is computed, each burst covering whole lines; outputs past M
// or Cout are dropped by the buffer store's range check instead of per-lane branches. Same arithmetic, in the same
// order per value, as the general epilogue below.
// RES: a BF16 residual laid out as the output ([M, Cout] dense, so its element offset is the output's), added after
// the activation with the conv semantics relu(y + r) (ops/conv.py:198-203): loaded per row block with the same
// out-of-range handling as the stores.
// The lane's per-channel epilogue operands: for each of its NB channel blocks, the scale and bias of its 4 channels
// and their output scale (the lane's 4 channels, aligned by 4, share one 32-channel scale block).
template <int NB>
struct EpiChannels {
  float cs[NB][4], cb[NB][4], osc[NB];
};

template <int NB>
__device__ __forceinline__ EpiChannels<NB> epi_channels(int nl0, const float* ep_scale, const float* ep_bias,
                                                        const float* ep_osc) {
  const int g = (threadIdx.x & 63) >> 4;
  EpiChannels<NB> ch;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int nl = nl0 + i * 16 + 4 * g;
    const float4 cs4 = *reinterpret_cast<const float4*>(&ep_scale[nl]);
    const float4 cb4 = *reinterpret_cast<const float4*>(&ep_bias[nl]);
    ch.cs[i][0] = cs4.x; ch.cs[i][1] = cs4.y; ch.cs[i][2] = cs4.z; ch.cs[i][3] = cs4.w;
    ch.cb[i][0] = cb4.x; ch.cb[i][1] = cb4.y; ch.cb[i][2] = cb4.z; ch.cb[i][3] = cb4.w;
    ch.osc[i] = ep_osc[nl];
  }
  return ch;
}

// Staged output: the values go to an LDS tile instead of global memory, row (tile pixel) spix[j] of STAGE_RB bytes per
// pixel, 16-byte slot s of row p at slot s ^ stage_swz(p) (the caller writes the tile out in whole lines).
__device__ __forceinline__ int stage_swz(int p) { return (p >> 1) & 7; }

// GELU: 0 none (ReLU or the identity as one IEEE maximum), 1 GELU without ReLU (no maximum), 2 ReLU then GELU.
template <int KIND, int OUT, int MB, int NB, int GELU, bool RES = false, int STAGE_RB = 0>
__device__ __forceinline__ void conv_epilogue_fast(const ConvArgs& a, const v4i (&acc_i)[NB][MB],
                                                   const v4f (&acc_f)[NB][MB], const int (&mrow)[MB], int n_tile0,
                                                   int nl0, const EpiChannels<NB>& ch, uint8_t* stage = nullptr,
                                                   const int* spix = nullptr) {
  constexpr int ESZ = OUT == OUT_BF16 ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const float out_scale = OUT == OUT_INT8 ? *a.out_scale : 1.0f;
  const float out_inv = OUT == OUT_INT8 ? __fdiv_rn(1.0f, out_scale) : 1.0f;
  // ReLU as IEEE maximum against 0 (on) or -inf (off: the identity, NaN kept): one operation, no select
  float relu_lo = a.relu_pre != 0 ? 0.0f : -__builtin_inff();
  asm("" : "+v"(relu_lo));  // opaque: otherwise the compiler folds the bound back into a per-value select
  const bool row_scales = KIND == KIND_INT8 && a.a_scale_rows != nullptr;
  // descriptor operands through readfirstlane: provably uniform, so the descriptor stays in SGPRs (a descriptor the
  // compiler cannot prove uniform turns every store into a readfirstlane loop)
  const int nbytes = __builtin_amdgcn_readfirstlane((int)((uint32_t)a.M * (uint32_t)a.out_ld * ESZ));
  const uint64_t out_addr = (uint64_t)a.out;
  const uint64_t out_u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(out_addr >> 32)) << 32) |
                         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)out_addr);
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(out_u), (short)0, nbytes, 0x00020000);
  __amdgpu_buffer_rsrc_t res_rsrc = rsrc;
  float relu_post_lo = -__builtin_inff();
  if constexpr (RES) {
    const uint64_t res_addr = (uint64_t)a.residual;
    const uint64_t res_u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(res_addr >> 32)) << 32) |
                           (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)res_addr);
    res_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(res_u), (short)0,
        __builtin_amdgcn_readfirstlane((int)((uint32_t)a.M * (uint32_t)a.Cout * 2)), 0x00020000);
    relu_post_lo = a.relu_post != 0 ? 0.0f : -__builtin_inff();
    asm("" : "+v"(relu_post_lo));
  }
  float arow[MB];
#pragma unroll
  for (int j = 0; j < MB; ++j) arow[j] = row_scales ? a.a_scale_rows[min(mrow[j], a.M - 1)] : 1.f;
  const auto& cs = ch.cs;
  const auto& cb = ch.cb;
  const auto& osc = ch.osc;
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    const int m = mrow[j];
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    u32x2 rv[NB];
    if constexpr (RES) {  // this row block's residual, in flight while its values are computed
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const bool nvalid = n_tile0 + nl0 + i * 16 < a.Cout;
        const uint32_t roff =
            nvalid ? ((uint32_t)m * (uint32_t)a.Cout + (uint32_t)(n_tile0 + nl0 + i * 16 + 4 * g)) * 2 : 0x80000000u;
        rv[i] = __builtin_amdgcn_raw_buffer_load_b64(res_rsrc, (int)roff, 0, 0);
      }
    }
    float y[NB][4];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      float* v = y[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t;
        if (KIND == KIND_INT8)
          t = row_scales ? __fmul_rn((float)acc_i[i][j][e], __fmul_rn(arow[j], cs[i][e]))
                         : __fmul_rn((float)acc_i[i][j][e], cs[i][e]);
        else
          t = acc_f[i][j][e];
        t = __fadd_rn(t, cb[i][e]);  // the staged bias is -0 when there is none
        v[e] = GELU == 1 ? t : __builtin_elementwise_maximum(t, relu_lo);
      }
      round_bf16x2(v[0], v[1]);
      round_bf16x2(v[2], v[3]);
      if (GELU) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu_erf(v[e]);
        if (RES || OUT == OUT_INT8) {  // a BF16 store's pack and the E4M3 conversion round the same way
          round_bf16x2(v[0], v[1]);
          round_bf16x2(v[2], v[3]);
        }
      }
      if constexpr (RES) {  // relu(y + r) in FP32, then BF16 (a BF16 store's pack rounds)
        v[0] = __builtin_elementwise_maximum(__fadd_rn(v[0], u2f(rv[i][0] << 16)), relu_post_lo);
        v[1] = __builtin_elementwise_maximum(__fadd_rn(v[1], u2f(rv[i][0] & 0xffff0000u)), relu_post_lo);
        v[2] = __builtin_elementwise_maximum(__fadd_rn(v[2], u2f(rv[i][1] << 16)), relu_post_lo);
        v[3] = __builtin_elementwise_maximum(__fadd_rn(v[3], u2f(rv[i][1] & 0xffff0000u)), relu_post_lo);
        if (OUT == OUT_INT8) {
          round_bf16x2(v[0], v[1]);
          round_bf16x2(v[2], v[3]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const float* v = y[i];
      const int nbase = n_tile0 + nl0 + i * 16 + 4 * g;
      const bool nvalid = n_tile0 + nl0 + i * 16 < a.Cout;  // whole 16-channel block in or out (Cout % 16 == 0)
      // rows past M land past the buffer's end; invalid channel blocks are sent there too
      const uint32_t off = nvalid ? ((uint32_t)m * (uint32_t)a.out_ld + (uint32_t)nbase) * ESZ : 0x80000000u;
      uint8_t* sd = nullptr;
      if constexpr (STAGE_RB > 0) {
        const int cb = (nl0 + i * 16 + 4 * g) * ESZ;  // the lane's bytes within the staged row
        const int sl = ((cb >> 4) ^ stage_swz(spix[j])) & (STAGE_RB / 16 - 1);
        sd = stage + spix[j] * STAGE_RB + sl * 16 + (cb & 15);
      }
      if (OUT == OUT_BF16) {
        const uint32_t lo = pack_bf16x2(v[0], v[1]), hi = pack_bf16x2(v[2], v[3]);
        if constexpr (STAGE_RB > 0)
          *reinterpret_cast<u32x2*>(sd) = u32x2{lo, hi};
        else
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{lo, hi}, rsrc, (int)off, 0, 0);
      } else {
        uint32_t pk;
        if (OUT == OUT_INT8) {  // the block's 4 values share one near-tie test (one wave-uniform branch)
          const float vq[4] = {v[0], v[1], v[2], v[3]};
          int qi[4];
          quantize_int8_fast_n<4>(vq, out_scale, out_inv, qi);
          pk = (uint32_t)(qi[0] & 0xff) | ((uint32_t)(qi[1] & 0xff) << 8) | ((uint32_t)(qi[2] & 0xff) << 16) |
               ((uint32_t)qi[3] << 24);
        } else {
          pk = e4m3x4_of_bf16(v[0], v[1], v[2], v[3], osc[i], 448.0f * osc[i]);  // rounds to BF16 first
        }
        if constexpr (STAGE_RB > 0)
          *reinterpret_cast<uint32_t*>(sd) = pk;
        else
          __builtin_amdgcn_raw_buffer_store_b32(pk, rsrc, (int)off, 0, 0);
      }
    }
    // this row block's stores (all NB x 16 channels of 16 pixels: whole 128-byte lines of a BF16 output) go out before
    // the next block is computed, so the writes stream during the epilogue and each line is written in one burst
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The fast epilogue's variants (GELU with or without a ReLU before it, dense residual) for lane rows mrow, into global
// memory (STAGE_RB = 0) or an LDS staging tile (see conv_epilogue_fast's STAGE_RB); the caller has checked
// conv_fast_ok.
template <int KIND, int OUT, int MB, int NB, int STAGE_RB = 0>
__device__ __forceinline__ void conv_epilogue_any(const ConvArgs& a, const v4i (&acc_i)[NB][MB],
                                                  const v4f (&acc_f)[NB][MB], const int (&mrow)[MB], int n_tile0,
                                                  int nl0, const EpiChannels<NB>& ch, uint8_t* stage = nullptr,
                                                  const int* spix = nullptr) {
#define FIM_EPI(G, R) \
  conv_epilogue_fast<KIND, OUT, MB, NB, G, R, STAGE_RB>(a, acc_i, acc_f, mrow, n_tile0, nl0, ch, stage, spix)
  const int act = a.gelu ? (a.relu_pre ? 2 : 1) : 0;
  if (a.residual != nullptr) {
    if (act == 1) FIM_EPI(1, true);
    else if (act == 2) FIM_EPI(2, true);
    else FIM_EPI(0, true);
  } else {
    if (act == 1) FIM_EPI(1, false);
    else if (act == 2) FIM_EPI(2, false);
    else FIM_EPI(0, false);
  }
#undef FIM_EPI
}

// Calls f(integral_constant<int, GELU>, integral_constant<bool, RES>) with the fast epilogue's variant for this launch:
// kernels whose epilogue is a loop of calls select the variant once, outside the loop, so the loop body holds one
// variant and unrolls (with the selection inside, the body holds all six and the compiler stops unrolling, which turns
// the accumulator indexing dynamic and puts the accumulators in scratch memory).
template <typename F>
__device__ __forceinline__ void with_epilogue_variant(const ConvArgs& a, F&& f) {
  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;
  using G2 = std::integral_constant<int, 2>;
  using RY = std::integral_constant<bool, true>;
  using RN = std::integral_constant<bool, false>;
  const int act = a.gelu ? (a.relu_pre ? 2 : 1) : 0;
  if (a.residual != nullptr) {
    if (act == 1) f(G1{}, RY{});
    else if (act == 2) f(G2{}, RY{});
    else f(G0{}, RY{});
  } else {
    if (act == 1) f(G1{}, RN{});
    else if (act == 2) f(G2{}, RN{});
    else f(G0{}, RN{});
  }
}

template <int KIND, int OUT, int MB, int NB>
__device__ __forceinline__ void conv_epilogue_rows(const ConvArgs& a, const v4i (&acc_i)[NB][MB],
                                                   const v4f (&acc_f)[NB][MB], const int (&mrow)[MB], int n_tile0,
                                                   int nl0, const EpiChannels<NB>& ch) {
  conv_epilogue_any<KIND, OUT, MB, NB>(a, acc_i, acc_f, mrow, n_tile0, nl0, ch);
}

template <int KIND, int OUT, int MB, int NB>
__device__ __forceinline__ void conv_epilogue_rows(const ConvArgs& a, const v4i (&acc_i)[NB][MB],
                                                   const v4f (&acc_f)[NB][MB], const int (&mrow)[MB], int n_tile0,
                                                   int nl0, const float* ep_scale, const float* ep_bias,
                                                   const float* ep_osc) {
  conv_epilogue_rows<KIND, OUT, MB, NB>(a, acc_i, acc_f, mrow, n_tile0, nl0,
                                        epi_channels<NB>(nl0, ep_scale, ep_bias, ep_osc));
}

// Whether the fast epilogue applies: no residual or a BF16 residual laid out as the output (the refiner blocks'
// contract convs), no pooling, Cout % 16 == 0, the output below 2 GiB.
template <int OUT>
__host__ __device__ __forceinline__ bool conv_fast_ok(const ConvArgs& a) {
  const bool res_dense = a.residual != nullptr && a.res_dtype == FIM_BF16 && a.res_channels == a.Cout && a.rs_c == 1 &&
                         a.rs_w == a.Cout && a.rs_h == (int64_t)a.Wo * a.Cout &&
                         a.rs_b == (int64_t)a.Ho * a.Wo * a.Cout && ((uintptr_t)a.residual & 7) == 0 &&
                         (int64_t)a.M * a.Cout * 2 < (int64_t)0x7fffffff;
  return a.pool_out == nullptr && (a.residual == nullptr || res_dense) && (a.Cout & 15) == 0 &&
         (int64_t)a.M * a.out_ld * (OUT == OUT_BF16 ? 2 : 1) < (int64_t)0x7fffffff;
}

template <int KIND, int OUT, int POOL, int MB, int NB>
__device__ __forceinline__ void conv_epilogue(const ConvArgs& a, const v4i (&acc_i)[NB][MB], const v4f (&acc_f)[NB][MB],
                                              int row0, int n_tile0, int nl0, const float* ep_scale,
                                              const float* ep_bias, const float* ep_osc) {
  if (!POOL && conv_fast_ok<OUT>(a)) {
    int mrow[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) mrow[j] = row0 + j * 16 + (threadIdx.x & 15);
    conv_epilogue_rows<KIND, OUT, MB, NB>(a, acc_i, acc_f, mrow, n_tile0, nl0, ep_scale, ep_bias, ep_osc);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  // flags are uniform (scalar branches); the output format is a template parameter
  const float out_scale = (OUT == OUT_INT8 || POOL) ? *a.out_scale : 1.0f;
  const float out_inv = (OUT == OUT_INT8 || POOL) ? __fdiv_rn(1.0f, out_scale) : 1.0f;
  const bool has_bias = a.bias != nullptr;
  const bool res = a.residual != nullptr;
  const bool relu_pre = a.relu_pre != 0;
  const bool relu_post = a.relu_post != 0;
  const bool res_vec = res && a.res_dtype == FIM_BF16 && a.rs_c == 1 && (((uintptr_t)a.residual) & 7) == 0 &&
                       (a.rs_w % 4) == 0 && (a.rs_h % 4) == 0 && (a.rs_b % 4) == 0;
  const bool out_vec = (a.Cout % 4) == 0;
  int pm[MB], px[MB];
  int64_t roff[MB];
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    const int m = row0 + j * 16 + (lane & 15);
    pm[j] = m;
    roff[j] = 0;
    int img, oh, ow;
    px[j] = pixel_of_row<POOL>(a, m < a.M ? m : 0, img, oh, ow);
    if (res) roff[j] = (int64_t)img * a.rs_b + (int64_t)oh * a.rs_h + (int64_t)ow * a.rs_w;
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int nl = nl0 + i * 16 + 4 * g;
    const int nbase = n_tile0 + nl;
    const float4 cs4 = *reinterpret_cast<const float4*>(&ep_scale[nl]);
    const float4 cb4 = *reinterpret_cast<const float4*>(&ep_bias[nl]);
    const float osc = ep_osc[nl];  // E4M3 output scale of the lane's 4 channels (one 32-channel block)
    const float cs[4] = {cs4.x, cs4.y, cs4.z, cs4.w};
    const float cb[4] = {cb4.x, cb4.y, cb4.z, cb4.w};
    const bool full = nbase + 4 <= a.Cout;
    const bool any = nbase < a.Cout;
    const bool res_full = res_vec && nbase + 4 <= a.res_channels;
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int m = pm[j];
      if (!any || m >= a.M) continue;
      float y[4];
      if (KIND == KIND_INT8 && a.a_scale_rows != nullptr) {
        const float arow = a.a_scale_rows[m];
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = __fmul_rn((float)acc_i[i][j][v], __fmul_rn(arow, cs[v]));
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = KIND == KIND_INT8 ? __fmul_rn((float)acc_i[i][j][v], cs[v]) : acc_f[i][j][v];
      }
      if (has_bias) {
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = __fadd_rn(y[v], cb[v]);
      }
      if (relu_pre) {
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = fmaxf(y[v], 0.0f);
      }
      round_bf16x2(y[0], y[1]);
      round_bf16x2(y[2], y[3]);
      if (a.gelu) {
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = gelu_erf(y[v]);
        round_bf16x2(y[0], y[1]);
        round_bf16x2(y[2], y[3]);
      }
      if (res) {
        float rv[4] = {0.f, 0.f, 0.f, 0.f};
        if (res_full) {
          const uint2 pk = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.residual) + roff[j] + nbase);
          rv[0] = u2f(pk.x << 16);
          rv[1] = u2f(pk.x & 0xffff0000u);
          rv[2] = u2f(pk.y << 16);
          rv[3] = u2f(pk.y & 0xffff0000u);
#pragma unroll
          for (int v = 0; v < 4; ++v) y[v] = __fadd_rn(y[v], rv[v]);
          if (relu_post) {
#pragma unroll
            for (int v = 0; v < 4; ++v) y[v] = fmaxf(y[v], 0.0f);
          }
          round_bf16x2(y[0], y[1]);
          round_bf16x2(y[2], y[3]);
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int n = nbase + v;
            if (n < a.res_channels) {
              const int64_t off = roff[j] + (int64_t)n * a.rs_c;
              const float r = a.res_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.residual)[off])
                                                      : static_cast<const float*>(a.residual)[off];
              float t = __fadd_rn(y[v], r);
              if (relu_post) t = fmaxf(t, 0.0f);
              y[v] = round_bf16_hw(t);
            } else if (relu_post) {
              y[v] = fmaxf(y[v], 0.0f);
            }
          }
        }
      }
      const int64_t o = (int64_t)px[j] * a.out_ld + nbase;
      if (POOL) {
        // the window's 4 pixels sit on lanes 4k .. 4k + 3 of this 16-lane group (rows m = 4 * window + 0..3), all
        // valid or all past M together: max across them, quantize (monotonic, so equal to quantizing the max of the
        // quantized values), one 4-channel store per window
        float p[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          p[v] = fmaxf(y[v], __shfl_xor(y[v], 1));
          p[v] = fmaxf(p[v], __shfl_xor(p[v], 2));
        }
        if ((lane & 3) == 0) {
          uint32_t pk = 0;
#pragma unroll
          for (int v = 0; v < 4; ++v) pk |= (uint32_t)(uint8_t)quantize_int8_fast(p[v], out_scale, out_inv) << (8 * v);
          uint8_t* pdst = reinterpret_cast<uint8_t*>(a.pool_out) + (int64_t)(m >> 2) * a.Cout + nbase;
          if (out_vec && full) {
            *reinterpret_cast<uint32_t*>(pdst) = pk;
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              if (nbase + v < a.Cout) pdst[v] = (uint8_t)(pk >> (8 * v));
          }
        }
      }
      if (OUT == OUT_BF16) {
        uint16_t* dst = static_cast<uint16_t*>(a.out) + o;
        const uint32_t lo = pack_bf16x2(y[0], y[1]), hi = pack_bf16x2(y[2], y[3]);
        if (out_vec && full) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
        } else {
          const uint16_t h[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (nbase + v < a.Cout) dst[v] = h[v];
        }
      } else {
        uint32_t pk;
        if (OUT == OUT_INT8) {
          pk = 0;
#pragma unroll
          for (int v = 0; v < 4; ++v) pk |= (uint32_t)(uint8_t)quantize_int8_fast(y[v], out_scale, out_inv) << (8 * v);
        } else {
          pk = e4m3x4_of_bf16(y[0], y[1], y[2], y[3], osc, 448.0f * osc);
        }
        uint8_t* dst = static_cast<uint8_t*>(a.out) + o;
        if (out_vec && full) {
          *reinterpret_cast<uint32_t*>(dst) = pk;
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (nbase + v < a.Cout) dst[v] = (uint8_t)(pk >> (8 * v));
        }
      }
    }
  }
}

// ONE: the launch has a single K step (K <= 128): one LDS stage and one register set (127-146 VGPRs instead of 254),
// so three workgroups fit on a CU instead of two and more tiles' loads overlap the others' epilogues (refiner stack
// MXFP8 20.4 -> 19.9 ms). A single-stage loop over several K steps keeps the next step's registers live through the
// MFMAs and spills at the three-workgroup register budget.
template <int KIND, int BN, int LW, int OUT, int XS, int POOL, int MBW = 4, bool PACK = false, bool ONE = false>
__global__ __launch_bounds__(256, ONE ? 3 : 2) void conv_igemm_kernel(const ConvArgs a) {
  constexpr int MB = MBW;                // 16-pixel blocks per wavefront (64 pixels; 32 in the tail's small tiles)
  constexpr int BM = 32 * MB;            // pixel rows per tile: two wavefronts of MB blocks
  constexpr int SXN = XS ? MB : 1;       // activation scale registers per set: one per 16-pixel block with row scales
  constexpr int NB = BN / 32;            // 16-channel blocks per wavefront (BN/2 channels)
  constexpr int A_PASSES = BM / 32;      // 256 lanes x 16 B cover 32 rows x 128 B per pass
  constexpr int B_PASSES = BN / 32;
  constexpr int STAGE = (BM + BN) * KC;  // pixel rows first, then weight rows; 128 B per row, XOR-swizzled
  __shared__ __attribute__((aligned(16))) uint8_t lds[(ONE ? 1 : 2) * STAGE];
  __shared__ __attribute__((aligned(16))) float ep_scale[BN], ep_bias[BN], ep_osc[BN];  // per-channel epilogue operands of this N tile

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1;

  // XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs (pid % 8), so each XCD takes a
  // contiguous run of tiles; a run walks the N tiles of one M tile back to back, and consecutive M tiles (which share
  // input halo rows) stay on the same XCD's L2.
  const int per_xcd = gridDim.x >> 3;
  const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (t >= a.n_tiles * a.m_tiles) return;
  const int n0 = (t % a.n_tiles) * BN;
  const int m0 = a.m_base + (t / a.n_tiles) * BM;

  // per-channel epilogue operands, staged once (their loads overlap the prologue; the prologue barrier orders them)
  if (tid < BN) {
    const int n = n0 + tid;
    const bool nok = n < a.Cout;
    ep_scale[tid] = (KIND == KIND_INT8 && nok) ? (a.a_scale_rows != nullptr ? a.w_scale[n] : *a.a_scale * a.w_scale[n])
                                               : 1.0f;
    float bias = -0.0f;  // x + (-0) == x for every x, -0 included: the fast epilogue adds it unconditionally
    if (a.bias != nullptr && nok)
      bias = a.bias_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.bias)[n])
                                      : static_cast<const float*>(a.bias)[n];
    ep_bias[tid] = bias;
    ep_osc[tid] = (OUT == OUT_E4M3 && nok) ? exp2_int((int)a.out_expo[n >> 5]) : 1.0f;  // E4M3 output scale 2^e
  }

  const int seg = tid & 7;    // 16-byte segment of the 128-byte K chunk this lane stages
  const int rsub = tid >> 3;  // row within a 32-row pass
  const int64_t wrow = (int64_t)a.kh * a.kw * a.Cin;

  // gather geometry of this lane's staged pixel rows (32-bit: the host guarantees M < 2^31)
  const uint8_t* a_ptr[A_PASSES];
  int a_h[A_PASSES], a_w[A_PASSES];
#pragma unroll
  for (int j = 0; j < A_PASSES; ++j) {
    const int m = m0 + rsub + 32 * j;
    const bool ok = m < a.M;
    int img, oh, ow;
    pixel_of_row<POOL>(a, ok ? m : 0, img, oh, ow);
    const int ih = oh * a.sh - a.ph, iw = ow * a.sw - a.pw;
    a_h[j] = ok ? ih : -(1 << 28);  // an invalid row never passes the bounds test
    a_w[j] = iw;
    a_ptr[j] = a.x + ((int64_t)(img * a.H + ih) * a.W + iw) * a.Cin + seg * 16;
  }
  const uint8_t* b_ptr[B_PASSES];
  bool b_ok[B_PASSES];
#pragma unroll
  for (int j = 0; j < B_PASSES; ++j) {
    const int n = n0 + rsub + 32 * j;
    b_ok[j] = n < a.Cout;
    b_ptr[j] = a.w + (int64_t)(b_ok[j] ? n : 0) * wrow + seg * 16;
  }
  // LDS byte offsets of this lane's staged segments (swizzle: slot = seg ^ ((row >> 1) & 7))
  int st_a[A_PASSES], st_b[B_PASSES];
#pragma unroll
  for (int j = 0; j < A_PASSES; ++j) {
    const int r = rsub + 32 * j;
    st_a[j] = r * KC + ((seg ^ ((r >> 1) & 7)) << 4);
  }
#pragma unroll
  for (int j = 0; j < B_PASSES; ++j) {
    const int r = BM + rsub + 32 * j;
    st_b[j] = r * KC + ((seg ^ ((r >> 1) & 7)) << 4);
  }
  // LDS byte offsets of this lane's MFMA fragments: row (lane & 15) of each block, K pieces g and g + 4
  const int g = lane >> 4;
  int fr_x[MB], fr_w[NB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int r = wm * (MB * 16) + i * 16 + (lane & 15);
    fr_x[i] = r * KC + ((g ^ ((r >> 1) & 7)) << 4);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int r = BM + wn * (BN / 2) + i * 16 + (lane & 15);
    fr_w[i] = r * KC + ((g ^ ((r >> 1) & 7)) << 4);
  }
  const int cblocks = a.Cin >> 5;
  const int wexp_stride = (int)(wrow >> 5);
  const int8_t* wexp_row[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int n = n0 + wn * (BN / 2) + i * 16 + (lane & 15);
    wexp_row[i] = KIND == KIND_MX ? a.w_expo + (int64_t)(n < a.Cout ? n : 0) * wexp_stride : nullptr;
  }

  // two register sets: the loads of step kt + 2 are issued while step kt + 1 (loaded one step earlier) waits in the
  // other set to be staged, so each load has two steps of MFMA work to land behind
  uint4 ra0[A_PASSES], rb0[B_PASSES], ra1[A_PASSES], rb1[B_PASSES];
  int sx0[SXN], sw0[NB], sx1[SXN], sw1[NB];
#pragma unroll
  for (int j = 0; j < SXN; ++j) sx0[j] = sx1[j] = 0;
  bool bok0 = true, bok1 = true;  // the set's channel block lies inside Cin (else zero data, scale 2^0)
#pragma unroll
  for (int i = 0; i < NB; ++i) sw0[i] = sw1[i] = 0;

  // (tap, channel chunk) of the step being loaded; advanced uniformly
  int ld_ky = 0, ld_kx = 0, ld_c0 = 0;
  int ld_tap0 = 0;  // packed taps (tps > 1): the step's first tap
  const int taps_total = a.kh * a.kw;
  const int seg_sub = (seg * 16) / a.Cin, seg_coff = (seg * 16) % a.Cin;  // packed: this segment's tap and channel
  auto gload = [&](uint4 (&ra)[A_PASSES], uint4 (&rb)[B_PASSES], int (&pre_sx)[SXN], int (&pre_sw)[NB], bool& pre_ok) {
    int dy, dx, cvalid;
    int64_t delta, wdelta;
    if constexpr (PACK) {
      // several taps per step: segment seg holds channels [seg_coff, + 16) of tap ld_tap0 + seg_sub (taps past the
      // filter load the zero segment); the weights of consecutive taps are contiguous in a weight row
      const int tap = ld_tap0 + seg_sub;
      const bool tap_ok = tap < taps_total;
      const int ky = tap_ok ? tap / a.kw : 0, kx = tap_ok ? tap - ky * a.kw : 0;
      dy = ky * a.dh;
      dx = kx * a.dw;
      delta = (int64_t)(dy * a.W + dx) * a.Cin + seg_coff - seg * 16;
      cvalid = tap_ok ? 16 : 0;
      wdelta = (int64_t)ld_tap0 * a.Cin;
    } else {
      dy = ld_ky * a.dh;
      dx = ld_kx * a.dw;
      delta = (int64_t)(dy * a.W + dx) * a.Cin + ld_c0;
      cvalid = a.Cin - ld_c0 - seg * 16;
      wdelta = (int64_t)(ld_ky * a.kw + ld_kx) * a.Cin + ld_c0;
    }
#pragma unroll
    for (int j = 0; j < A_PASSES; ++j) {
      const bool ok = (unsigned)(a_h[j] + dy) < (unsigned)a.H && (unsigned)(a_w[j] + dx) < (unsigned)a.W;
      ra[j] = load_seg<LW>(a_ptr[j] + delta, ok, cvalid);
    }
#pragma unroll
    for (int j = 0; j < B_PASSES; ++j) rb[j] = load_seg<LW>(b_ptr[j] + wdelta, b_ok[j], cvalid);
    if (KIND == KIND_MX) {
      // raw exponent bytes, loaded unconditionally from clamped indices and only turned into E8M0 when the step is
      // computed: consuming them here would make the compiler wait for every load issued so far
      // K block g of the step: packed taps take tap ld_tap0 + 32 g / Cin, channel block (32 g % Cin) / 32
      const int ptap = ld_tap0 + (32 * g) / a.Cin;
      const int blk = PACK ? ((32 * g) % a.Cin) >> 5 : (ld_c0 >> 5) + g;
      const int cblk = blk < cblocks ? blk : cblocks - 1;
      if (XS == 0) {
        pre_sx[0] = (int)a.x_expo[cblk];
      } else {
#pragma unroll
        for (int j = 0; j < SXN; ++j) {
          int r = m0 + wm * (MB * 16) + j * 16 + (lane & 15);
          r = r < a.M ? r : a.M - 1;
          const int rt = r & 127;
          pre_sx[j] = (int)a.x_swz[(((int64_t)(r >> 7) * a.x_swz_tiles_k + (cblk >> 2)) << 9) + (rt & 31) * 16 +
                                   (rt >> 5) * 4 + (cblk & 3)];
        }
      }
      pre_ok = PACK ? ptap < taps_total : blk < cblocks;
      const int wblk = PACK ? min(ptap, taps_total - 1) * cblocks + cblk : (ld_ky * a.kw + ld_kx) * cblocks + cblk;
#pragma unroll
      for (int i = 0; i < NB; ++i) pre_sw[i] = (int)wexp_row[i][wblk];
    }
    ld_tap0 += a.tps;
    ld_c0 += KC;
    if (ld_c0 >= a.Cin) {
      ld_c0 = 0;
      if (++ld_kx == a.kw) {
        ld_kx = 0;
        ++ld_ky;
      }
    }
  };
  auto sstore = [&](int buf, const uint4 (&ra)[A_PASSES], const uint4 (&rb)[B_PASSES]) {
    uint8_t* st = lds + buf * STAGE;
#pragma unroll
    for (int j = 0; j < A_PASSES; ++j) *reinterpret_cast<uint4*>(st + st_a[j]) = ra[j];
#pragma unroll
    for (int j = 0; j < B_PASSES; ++j) *reinterpret_cast<uint4*>(st + st_b[j]) = rb[j];
  };

  v4i acc_i[NB][MB];
  v4f acc_f[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      acc_i[i][j] = v4i{0, 0, 0, 0};
      acc_f[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    }

  const int nk = PACK ? (a.kh * a.kw + a.tps - 1) / a.tps : a.kh * a.kw * a.kchunks;
  gload(ra0, rb0, sx0, sw0, bok0);
  if (!ONE && nk > 1) gload(ra1, rb1, sx1, sw1, bok1);
  sstore(0, ra0, rb0);
  lds_barrier();

  // one K step from LDS stage `buf`; (rsx, rsw): the raw exponent bytes loaded with it; blk_ok false marks a
  // channel block past Cin (zero data: any scale works, use 2^0)
  auto compute = [&](int buf, const int (&rsx)[SXN], const int (&rsw)[NB], bool blk_ok) {
    int sxs[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) sxs[j] = !blk_ok ? 127 : XS ? rsx[j] : rsx[0] + 127;
    int sw[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) sw[i] = blk_ok ? w_scale_byte(a, rsw[i]) : 127;
    const uint8_t* st = lds + buf * STAGE;
    if constexpr (KIND == KIND_INT8) {
      v4i xlo[MB], xhi[MB];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        xlo[i] = *reinterpret_cast<const v4i*>(st + fr_x[i]);
        xhi[i] = *reinterpret_cast<const v4i*>(st + (fr_x[i] ^ 64));
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const v4i wlo = *reinterpret_cast<const v4i*>(st + fr_w[i]);
        const v4i whi = *reinterpret_cast<const v4i*>(st + (fr_w[i] ^ 64));
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wlo, xlo[j], acc_i[i][j], 0, 0, 0);
          acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(whi, xhi[j], acc_i[i][j], 0, 0, 0);
        }
      }
    } else {
      // each operand is built once as the 8-register tuple the MFMA reads, straight from its two LDS reads
      v8i xf[MB];
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const v4i lo = *reinterpret_cast<const v4i*>(st + fr_x[j]);
        const v4i hi = *reinterpret_cast<const v4i*>(st + (fr_x[j] ^ 64));
        xf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const v4i lo = *reinterpret_cast<const v4i*>(st + fr_w[i]);
        const v4i hi = *reinterpret_cast<const v4i*>(st + (fr_w[i] ^ 64));
        const v8i wf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int j = 0; j < MB; ++j)
          acc_f[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf, xf[j], acc_f[i][j], 0, 0, 0, sw[i], 0,
                                                                         sxs[j]);
      }
    }
  };

  if constexpr (ONE) {
    compute(0, sx0, sw0, bok0);
  } else
  // steps alternate register sets: even steps were loaded into set 0, odd steps into set 1
  for (int kt = 0; kt < nk; kt += 2) {
    // even step kt (LDS stage 0, scales in set 0); set 0 is free once staged: load step kt + 2 into it
    {
      int sx[SXN], sw[NB];
      const bool bok = bok0;
#pragma unroll
      for (int j = 0; j < SXN; ++j) sx[j] = sx0[j];
#pragma unroll
      for (int i = 0; i < NB; ++i) sw[i] = sw0[i];
      if (kt + 2 < nk) gload(ra0, rb0, sx0, sw0, bok0);
      compute(0, sx, sw, bok);
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 1 < nk) sstore(1, ra1, rb1);
      lds_barrier();
    }
    if (kt + 1 < nk) {  // odd step kt + 1 (LDS stage 1, set 1); then stage step kt + 2 from set 0
      int sx[SXN], sw[NB];
      const bool bok = bok1;
#pragma unroll
      for (int j = 0; j < SXN; ++j) sx[j] = sx1[j];
#pragma unroll
      for (int i = 0; i < NB; ++i) sw[i] = sw1[i];
      if (kt + 3 < nk) gload(ra1, rb1, sx1, sw1, bok1);
      compute(1, sx, sw, bok);
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 2 < nk) sstore(0, ra0, rb0);
      lds_barrier();
    }
  }

  conv_epilogue<KIND, OUT, POOL, MB, NB>(a, acc_i, acc_f, m0 + wm * (MB * 16), n0, wn * (BN / 2), ep_scale, ep_bias, ep_osc);
}


// Wide tiles: one workgroup of 8 wavefronts per CU over a (WM x 80) x (WN x 64) tile, WM x WN = 8 (160 x 256 or
// 320 x 128), each wavefront 5 x 4 blocks of 16 x 16. Against two resident 128 x 128 workgroups per CU, a CU holds 25%
// more outputs, every operand byte fetched from L2 feeds more MFMAs (config 2: 52 instead of 81 MB of L2 -> CU traffic
// per launch), and the tile counts of large layers fill one round of CUs (config 2: 125 x 2 = 250 tiles on 256 CUs).
// The accumulators take 80 VGPRs, so the operands bypass registers: each 8-row x 128-byte piece of a stage is one
// wave-wide `buffer_load_dwordx4 ... lds` (lane l writes 16 bytes at LDS base + 16 l, so lane l fetches the global
// segment that the XOR swizzle puts at that slot). Out-of-range offsets read as zero, which supplies the conv padding,
// the rows past M and the channels past Cout without branches. Per K step: read this step's fragments from LDS, issue
// the next step's loads into the other stage, run the MFMAs, then wait for the loads and barrier.
// Requires 16-byte-aligned operands with Cin % 16 == 0, x and w below 2 GiB, per-channel MXFP8 activation exponents,
// no pooling; the same MFMA per 16 x 16 block and K step, and the same epilogue, as the 128-row kernel.
constexpr int WIDE_MB = 5, WIDE_NB = 4;
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void vm_lds_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int KIND, int WM, int OUT>
__global__ __launch_bounds__(512, 1) void conv_igemm_wide_kernel(const ConvArgs a) {
  constexpr int WN = 8 / WM;
  constexpr int MB = WIDE_MB, NB = WIDE_NB;
  constexpr int BM = WM * MB * 16, BN = WN * NB * 16;
  constexpr int STAGE = (BM + BN) * KC;
  constexpr int CHUNKS = (BM + BN) / 8;  // 8 rows x 128 bytes: one wave-wide 16-byte-per-lane load
  constexpr int CPW = (CHUNKS + 7) / 8;  // chunks per wavefront (the first CHUNKS % 8 wavefronts take one more)
  constexpr int CPW_MIN = CHUNKS / 8;
  static_assert(BM % 8 == 0 && BN % 8 == 0, "a chunk lies in one operand");
  // Three stages (loads two steps ahead) when they fit in the 160 KB of LDS next to the epilogue operands, else two.
  // Each stage is its own array, so the compiler can tell a stage's reads from the loads in flight into the others.
  constexpr int NST = 3 * STAGE + 3 * BN * 4 <= 163840 ? 3 : 2;
  __shared__ __attribute__((aligned(16))) uint8_t st0[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t st1[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t st2[NST == 3 ? STAGE : 16];
  __shared__ __attribute__((aligned(16))) float ep_scale[BN], ep_bias[BN], ep_osc[BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // provably uniform: the loads' LDS base and descriptor
  const int wm = wave % WM, wn = wave / WM;

  // XCD-aware order as in the 128-row kernel: each XCD takes a contiguous run of tiles, N tiles of an M tile adjacent
  const int per_xcd = gridDim.x >> 3;
  const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (t >= a.n_tiles * a.m_tiles) return;
  const int n0 = (t % a.n_tiles) * BN;
  const int m0 = a.m_base + (t / a.n_tiles) * BM;

  if (tid < BN) {
    const int n = n0 + tid;
    const bool nok = n < a.Cout;
    ep_scale[tid] = (KIND == KIND_INT8 && nok) ? *a.a_scale * a.w_scale[n] : 1.0f;
    float bias = -0.0f;  // x + (-0) == x for every x, -0 included: the fast epilogue adds it unconditionally
    if (a.bias != nullptr && nok)
      bias = a.bias_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.bias)[n])
                                      : static_cast<const float*>(a.bias)[n];
    ep_bias[tid] = bias;
    ep_osc[tid] = (OUT == OUT_E4M3 && nok) ? exp2_int((int)a.out_expo[n >> 5]) : 1.0f;  // E4M3 output scale 2^e
  }

  const int wrow = a.kh * a.kw * a.Cin;  // < 2^31: the host bounds the weight bytes
  // buffer sizes in bytes (< 2^31: checked by the host), through readfirstlane so the descriptors stay in SGPRs
  const int x_nrec = __builtin_amdgcn_readfirstlane((int)((int64_t)a.B * a.H * a.W * a.Cin));
  const int w_nrec = __builtin_amdgcn_readfirstlane(a.Cout * wrow);
  constexpr uint32_t OOB = 0x80000000u;  // past both buffers: reads as zero

  // this lane's 16-byte segment in each of its wavefront's chunks: LDS row r = 8 c + lane / 8, slot lane % 8, holding
  // global segment (lane % 8) ^ ((r / 2) % 8)
  int ch_base[CPW], ch_h[CPW], ch_w[CPW], ch_cof[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int c = wave + 8 * i;
    const int r = 8 * c + (lane >> 3);
    const int seg = (lane & 7) ^ ((r >> 1) & 7);
    ch_cof[i] = seg * 16;
    ch_h[i] = -(1 << 28);
    ch_w[i] = 0;
    ch_base[i] = 0;
    if (c < CHUNKS && r < BM) {
      const int m = m0 + r;
      if (m < a.M) {
        int img, oh, ow;
        pixel_of_row<0>(a, m, img, oh, ow);
        const int ih = oh * a.sh - a.ph, iw = ow * a.sw - a.pw;
        ch_h[i] = ih;
        ch_w[i] = iw;
        ch_base[i] = ((img * a.H + ih) * a.W + iw) * a.Cin + seg * 16;
      }
    } else if (c < CHUNKS) {
      const int n = n0 + r - BM;
      ch_h[i] = n < a.Cout ? 0 : -(1 << 28);  // weight rows: only the row test applies
      ch_base[i] = (n < a.Cout ? n : 0) * wrow + seg * 16;
    }
  }

  const int g = lane >> 4;
  int fr_x[MB], fr_w[NB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int r = wm * (MB * 16) + i * 16 + (lane & 15);
    fr_x[i] = r * KC + ((g ^ ((r >> 1) & 7)) << 4);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int r = BM + wn * (NB * 16) + i * 16 + (lane & 15);
    fr_w[i] = r * KC + ((g ^ ((r >> 1) & 7)) << 4);
  }
  const int cblocks = a.Cin >> 5;
  const int wexp_stride = wrow >> 5;
  const int8_t* wexp_row[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int n = n0 + wn * (NB * 16) + i * 16 + (lane & 15);
    wexp_row[i] = KIND == KIND_MX ? a.w_expo + (int64_t)(n < a.Cout ? n : 0) * wexp_stride : nullptr;
  }

  int ld_ky = 0, ld_kx = 0, ld_c0 = 0;
  // the raw MX exponent bytes of the next (tap, channel chunk) step into (sx, sw). Loaded on every step, also past the
  // last (then from step 0's address, unused): a load issued only on some paths leaves its register a join of two
  // values, and the copy at the join waits for the load (a full vmcnt wait that drains the operand prefetch)
  auto load_exponents = [&](bool more, int& sx, int (&sw)[NB], bool& ok) __attribute__((always_inline)) {
    if (KIND == KIND_MX) {
      const int blk = (ld_c0 >> 5) + g;
      const int cblk = blk < cblocks ? blk : cblocks - 1;
      sx = (int)a.x_expo[more ? cblk : 0];
      ok = blk < cblocks;
      const int wblk = more ? (ld_ky * a.kw + ld_kx) * cblocks + cblk : 0;
#pragma unroll
      for (int i = 0; i < NB; ++i) sw[i] = (int)wexp_row[i][wblk];
    }
  };
  // issue the loads of the next (tap, channel chunk) step into LDS stage `st` and move to the step after it
  auto issue = [&](uint8_t* st) __attribute__((always_inline)) {
    const int dy = ld_ky * a.dh, dx = ld_kx * a.dw;
    const int xdelta = (dy * a.W + dx) * a.Cin + ld_c0;
    const int wdelta = (ld_ky * a.kw + ld_kx) * a.Cin + ld_c0;
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int c = wave + 8 * i;
      if (c < CHUNKS) {  // uniform
        const bool a_rows = 8 * c < BM;
        const bool ok_c = ch_cof[i] < a.Cin - ld_c0;
        const bool ok_r = a_rows ? ((unsigned)(ch_h[i] + dy) < (unsigned)a.H && (unsigned)(ch_w[i] + dx) < (unsigned)a.W)
                                 : ch_h[i] == 0;
        const uint32_t off = (ok_c && ok_r) ? (uint32_t)(ch_base[i] + (a_rows ? xdelta : wdelta)) : OOB;
        // uniform branch; each call builds its descriptor from kernel arguments, so it is provably uniform (a
        // descriptor the compiler cannot prove uniform turns every load into a readfirstlane loop)
        if (a_rows)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.x), (short)0, x_nrec, 0x00020000),
              (lds_void_t*)(st + c * 1024), 16, off, 0, 0, 0);
        else
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), (short)0, w_nrec, 0x00020000),
              (lds_void_t*)(st + c * 1024), 16, off, 0, 0, 0);
      }
    }
    ld_c0 += KC;
    if (ld_c0 >= a.Cin) {
      ld_c0 = 0;
      if (++ld_kx == a.kw) {
        ld_kx = 0;
        ++ld_ky;
      }
    }
  };

  v4i acc_i[NB][MB];
  v4f acc_f[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      acc_i[i][j] = v4i{0, 0, 0, 0};
      acc_f[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    }

  const int nk = a.kh * a.kw * a.kchunks;
  int esx[NST], esw[NST][NB];
  bool eok[NST];
#pragma unroll
  for (int s = 0; s < NST; ++s) {
    esx[s] = 0;
    eok[s] = true;
#pragma unroll
    for (int i = 0; i < NB; ++i) esw[s][i] = 0;
  }

  // one K step from stage `cur` (exponent set ec); the loads of step kt + NST - 1 go into stage `nxt` (set en)
  auto step_live = [&](int kt, const uint8_t* cur, uint8_t* nxt, int ec, int en) __attribute__((always_inline)) {
    // this step's fragments first: the next loads into LDS are issued after them, so no read waits on those. MXFP8
    // operands are built as the 8-register tuples the MFMA reads, straight from their two LDS reads (built later,
    // each tuple costs four 64-bit register moves per step)
    v4i xlo[MB], xhi[MB], wlo[NB], whi[NB];
    v8i xf[MB], wf[NB];
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const v4i lo = *reinterpret_cast<const v4i*>(cur + fr_x[j]);
      const v4i hi = *reinterpret_cast<const v4i*>(cur + (fr_x[j] ^ 64));
      if constexpr (KIND == KIND_MX) {
        xf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      } else {
        xlo[j] = lo;
        xhi[j] = hi;
      }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const v4i lo = *reinterpret_cast<const v4i*>(cur + fr_w[i]);
      const v4i hi = *reinterpret_cast<const v4i*>(cur + (fr_w[i] ^ 64));
      if constexpr (KIND == KIND_MX) {
        wf[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      } else {
        wlo[i] = lo;
        whi[i] = hi;
      }
    }
    int sxs = 127, sw[NB];
    if (KIND == KIND_MX) {
      // the raw bytes made opaque here, where they are used: otherwise the scale arithmetic is moved up to the loads
      // (two steps earlier), which then wait for their data on the spot
      asm volatile("" : "+v"(esx[ec]));
#pragma unroll
      for (int i = 0; i < NB; ++i) asm volatile("" : "+v"(esw[ec][i]));
      sxs = eok[ec] ? esx[ec] + 127 : 127;
#pragma unroll
      for (int i = 0; i < NB; ++i) sw[i] = eok[ec] ? w_scale_byte(a, esw[ec][i]) : 127;
    }
    const bool more = kt + NST - 1 < nk;
    __builtin_amdgcn_sched_barrier(0);
    load_exponents(more, esx[en], esw[en], eok[en]);  // before the stage loads: the wait below then spares those
    __builtin_amdgcn_sched_barrier(0);
    if (more) issue(nxt);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (KIND == KIND_INT8) {
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wlo[i], xlo[j], acc_i[i][j], 0, 0, 0);
          acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(whi[i], xhi[j], acc_i[i][j], 0, 0, 0);
        }
    } else {
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j)
          acc_f[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[i], xf[j], acc_f[i][j], 0, 0, 0, sw[i], 0, sxs);
    }
    __builtin_amdgcn_sched_barrier(0);  // the wait for the next stage stays behind this step's MFMAs
    // step kt + 1's stage loads were issued one step earlier (or in the prologue); when this step issued loads, at
    // least CPW_MIN of this wavefront's loads (its stage loads) are younger than all of them, so vmcnt <= CPW_MIN means
    // they have landed (it may also wait for this step's exponent bytes, issued first, a whole MFMA phase earlier)
    if (NST == 3 && more)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(CPW_MIN) : "memory");
    else
      vm_lds_barrier();
  };
  // a step of the unconditional stage rotation: past the last step (kt >= nk: a uniform branch) only the exponent
  // registers are loaded, so that no loaded register is a join of a load with an older value
  auto step = [&](int kt, const uint8_t* cur, uint8_t* nxt, int ec, int en) __attribute__((always_inline)) {
    if (kt < nk)
      step_live(kt, cur, nxt, ec, en);
    else
      load_exponents(false, esx[en], esw[en], eok[en]);
  };

  if constexpr (NST == 3) {
    load_exponents(true, esx[0], esw[0], eok[0]);
    issue(st0);
    if (nk > 1) {
      load_exponents(true, esx[1], esw[1], eok[1]);
      issue(st1);
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(CPW_MIN) : "memory");
    } else {
      vm_lds_barrier();
    }
    for (int kt = 0; kt < nk; kt += 3) {
      step(kt, st0, st2, 0, 2);
      step(kt + 1, st1, st0, 1, 0);
      step(kt + 2, st2, st1, 2, 1);
    }
  } else {
    load_exponents(true, esx[0], esw[0], eok[0]);
    issue(st0);
    vm_lds_barrier();
    for (int kt = 0; kt < nk; kt += 2) {
      step(kt, st0, st1, 0, 1);
      step(kt + 1, st1, st0, 1, 0);
    }
  }

  conv_epilogue<KIND, OUT, 0, MB, NB>(a, acc_i, acc_f, m0 + wm * (MB * 16), n0, wn * (NB * 16), ep_scale, ep_bias,
                                      ep_osc);
}

// ---- Patch tiles -----------------------------------------------------------------------------------------------
// Stride-1, dilation-1 3 x 3 convolutions with Cin == 128 (each of the 9 K steps is one tap's 128 channels).
// Persistent workgroups of 8 wavefronts, one per CU, walk tiles of TH x TW (8 x 16) output pixels of one image x 64
// output channels.
// * The workgroup's 64 output channels of the weights (9 taps x 64 x 128 B = 72 KB) stay in LDS for all its tiles
//   (tiles are dealt so a workgroup keeps one channel block), with their MX exponents packed into registers.
// * Per tile the (TH + 2) x (TW + 2) x 128-byte input patch is staged in LDS once (wave-wide `buffer_load ... lds`,
//   pixels outside the image read as zero) and every tap reads its operand rows from the patch at the tap's offset:
//   each activation byte crosses L2 -> LDS once instead of once per tap.
// * Two groups of four wavefronts work on alternate tiles, half a tile period apart: while one group's K loop keeps
//   the matrix cores busy, the other group (one wavefront per SIMD as well) runs its previous tile's epilogue on the
//   VALU, stages the output in LDS, writes it out in whole 128-byte lines and loads its next patch.
// * The K loop has no barrier and no global load: the next tap's operand rows are read from LDS between the current
//   tap's MFMAs.
// The epilogue is the conv kernels' fast epilogue (same arithmetic per value).

// LDS slots. ds_read_b128 serves a wavefront in four passes of 16 lanes (the lanes with equal bit 5 and equal parity
// of bits 2..4 of the lane index) over 64 four-byte banks, i.e. 16 groups of 16 bytes: a pass is conflict-free when its
// 16 addresses fall in 16 distinct groups. A 128-byte row r covers groups 8 (r % 2) .. + 8, its 16-byte slot s
// group 8 (r % 2) + s.
// Weight rows: channel segment s of output channel r sits in slot s ^ patch_swz(r); a wavefront's 16 consecutive
// channels read conflict-free.
__device__ __forceinline__ int patch_swz(int r) { return (r >> 1) & 7; }
// Patch pixels (rows of 18 pixels): segment s of the pixel in column c sits in slot s ^ patch_col_swz(c), from a table
// of 3-bit entries searched so that the reads of 16 consecutive columns starting at column 0, 1 or 2 (the three tap
// columns), low and high K halves (slots s and s ^ 4), are conflict-free in every pass (and measured so).
constexpr uint64_t PATCH_COL_SWZ = 0x27c980a7358f67ULL;
__device__ __forceinline__ int patch_col_swz(int c) { return (int)((PATCH_COL_SWZ >> (3 * c)) & 7); }

// s_waitcnt immediate (gfx9 encoding) for at most `vm` outstanding vector memory operations and no LDS/scalar ones:
// vmcnt in bits 3:0 and 15:14, expcnt (7: no wait) in 6:4, lgkmcnt (0) in 11:8. Issued through the builtin, so the
// compiler's own wait counting sees it.
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 0xF) | (0x7 << 4) | (((vm >> 4) & 0x3) << 14); }

// s_waitcnt for at most n (wave-uniform, at most 15; larger waits for 15) outstanding vector memory operations
__device__ __forceinline__ void wait_vm_at_most(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0)); break;
    case 1: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(1)); break;
    case 2: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2)); break;
    case 3: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(3)); break;
    case 4: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(4)); break;
    case 5: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(5)); break;
    case 6: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(6)); break;
    case 7: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(7)); break;
    case 8: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(8)); break;
    case 9: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(9)); break;
    case 10: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(10)); break;
    case 11: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(11)); break;
    case 12: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(12)); break;
    case 13: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(13)); break;
    case 14: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(14)); break;
    default: __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(15)); break;
  }
}

// Scaled MXFP8 MFMA with the A-operand scale taken from byte i (0..3, a constant after unrolling) of scale_a.
__device__ __forceinline__ v4f mfma_scale_opsel(const v8i& a, const v8i& b, v4f c, int i, int scale_a, int scale_b) {
  switch (i) {
    case 0: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, scale_a, 0, scale_b);
    case 1: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 1, scale_a, 0, scale_b);
    case 2: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 2, scale_a, 0, scale_b);
    default: return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 3, scale_a, 0, scale_b);
  }
}

// Two groups of four wavefronts (wavefront w in group w / 4 runs on SIMD w % 4, so each SIMD holds one wavefront of each
// group) take alternate tiles in a two-phase software pipeline: in each phase one group runs a tile's K loop (MFMA and
// LDS reads) while the other runs the epilogue of its previous tile (VALU, LDS staging, stores) and loads its next
// patch, and a workgroup barrier ends the phase. Each group has its own patch buffer; wavefront w % 4 of a group owns
// tile pixels [16 MB (w % 4), +16 MB) x the 64 channels.
template <int KIND, int OUT, int TH, int TW>
__global__ __launch_bounds__(512, 1) void conv_patch_kernel(const ConvArgs a) {
  constexpr int KW = 3, TAPS = 9, NB = 4, BN = 64;
  constexpr int MB = TH * TW / 64;  // 16-pixel blocks per wavefront
  static_assert(MB * 64 == TH * TW, "four wavefronts of MB blocks cover the tile");
  // patch rows of PW = TW + 2 pixels; a 16-pixel block is one tile row, and the slot follows the column, so the operand
  // addresses of the 9 taps are 3 column-offset sets plus constant row offsets
  static_assert(TW == 16, "pixel blocks are tile rows, patch rows the 18 columns the slot table covers");
  constexpr int PW = TW + 2, NP = (TH + 2) * PW;
  constexpr int PCHUNKS = (NP + 7) / 8;          // wave-wide 1 KB loads of 8 patch pixels
  constexpr int PATCH_BYTES = PCHUNKS * 1024;    // one patch buffer
  constexpr int WTS_BYTES = TAPS * BN * KC;
  constexpr int WEXP_BYTES = KIND == KIND_MX ? TAPS * 4 * BN : 16;
  // output staging: a wavefront's pixels in SROUNDS rounds of SPIX pixels, RB bytes (64 channels) each
  constexpr int ESZ = OUT == OUT_BF16 ? 2 : 1;
  constexpr int RB = BN * ESZ, LPP = RB / 16, PPC = 64 / LPP;
  constexpr int SROUNDS = MB, SPIX = 16;          // one 16-pixel block per round
  constexpr int SCH = SPIX / PPC;                // 1 KB stores per round
  static_assert(SPIX % PPC == 0, "whole 1 KB stores per round");
  constexpr int STAGE_BYTES = 4 * SPIX * RB;
  // one LDS block with fixed offsets, the two patch buffers first: a patch operand read is the lane's column offset
  // (plus the group's buffer) in a register and the tap-row offset as the instruction's 16-bit immediate
  static_assert(2 * PW * KC < 65536, "tap row offsets fit the immediate");
  __shared__ __attribute__((aligned(1024)))
  uint8_t smem[2 * PATCH_BYTES + WTS_BYTES + STAGE_BYTES + WEXP_BYTES + 3 * BN * 4 + 16];
  uint8_t* const wts = smem + 2 * PATCH_BYTES;           // [tap][channel][128 B]
  uint8_t* const stage = wts + WTS_BYTES;                // [wavefront % 4][pixel][RB]
  uint8_t* const wexp_s = stage + STAGE_BYTES;           // [channel][tap][block] (MXFP8)
  float* const ep_scale = reinterpret_cast<float*>(wexp_s + WEXP_BYTES);
  float* const ep_bias = ep_scale + BN;
  float* const ep_osc = ep_bias + BN;
  uint8_t* const xexp_s = reinterpret_cast<uint8_t*>(ep_osc + BN);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  const int grp = wave >> 2, wq = wave & 3;

  const int tiles_x = (a.Wo + TW - 1) / TW, tiles_y = (a.Ho + TH - 1) / TH;
  const int total = a.n_tiles * tiles_x * tiles_y * a.B;
  // XCD-aware deal (workgroup p runs on XCD p % 8): each XCD takes contiguous runs of tiles; the grid is a multiple of
  // the channel-block count, so every tile of a workgroup has the same channel block. The workgroup's tiles are
  // first, first + stride, ...; group q takes those with an even (q = 0) or odd (q = 1) index.
  const int stride = gridDim.x;
  const int per_xcd = stride >> 3;
  const int first = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (first >= total) return;
  const int n0 = (first % a.n_tiles) * BN;
  const int n_mine = (total - first + stride - 1) / stride;  // tiles of the workgroup
  const int n_grp = (n_mine - grp + 1) >> 1;                 // ... of this group
  // phases: the group's k-th tile runs its K loop in phase 2 k + grp and its epilogue in the phase after
  const int n_phases = max(2 * ((n_mine + 1) >> 1), 2 * (n_mine >> 1) + 1);
  uint8_t* const buf = smem + grp * PATCH_BYTES;

  const int x_nrec = __builtin_amdgcn_readfirstlane((int)((int64_t)a.B * a.H * a.W * KC));
  const int w_nrec = __builtin_amdgcn_readfirstlane(a.Cout * TAPS * KC);
  constexpr uint32_t OOB = 0x80000000u;

  // weights: chunk k = wave + 8 i (i < 9) holds rows (tap k / 8, channels 8 (k % 8) .. + 8) at wts + 1024 k
#pragma unroll
  for (int i = 0; i < TAPS * BN / 64; ++i) {
    const int k = wave + 8 * i;
    const int tap = k >> 3, r = 8 * (k & 7) + (lane >> 3);
    const int seg = (lane & 7) ^ patch_swz(r);
    const uint32_t off = n0 + r < a.Cout ? (uint32_t)(((n0 + r) * TAPS + tap) * KC + seg * 16) : OOB;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), (short)0, w_nrec, 0x00020000),
        (lds_void_t*)(wts + k * 1024), 16, off, 0, 0, 0);
  }

  auto tile_origin = [&](int t, int& img, int& oy0, int& ox0) __attribute__((always_inline)) {
    int rest = t / a.n_tiles;
    ox0 = (rest % tiles_x) * TW;
    rest /= tiles_x;
    oy0 = (rest % tiles_y) * TH;
    img = rest / tiles_y;
  };
  // patch of tile t into this group's buffer: load i of the group's wavefront q brings patch pixels 8 (q + 4 i) .. + 8
  // (pixels outside the image and past NP read as zero)
  constexpr int PLOADS = (PCHUNKS + 3) / 4;
  const int my_patch = (PCHUNKS - wq + 3) >> 2;  // this wavefront's loads per patch
  auto load_patch = [&](int t) __attribute__((always_inline)) {
    int img, oy0, ox0;
    tile_origin(t, img, oy0, ox0);
    int lid = lane;
    asm volatile("" : "+v"(lid));  // per-lane coordinates recomputed per tile instead of held in registers
#pragma unroll
    for (int i = 0; i < PLOADS; ++i) {
      const int c = wq + 4 * i;
      if (c < PCHUNKS) {
        const int q = 8 * c + (lid >> 3);
        const int col = q % PW;
        const int seg = (lid & 7) ^ patch_col_swz(col);
        const int iy = oy0 - a.ph + q / PW, ix = ox0 - a.pw + col;
        const bool ok = q < NP && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
        const uint32_t off = ok ? (uint32_t)(((img * a.H + iy) * a.W + ix) * KC + seg * 16) : OOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.x), (short)0, x_nrec, 0x00020000),
            (lds_void_t*)(buf + c * 1024), 16, off, 0, 0, 0);
      }
    }
  };
  if (grp < n_mine) load_patch(first + grp * stride);

  if (tid < BN) {
    const int n = n0 + tid;
    const bool nok = n < a.Cout;
    ep_scale[tid] = (KIND == KIND_INT8 && nok) ? *a.a_scale * a.w_scale[n] : 1.0f;
    float bias = -0.0f;
    if (a.bias != nullptr && nok)
      bias = a.bias_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.bias)[n])
                                      : static_cast<const float*>(a.bias)[n];
    ep_bias[tid] = bias;
    ep_osc[tid] = (OUT == OUT_E4M3 && nok) ? exp2_int((int)a.out_expo[n >> 5]) : 1.0f;
  }
  if constexpr (KIND == KIND_MX) {
    // E8M0 bytes of the weight rows (past Cout: 2^0), one contiguous run of BN x 36 bytes: every load is issued
    // before the first LDS store, so the prologue waits for one memory round trip, not one per pass
    constexpr int WEXP_N = TAPS * 4 * BN, WEXP_PASSES = (WEXP_N + 511) / 512;
    const int64_t wexp_valid = ((int64_t)a.Cout - n0) * (TAPS * 4);
    int e[WEXP_PASSES];
#pragma unroll
    for (int i = 0; i < WEXP_PASSES; ++i) {
      const int idx = tid + 512 * i;
      e[i] = idx < WEXP_N && idx < wexp_valid ? w_scale_byte(a, a.w_expo[(int64_t)n0 * (TAPS * 4) + idx]) : 127;
    }
#pragma unroll
    for (int i = 0; i < WEXP_PASSES; ++i)
      if (tid + 512 * i < WEXP_N) wexp_s[tid + 512 * i] = (uint8_t)e[i];
    if (tid < 4) xexp_s[tid] = (uint8_t)((int)a.x_expo[tid] + 127);
  }

  // operand rows: this wavefront's pixel blocks as patch pixels at tap (0, 0) in its group's buffer, the weight rows
  int pofs[KW][MB][2];  // LDS byte offsets at tap column dx (row dy adds dy * PW rows): K pieces g and g + 4
#pragma unroll
  for (int dx = 0; dx < KW; ++dx)
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int p = wq * (MB * 16) + j * 16 + (lane & 15);
      const int q = (p / TW) * PW + (p % TW) + dx;
      pofs[dx][j][0] = grp * PATCH_BYTES + q * KC + ((g ^ patch_col_swz(q % PW)) << 4);
      pofs[dx][j][1] = pofs[dx][j][0] ^ 64;
    }
  int fr_w[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int r = i * 16 + (lane & 15);
    fr_w[i] = r * KC + ((g ^ patch_swz(r)) << 4);
  }
  int fw[NB][2];  // the weight offsets, made opaque per tile (else all 9 taps' weight rows are hoisted into registers)
  auto read_x = [&](int kt, int j, v8i& xf) __attribute__((always_inline)) {
    const uint8_t* prow = smem + (kt / KW) * PW * KC;
    const v4i lo = *reinterpret_cast<const v4i*>(prow + pofs[kt % KW][j][0]);
    const v4i hi = *reinterpret_cast<const v4i*>(prow + pofs[kt % KW][j][1]);
    xf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  auto read_w = [&](int kt, v8i (&wf)[NB]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const v4i lo = *reinterpret_cast<const v4i*>(smem + fw[i][0] + kt * (BN * KC));
      const v4i hi = *reinterpret_cast<const v4i*>(smem + fw[i][1] + kt * (BN * KC));
      wf[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };

  v4i acc_i[NB][MB];
  v4f acc_f[NB][MB];
  // MXFP8 scales in registers for every tile: the lane's activation block g, and per tap one dword of the E8M0 bytes
  // of its 4 weight rows (the MFMA's op_sel picks byte i)
  int sx = 127, swp[TAPS];
  // the group's first patch, the weights and the staged operands
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  asm volatile("s_barrier" ::: "memory");
  if constexpr (KIND == KIND_MX) {
    sx = xexp_s[g];
#pragma unroll
    for (int t = 0; t < TAPS; ++t) {
      uint32_t packed = 0;
#pragma unroll
      for (int i = 0; i < NB; ++i)
        packed |= (uint32_t)wexp_s[(i * 16 + (lane & 15)) * (TAPS * 4) + t * 4 + g] << (8 * i);
      swp[t] = (int)packed;
    }
  }

  // K loop of a tile: the activation rows of the next tap and the weight rows of the next tap are read while a tap's
  // MFMAs are issued (two register sets each)
  auto k_loop = [&]() __attribute__((always_inline)) {
    v8i xs[2][MB], ws[2][NB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        acc_i[i][j] = v4i{0, 0, 0, 0};
        acc_f[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      fw[i][0] = 2 * PATCH_BYTES + fr_w[i];
      fw[i][1] = 2 * PATCH_BYTES + (fr_w[i] ^ 64);
      asm volatile("" : "+v"(fw[i][0]), "+v"(fw[i][1]));
    }
#pragma unroll
    for (int j = 0; j < MB; ++j) read_x(0, j, xs[0][j]);
    read_w(0, ws[0]);
#pragma unroll
    for (int kt = 0; kt < TAPS; ++kt) {
      if (kt + 1 < TAPS) {
#pragma unroll
        for (int j = 0; j < MB; ++j) read_x(kt + 1, j, xs[(kt + 1) & 1][j]);
        read_w(kt + 1, ws[(kt + 1) & 1]);
      }
      const v8i (&xf)[MB] = xs[kt & 1];
      const v8i (&wc)[NB] = ws[kt & 1];
#pragma unroll
      for (int j = 0; j < MB; ++j)
#pragma unroll
        for (int i = 0; i < NB; ++i) {
          if constexpr (KIND == KIND_INT8) {
            acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(wc[i], wc[i], 0, 1, 2, 3),
                                                                __builtin_shufflevector(xf[j], xf[j], 0, 1, 2, 3),
                                                                acc_i[i][j], 0, 0, 0);
            acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(wc[i], wc[i], 4, 5, 6, 7),
                                                                __builtin_shufflevector(xf[j], xf[j], 4, 5, 6, 7),
                                                                acc_i[i][j], 0, 0, 0);
          } else {
            acc_f[i][j] = mfma_scale_opsel(wc[i], xf[j], acc_f[i][j], i, swp[kt], sx);
          }
        }
      // one wavefront per SIMD runs the K loop: the next tap's LDS reads are issued one by one between this tap's
      // MFMAs, in their shadow, instead of as a burst the matrix core waits behind
      if (kt + 1 < TAPS) {
        constexpr int NMFMA = MB * NB * (KIND == KIND_INT8 ? 2 : 1), NREAD = 2 * (MB + NB);
#pragma unroll
        for (int n = 0; n < NMFMA; ++n) {
          if (n < NREAD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // one MFMA
        }
        if (NREAD > NMFMA) __builtin_amdgcn_sched_group_barrier(0x100, NREAD > NMFMA ? NREAD - NMFMA : 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // the accumulators pinned here: left free, the MFMAs would be sunk into the epilogue phase, and every operand they
    // read would stay live until then
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        if constexpr (KIND == KIND_INT8)
          asm volatile("" : "+v"(acc_i[i][j]));
        else
          asm volatile("" : "+v"(acc_f[i][j]));
      }
  };

  // epilogue of tile t: first the loads of the group's next patch (its buffer is free: the K loop finished in the
  // previous phase), then the values, staged per wavefront in rounds and written out in whole lines; at the end this
  // wavefront's patch loads (issued before its stores) are waited for
  const int nbytes = __builtin_amdgcn_readfirstlane((int)((uint32_t)a.M * (uint32_t)a.out_ld * ESZ));
  auto epilogue = [&](int t, int next) __attribute__((always_inline)) {
    if (next < total) load_patch(next);
    int eo = 0;
    asm volatile("" : "+v"(eo));  // the per-channel operands re-read from LDS per tile, not held across the K loop
    const EpiChannels<NB> ch = epi_channels<NB>(0, ep_scale + eo, ep_bias + eo, ep_osc + eo);
    int img, oy0, ox0;
    tile_origin(t, img, oy0, ox0);
    const uint64_t out_addr = (uint64_t)a.out;
    const uint64_t out_u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(out_addr >> 32)) << 32) |
                           (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)out_addr);
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(out_u), (short)0, nbytes, 0x00020000);
    uint8_t* const my_stage = stage + wq * (SPIX * RB);
    const int sl = lane % LPP;
    const bool cvalid = n0 + sl * (16 / ESZ) < a.Cout;
    with_epilogue_variant(a, [&](auto gv, auto rv) __attribute__((always_inline)) {
      constexpr int G = decltype(gv)::value;
      constexpr bool R = decltype(rv)::value;
#pragma unroll
      for (int r = 0; r < SROUNDS; ++r) {
        constexpr int RMB = MB / SROUNDS;  // pixel blocks per round
        static_assert(RMB * SROUNDS == MB, "rounds split the blocks");
        int mrow[RMB], spix[RMB];
        v4i ai[NB][RMB];
        v4f af[NB][RMB];
#pragma unroll
        for (int j = 0; j < RMB; ++j) {
          const int p = wq * (MB * 16) + (r * RMB + j) * 16 + (lane & 15);
          const int oy = oy0 + p / TW, ox = ox0 + p % TW;
          mrow[j] = (oy < a.Ho && ox < a.Wo) ? (img * a.Ho + oy) * a.Wo + ox : a.M;
          spix[j] = j * 16 + (lane & 15);
#pragma unroll
          for (int i = 0; i < NB; ++i) {
            ai[i][j] = acc_i[i][r * RMB + j];
            af[i][j] = acc_f[i][r * RMB + j];
          }
        }
        conv_epilogue_fast<KIND, OUT, RMB, NB, G, R, RB>(a, ai, af, mrow, n0, 0, ch, my_stage, spix);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));  // this wavefront's staged rows (LDS ops run in order)
#pragma unroll
        for (int c = 0; c < SCH; ++c) {
          const int pl = c * PPC + lane / LPP;                              // pixel within the round
          const int p = wq * (MB * 16) + r * SPIX + pl;                     // pixel within the tile
          typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
          const u32x4 v = *reinterpret_cast<const u32x4*>(my_stage + pl * RB + ((sl ^ stage_swz(pl)) & (LPP - 1)) * 16);
          const int oy = oy0 + p / TW, ox = ox0 + p % TW;
          const bool ok = cvalid && oy < a.Ho && ox < a.Wo;
          const uint32_t off =
              ok ? ((uint32_t)((img * a.Ho + oy) * a.Wo + ox) * (uint32_t)a.out_ld + (uint32_t)n0) * ESZ + sl * 16
                 : OOB;
          __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, (int)off, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));  // the staged rows read before the next round overwrites them
      }
    });
    // this wavefront's patch loads landed before the phase barrier hands the patch to its group: a full vmcnt(0), as
    // the stores issued after them may complete first (the counter makes no order between loads and stores)
    if (next < total) __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  };

  for (int ph = 0; ph < n_phases; ++ph) {
    const int kk = ph - grp;
    if (kk >= 0) {
      const int k = kk >> 1;  // the group's k-th tile: the workgroup's tile 2 k + grp
      const int t = first + (2 * k + grp) * stride;
      if (k < n_grp) {
        if ((kk & 1) == 0)
          k_loop();
        else
          epilogue(t, t + 2 * stride);
      }
    }
    asm volatile("s_barrier" ::: "memory");
  }
}

// Patch tiles: 8 x 16 output pixels x 64 channels (config 3: 1300 tiles, at most 6 per workgroup for 5.08 on average:
// 18.98 us; 12 x 16 tiles, 884 of them, at most 4 for 3.45, 19.5 us; 4 x 16, 19.8 us).
constexpr int PATCH_TH = 8, PATCH_TW = 16;

static int64_t patch_grid(int64_t tiles, int64_t n_tiles) {
  // a multiple of 8 (XCDs) and of the channel-block count (each workgroup keeps one), at most one per CU
  int64_t x = 8, y = n_tiles;
  while (y != 0) {
    const int64_t r = x % y;
    x = y;
    y = r;
  }
  const int64_t unit = 8 * n_tiles / x;
  const int64_t cap = std::max<int64_t>(unit, device_cus() / unit * unit);
  return std::min<int64_t>(cdiv(tiles, unit) * unit, cap);
}

// Whether the patch kernel applies: 3 x 3, stride 1, dilation 1, Cin == 128, the fast epilogue's output layout (with a
// 16-byte aligned output for the whole-line stores), no pooling, per-row scales or pre-swizzled input.
static bool patch_ok(const ConvArgs& a, int lw, bool fast_ok) {
  if (lw != 16 || !fast_ok || a.x_swz != nullptr || a.pool_out != nullptr || a.a_scale_rows != nullptr) return false;
  if (a.Cin != KC || a.kh != 3 || a.kw != 3 || a.sh != 1 || a.sw != 1 || a.dh != 1 || a.dw != 1) return false;
  if (((uintptr_t)a.out & 15) != 0 || a.out_ld != a.Cout) return false;
  if ((int64_t)a.B * a.H * a.W * a.Cin >= (1LL << 31) - 16 || (int64_t)a.Cout * a.kh * a.kw * a.Cin >= (1LL << 31))
    return false;
  return (int64_t)a.B * cdiv(a.Ho, PATCH_TH) * cdiv(a.Wo, PATCH_TW) * cdiv(a.Cout, 64) < (1LL << 30);
}

template <int KIND>
static int launch_patch(ConvArgs a, hipStream_t stream) {
  a.n_tiles = (int)cdiv(a.Cout, 64);
  const int64_t tiles = (int64_t)a.B * cdiv(a.Ho, PATCH_TH) * cdiv(a.Wo, PATCH_TW) * a.n_tiles;
  const dim3 grid((unsigned)patch_grid(tiles, a.n_tiles));
  constexpr int QOUT = KIND == KIND_INT8 ? OUT_INT8 : OUT_E4M3;
  if (a.out_mode == OUT_BF16)
    conv_patch_kernel<KIND, OUT_BF16, PATCH_TH, PATCH_TW><<<grid, dim3(512), 0, stream>>>(a);
  else
    conv_patch_kernel<KIND, QOUT, PATCH_TH, PATCH_TW><<<grid, dim3(512), 0, stream>>>(a);
  return launch_status();
}

// ---- Pointwise, register operands --------------------------------------------------------------------------------
// Pointwise (1 x 1, stride 1) convolutions, a GEMM over pixels, with Cin % 128 == 0, Cin <= 512 or 1024, and Cout >=
// 128, where the epilogue (GELU above all) or the HBM traffic (big-K contracts) outweighs the MFMAs. Persistent
// workgroups of 8 wavefronts, one per CU, keep the weights of 128 output channels in LDS (128 x Cin bytes, read-only
// after the prologue); every wavefront then works alone, with no barrier: it loads its tile's 32 pixel rows of
// activations straight into MFMA operand registers (up to 4 K steps at a time), runs 2 x 8 blocks of 16 x 16 against
// the LDS weights, and writes its epilogue through a private LDS staging area in whole lines. Two wavefronts per SIMD drift apart, so one's loads
// and MFMAs run while the other's epilogue keeps the VALU busy.
// XS = 1: MXFP8 activations with per-row E8M0 scales in the 128x4 swizzled layout (mxfp8_scaled_mm's dynamic
// quantization), read per tile with the rows; XS = 0: per-channel-block exponents.
template <int KIND, int OUT, int KS, int XS = 0>
__global__ __launch_bounds__(512, 1) void conv_pw_kernel(const ConvArgs a) {
  constexpr int BN = 128, MB = 2, NB = 8, TMW = MB * 16;  // a wavefront's tile: 32 pixels x 128 channels
  constexpr int WTS_BYTES = KS * BN * KC;                // [K step][channel][128 B]
  constexpr int XEXP_BYTES = (KS * 4 + 15) / 16 * 16;    // the activations' MX exponent bytes (XS = 0)
  constexpr int WEXP_BYTES = KIND == KIND_MX ? BN * KS * 4 : 16;
  constexpr int ESZ = OUT == OUT_BF16 ? 2 : 1;
  // K steps per operand load phase: a tile's activations for KH steps sit in registers (2 KH x 8 VGPRs), so KS > 4
  // runs its K loop in phases of 4 steps
  constexpr int KH = KS < 4 ? KS : 4;
  static_assert(KS % KH == 0, "whole load phases");
  // staged row: the 64 channels of one pixel per channel half (HS: KS > 4, where the weights take 128 KB of LDS and a
  // BF16 half row is still one whole 128-byte line), else all 128
  constexpr bool HS = KS > 4;
  constexpr int RB = (HS ? BN / 2 : BN) * ESZ, LPP = RB / 16, PPC = 64 / LPP;
  constexpr int SCH = 16 / PPC;  // 1 KB stores per 16-pixel round
  static_assert(SCH * PPC == 16, "whole stores per round");
  constexpr int STAGE_BYTES = 8 * 16 * RB;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[WTS_BYTES + STAGE_BYTES + WEXP_BYTES + 3 * BN * 4 + XEXP_BYTES];
  uint8_t* const wts = smem;
  uint8_t* const stage = wts + WTS_BYTES;
  uint8_t* const wexp_s = stage + STAGE_BYTES;           // [channel][K block] (MXFP8)
  float* const ep_scale = reinterpret_cast<float*>(wexp_s + WEXP_BYTES);
  float* const ep_bias = ep_scale + BN;
  float* const ep_osc = ep_bias + BN;
  uint8_t* const xexp_s = reinterpret_cast<uint8_t*>(ep_osc + BN);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;

  // tiles: 8 x 32 pixels x 128 channels, wavefront w taking pixels [32 w, +32); XCD-aware deal as in the patch kernel,
  // the workgroup keeping one channel block
  const int m_tiles = (a.M + 8 * TMW - 1) / (8 * TMW);
  const int total = a.n_tiles * m_tiles;
  const int stride = gridDim.x;
  const int per_xcd = stride >> 3;
  const int first = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (first >= total) return;
  const int n0 = (first % a.n_tiles) * BN;

  const int x_nrec = __builtin_amdgcn_readfirstlane((int)((int64_t)a.M * a.Cin));
  const int w_nrec = __builtin_amdgcn_readfirstlane(a.Cout * a.Cin);
  constexpr uint32_t OOB = 0x80000000u;
#pragma unroll
  for (int i = 0; i < KS * BN / 64; ++i) {  // weights: chunk k (8 channels x 128 bytes of one K step) = wave + 8 i
    const int k = wave + 8 * i;
    const int ks = k / (BN / 8), r = 8 * (k % (BN / 8)) + (lane >> 3);
    const int seg = (lane & 7) ^ patch_swz(r);
    const uint32_t off = n0 + r < a.Cout ? (uint32_t)((n0 + r) * a.Cin + ks * KC + seg * 16) : OOB;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), (short)0, w_nrec, 0x00020000),
        (lds_void_t*)(wts + k * 1024), 16, off, 0, 0, 0);
  }
  if (tid < BN) {
    const int n = n0 + tid;
    const bool nok = n < a.Cout;
    ep_scale[tid] = (KIND == KIND_INT8 && nok) ? *a.a_scale * a.w_scale[n] : 1.0f;
    float bias = -0.0f;
    if (a.bias != nullptr && nok)
      bias = a.bias_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.bias)[n])
                                      : static_cast<const float*>(a.bias)[n];
    ep_bias[tid] = bias;
    ep_osc[tid] = (OUT == OUT_E4M3 && nok) ? exp2_int((int)a.out_expo[n >> 5]) : 1.0f;
  }
  if constexpr (KIND == KIND_MX) {
    constexpr int WEXP_N = BN * KS * 4, WEXP_PASSES = (WEXP_N + 511) / 512;
    const int64_t wexp_valid = ((int64_t)a.Cout - n0) * (KS * 4);
    int e[WEXP_PASSES];
#pragma unroll
    for (int i = 0; i < WEXP_PASSES; ++i) {
      const int idx = tid + 512 * i;
      e[i] = idx < WEXP_N && idx < wexp_valid ? w_scale_byte(a, a.w_expo[(int64_t)n0 * (KS * 4) + idx]) : 127;
    }
#pragma unroll
    for (int i = 0; i < WEXP_PASSES; ++i)
      if (tid + 512 * i < WEXP_N) wexp_s[tid + 512 * i] = (uint8_t)e[i];
    if (XS == 0 && tid < KS * 4) xexp_s[tid] = (uint8_t)((int)a.x_expo[tid] + 127);
  }

  // activation operands straight from global memory: block j, K step ks is the lane's row's bytes [16 g, +16) and
  // [64 + 16 g, +16) of the step (rows past M read as zero)
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.x), (short)0, x_nrec, 0x00020000);
  auto load_x = [&](int t, int kb, v8i (&xa)[MB][KH], int (&sr)[MB][KH]) __attribute__((always_inline)) {
    const int m0 = (t / a.n_tiles) * (8 * TMW) + wave * TMW;
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int m = m0 + j * 16 + (lane & 15);
      if constexpr (XS == 1) {  // the row's E8M0 byte of K block 4 ks + g
        const int r = m < a.M ? m : a.M - 1, rt = r & 127;
#pragma unroll
        for (int k = 0; k < KH; ++k) {
          const int cb = 4 * (kb + k) + g;
          sr[j][k] = (int)a.x_swz[(((int64_t)(r >> 7) * a.x_swz_tiles_k + (cb >> 2)) << 9) + (rt & 31) * 16 +
                                   (rt >> 5) * 4 + (cb & 3)];
        }
      }
      const uint32_t base = m < a.M ? (uint32_t)(m * a.Cin + 16 * g) : OOB;
#pragma unroll
      for (int k = 0; k < KH; ++k) {
        const int ks = kb + k;
        const v4i lo = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(base + ks * KC), 0, 0));
        const v4i hi =
            __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(base + ks * KC + 64), 0, 0));
        xa[j][k] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
  };

  int wo[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int r = i * 16 + (lane & 15);
    wo[i] = r * KC + ((g ^ patch_swz(r)) << 4);
  }
  auto read_w = [&](int ofs) __attribute__((always_inline)) {
    const v4i lo = *reinterpret_cast<const v4i*>(smem + ofs);
    const v4i hi = *reinterpret_cast<const v4i*>(smem + (ofs ^ 64));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  int sxs[KS], swp[KS][2];
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  asm volatile("s_barrier" ::: "memory");  // the weights and staged operands (the last barrier of the kernel)
  if constexpr (KIND == KIND_MX) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      sxs[ks] = XS == 0 ? (int)xexp_s[ks * 4 + g] : 127;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          packed |= (uint32_t)wexp_s[((4 * h + i) * 16 + (lane & 15)) * (KS * 4) + ks * 4 + g] << (8 * i);
        swp[ks][h] = (int)packed;
      }
    }
  }

  const int nbytes = __builtin_amdgcn_readfirstlane((int)((uint32_t)a.M * (uint32_t)a.out_ld * ESZ));
  const uint64_t out_addr = (uint64_t)a.out;
  const uint64_t out_u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(out_addr >> 32)) << 32) |
                         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)out_addr);
  const __amdgpu_buffer_rsrc_t orsrc =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(out_u), (short)0, nbytes, 0x00020000);
  uint8_t* const my_stage = stage + wave * (16 * RB);

  // one tile: its operand loads are waited for right away; the other wavefront on the SIMD runs meanwhile
  auto run_tile = [&](int t) __attribute__((always_inline)) {
    int wq[NB];  // weight offsets made opaque per tile (else all K steps' weight operands are hoisted)
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      wq[i] = wo[i];
      asm volatile("" : "+v"(wq[i]));
    }
    v4i acc_i[NB][MB];
    v4f acc_f[NB][MB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        acc_i[i][j] = v4i{0, 0, 0, 0};
        acc_f[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int kb = 0; kb < KS; kb += KH) {  // load phases: one for KS <= 4
      v8i xc[MB][KH];
      int sr[MB][KH];  // per-row scales (XS = 1)
      load_x(t, kb, xc, sr);
      v8i wc[2];
      wc[0] = read_w(wq[0] + kb * (BN * KC));
#pragma unroll
      for (int k = 0; k < KH; ++k)
#pragma unroll
        for (int i = 0; i < NB; ++i) {
          const int ks = kb + k;
          const int nx = k * NB + i + 1;  // the next weight block of this phase, read while this one's MFMAs run
          if (nx < KH * NB) wc[nx & 1] = read_w(wq[nx % NB] + (kb + nx / NB) * (BN * KC));
          const v8i& w = wc[(k * NB + i) & 1];
#pragma unroll
          for (int j = 0; j < MB; ++j) {
            if constexpr (KIND == KIND_INT8) {
              acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(w, w, 0, 1, 2, 3),
                                                                  __builtin_shufflevector(xc[j][k], xc[j][k], 0, 1, 2, 3),
                                                                  acc_i[i][j], 0, 0, 0);
              acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(w, w, 4, 5, 6, 7),
                                                                  __builtin_shufflevector(xc[j][k], xc[j][k], 4, 5, 6, 7),
                                                                  acc_i[i][j], 0, 0, 0);
            } else {
              acc_f[i][j] = mfma_scale_opsel(w, xc[j][k], acc_f[i][j], i & 3, swp[ks][i >> 2],
                                             XS == 1 ? sr[j][k] : sxs[ks]);
            }
          }
        }
    }
    // the accumulators pinned (else the MFMAs are sunk into the epilogue with their operands live)
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        if constexpr (KIND == KIND_INT8)
          asm volatile("" : "+v"(acc_i[i][j]));
        else
          asm volatile("" : "+v"(acc_f[i][j]));
      }
    // epilogue: 16 pixels per round, staged in this wavefront's LDS area and written in whole lines
    const int m0 = (t / a.n_tiles) * (8 * TMW) + wave * TMW;
    const int sl = lane % LPP;
    // the staged rows out in whole lines: 16 pixels x RB bytes, from channel n0 + nh on
    auto write_stage = [&](int r, int nh) __attribute__((always_inline)) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
      const bool cvalid = n0 + nh + sl * (16 / ESZ) < a.Cout;
#pragma unroll
      for (int c = 0; c < SCH; ++c) {
        const int pl = c * PPC + lane / LPP;
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = *reinterpret_cast<const u32x4*>(my_stage + pl * RB + ((sl ^ stage_swz(pl)) & (LPP - 1)) * 16);
        const int mm = m0 + r * 16 + pl;
        const uint32_t off =
            cvalid && mm < a.M ? ((uint32_t)mm * (uint32_t)a.out_ld + (uint32_t)(n0 + nh)) * ESZ + sl * 16 : OOB;
        __builtin_amdgcn_raw_buffer_store_b128(v, orsrc, (int)off, 0, 0);
      }
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
    };
    with_epilogue_variant(a, [&](auto gv, auto rv) __attribute__((always_inline)) {
      constexpr int G = decltype(gv)::value;
      constexpr bool R = decltype(rv)::value;
#pragma unroll
      for (int r = 0; r < MB; ++r) {
        int mrow[1], spix[1];
        const int m = m0 + r * 16 + (lane & 15);
        mrow[0] = m < a.M ? m : a.M;
        spix[0] = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // channel halves: 4 blocks' per-channel operands in registers at a time
          int eo = 0;
          asm volatile("" : "+v"(eo));
          const EpiChannels<4> ch = epi_channels<4>(64 * h, ep_scale + eo, ep_bias + eo, ep_osc + eo);
          v4i ai[4][1];
          v4f af[4][1];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            ai[i][0] = acc_i[4 * h + i][r];
            af[i][0] = acc_f[4 * h + i][r];
          }
          if constexpr (HS) {  // this half's 64 channels staged as a row of their own, then written out
            conv_epilogue_fast<KIND, OUT, 1, 4, G, R, RB>(a, ai, af, mrow, n0 + 64 * h, 0, ch, my_stage, spix);
            write_stage(r, 64 * h);
          } else {
            conv_epilogue_fast<KIND, OUT, 1, 4, G, R, RB>(a, ai, af, mrow, n0, 64 * h, ch, my_stage, spix);
          }
        }
        if constexpr (!HS) write_stage(r, 0);
      }
    });
  };

  for (int t = first; t < total; t += stride) run_tile(t);
}

// Whether the pointwise kernel applies: 1 x 1, stride 1, no padding, Cin one of 128, 256, 384, 512 or 1024,
// Cout >= 128 (Cout % 16 == 0 by the fast epilogue), dense 16-byte aligned output, no pooling / per-row scales.
static int pw_ks(const ConvArgs& a, int lw, bool fast_ok) {
  if (lw != 16 || !fast_ok || a.pool_out != nullptr || a.a_scale_rows != nullptr) return 0;
  if (a.kh != 1 || a.kw != 1 || a.sh != 1 || a.sw != 1 || a.ph != 0 || a.pw != 0) return 0;
  if (a.Cin % KC != 0 || (a.Cin > 4 * KC && a.Cin != 8 * KC) || a.Cout < 128 || ((uintptr_t)a.out & 15) != 0 ||
      a.out_ld != a.Cout)
    return 0;
  if ((int64_t)a.M * a.Cin >= (1LL << 31) - 16 || (int64_t)a.Cout * a.Cin >= (1LL << 31)) return 0;
  // at least two 256-pixel tiles per CU: with fewer, most wavefronts run one tile with nothing to overlap its loads
  // and epilogue against, and the one-round wide tiles are faster (config 2: 19.4 against 25 us; the refiner
  // stack's many-round layers: 19.0 -> 18.1 ms)
  if (cdiv((int64_t)a.M, 256) * cdiv((int64_t)a.Cout, 128) < 2 * device_cus()) return 0;
  return a.Cin / KC;
}

template <int KIND, int OUT, int XS>
static void launch_pw_ks(const ConvArgs& a, int ks, dim3 grid, hipStream_t stream) {
  switch (ks) {
    case 1: conv_pw_kernel<KIND, OUT, 1, XS><<<grid, dim3(512), 0, stream>>>(a); break;
    case 2: conv_pw_kernel<KIND, OUT, 2, XS><<<grid, dim3(512), 0, stream>>>(a); break;
    case 3: conv_pw_kernel<KIND, OUT, 3, XS><<<grid, dim3(512), 0, stream>>>(a); break;
    case 4: conv_pw_kernel<KIND, OUT, 4, XS><<<grid, dim3(512), 0, stream>>>(a); break;
    default: conv_pw_kernel<KIND, OUT, 8, XS><<<grid, dim3(512), 0, stream>>>(a); break;
  }
}

template <int KIND, int OUT>
static void launch_pw_out(const ConvArgs& a, int ks, dim3 grid, hipStream_t stream) {
  if constexpr (KIND == KIND_MX) {
    if (a.x_swz != nullptr) {
      launch_pw_ks<KIND, OUT, 1>(a, ks, grid, stream);
      return;
    }
  }
  launch_pw_ks<KIND, OUT, 0>(a, ks, grid, stream);
}

template <int KIND>
static int launch_pw(ConvArgs a, int ks, hipStream_t stream) {
  a.n_tiles = (int)cdiv(a.Cout, 128);
  const int64_t tiles = cdiv((int64_t)a.M, 256) * a.n_tiles;
  const dim3 grid((unsigned)patch_grid(tiles, a.n_tiles));
  constexpr int QOUT = KIND == KIND_INT8 ? OUT_INT8 : OUT_E4M3;
  if (a.out_mode == OUT_BF16)
    launch_pw_out<KIND, OUT_BF16>(a, ks, grid, stream);
  else
    launch_pw_out<KIND, QOUT>(a, ks, grid, stream);
  return launch_status();
}

// ---- Pointwise, whole K resident ---------------------------------------------------------------------------------
// 1 x 1 stride-1 convolutions with Cin a multiple of 128 up to 512 and about one to two 160-pixel tiles per CU (config
// 2: 125 x 4 tiles on 256 CUs), where every other kernel here runs each CU's work as one serial sequence of loads,
// MFMAs and a long GELU epilogue. Persistent workgroups of 8 wavefronts, one per CU, keep one 128-channel block:
// * the block's weights (128 x Cin bytes) and a tile's activations (160 x Cin bytes) are all in LDS at once (K steps
//   side by side, [step][row][128 B] with the conv stages' slot swizzle), so the K loop has no barrier and no wait;
// * after a tile's MFMAs, one barrier, then the next tile's activation loads (wave-wide `buffer_load ... lds`) are
//   issued and run while this tile's epilogue keeps the VALU busy; the weights are loaded once.
// Wavefront w takes 80 pixels (w % 2) x 32 channels (w / 2): 5 x 2 blocks of 16 x 16, 7 fragment reads per 10 MFMAs.
constexpr int RES_MB = 5, RES_NB = 2, RES_WM = 2, RES_BM = RES_WM * RES_MB * 16, RES_BN = 4 * RES_NB * 16;

template <int KIND, int OUT, int KS>
__global__ __launch_bounds__(512, 1) void conv_1x1_resident_kernel(const ConvArgs a) {
  constexpr int MB = RES_MB, NB = RES_NB, BM = RES_BM, BN = RES_BN;
  constexpr int STAGE = (BM + BN) * KC;       // one K step: activation rows, then weight rows
  constexpr int ACH = BM / 8, BCH = BN / 8;   // 1 KB chunks (8 rows x 128 B) per K step
  // one array per K step: the compiler tracks LDS-DMA writes per array, so a step's fragment reads wait only for the
  // loads into that step (one array for all would make every read wait for every load in flight)
  __shared__ __attribute__((aligned(1024))) uint8_t stage0[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t stage1[KS > 1 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage2[KS > 2 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage3[KS > 3 ? STAGE : 16];
  auto stage_of = [&](int st) __attribute__((always_inline)) -> uint8_t* {
    return st == 0 ? stage0 : st == 1 ? stage1 : st == 2 ? stage2 : stage3;
  };
  __shared__ __attribute__((aligned(16))) float ep_scale[BN], ep_bias[BN], ep_osc[BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % RES_WM, wn = wave / RES_WM;
  const int g = lane >> 4;

  // tiles (m tile, channel block), dealt as in the pointwise kernel: XCD-aware, one channel block per workgroup
  const int m_tiles = (a.M + BM - 1) / BM;
  const int total = a.n_tiles * m_tiles;
  const int stride = gridDim.x;
  const int per_xcd = stride >> 3;
  const int first = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (first >= total) return;
  const int n0 = (first % a.n_tiles) * BN;

  // Prologue: every load is issued without a branch (small operands by range-checked buffer loads, out-of-range and
  // absent operands reading as zero; the operand chunks unconditional), so the compiler counts them exactly and its
  // waits for the small operands do not wait for the operand chunks issued after them.
  const int n_ep = min(n0 + tid, a.Cout - 1);  // lanes >= BN compute a value nobody stores
  float ep_s = 1.0f, ep_b, ep_o = 1.0f;
  {
    const bool bf = a.bias_dtype == FIM_BF16, has = a.bias != nullptr;
    const int esz = bf ? 2 : 4;
    const void* bp = has ? a.bias : static_cast<const void*>(fim_zero_segment);
    const __amdgpu_buffer_rsrc_t br =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(bp), (short)0, has ? a.Cout * esz : 0, 0x00020000);
    // two 16-bit loads (the high one reads past a BF16 bias's last element as zero): both always issued, so no
    // branch; the value is selected afterwards
    const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(br, n_ep * esz, 0, 0);
    const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(br, n_ep * esz + 2, 0, 0);
    const uint32_t lsh = bf ? 16u : 0u, hmask = bf ? 0u : 0xffffffffu;  // arithmetic, so both loads are always used
    const uint32_t bits = (lo << lsh) | ((hi << 16) & hmask);
    ep_b = has ? __builtin_bit_cast(float, bits) : -0.0f;  // -0: x + (-0) == x
    if constexpr (KIND == KIND_INT8) {
      const float as = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.a_scale), (short)0, 4, 0x00020000), 0, 0, 0));
      const float ws = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.w_scale), (short)0, a.Cout * 4, 0x00020000),
          n_ep * 4, 0, 0));
      ep_s = as * ws;
    }
    if constexpr (OUT == OUT_E4M3) {
      const int8_t oe = (int8_t)__builtin_amdgcn_raw_buffer_load_b8(
          __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(a.out_expo), (short)0, (a.Cout + 31) >> 5, 0x00020000),
          n_ep >> 5, 0, 0);
      ep_o = exp2_int((int)oe);
    }
  }

  const int x_nrec = __builtin_amdgcn_readfirstlane((int)((int64_t)a.M * a.Cin));
  const int w_nrec = __builtin_amdgcn_readfirstlane(a.Cout * a.Cin);
  constexpr uint32_t OOB = 0x80000000u;
  // lane's row within a chunk and the global segment it fetches (slot lane % 8 holds segment (lane % 8) ^ ((r / 2) % 8))
  const int crow = lane >> 3;

  // MXFP8 scales per K step: the lane's activation block 4 st + g and its weight rows' bytes of that block
  int sx[KS], sw[KS][NB];
  if constexpr (KIND == KIND_MX) {
    const int cblocks = a.Cin >> 5;
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(a.x_expo), (short)0, cblocks, 0x00020000);
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(a.w_expo), (short)0, a.Cout * cblocks, 0x00020000);
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      sx[st] = (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(xr, 4 * st + g, 0, 0) + 127;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int n = min(n0 + wn * (NB * 16) + i * 16 + (lane & 15), a.Cout - 1);
        sw[st][i] = w_scale_byte(a, (int8_t)__builtin_amdgcn_raw_buffer_load_b8(wr, n * cblocks + 4 * st + g, 0, 0));
      }
    }
  }

  asm volatile("" ::: "memory");  // the small loads stay ahead of the operand loads (the compiler would sink them)

  // K step st of tile t's activation rows (rows past M read as zero): chunks wave + 8 i of the step's ACH; where that
  // is past ACH, the wavefront loads its chunk of the previous i again (the same bytes to the same place), so every
  // wavefront issues the same number of loads and no branch
  constexpr int NA = (ACH + 7) / 8, NW = (BCH + 7) / 8;
  auto load_a_step = [&](int t, int st) __attribute__((always_inline)) {
    const int m0 = (t / a.n_tiles) * BM;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int c = wave + 8 * i < ACH ? wave + 8 * i : wave + 8 * i - 8;
      const int r = 8 * c + crow;
      const int seg = (lane & 7) ^ ((r >> 1) & 7);
      const int m = m0 + r;
      const uint32_t off = m < a.M ? (uint32_t)(m * a.Cin + st * KC + seg * 16) : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.x), (short)0, x_nrec, 0x00020000),
          (lds_void_t*)(stage_of(st) + c * 1024), 16, off, 0, 0, 0);
    }
  };
  // K step st of the block's weight rows (channels past Cout read as zero)
  auto load_w_step = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const int c = wave + 8 * i < BCH ? wave + 8 * i : wave + 8 * i - 8;
      const int r = BM + 8 * c + crow;  // LDS row
      const int seg = (lane & 7) ^ ((r >> 1) & 7);
      const int n = n0 + r - BM;
      const uint32_t off = n < a.Cout ? (uint32_t)(n * a.Cin + st * KC + seg * 16) : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), (short)0, w_nrec, 0x00020000),
          (lds_void_t*)(stage_of(st) + (ACH + c) * 1024), 16, off, 0, 0, 0);
    }
  };
  // the first tile step by step, each step's weights and activations together: its K loop starts once step 0 landed
  // and waits for each further step as it reaches it, instead of for all of them
#pragma unroll
  for (int st = 0; st < KS; ++st) {
    load_w_step(st);
    load_a_step(first, st);
  }
  constexpr int PER_STEP = NA + NW;  // loads per step of every wavefront
  if (tid < BN) {
    ep_scale[tid] = ep_s;
    ep_bias[tid] = ep_b;
    ep_osc[tid] = ep_o;
  }

  // fragment offsets within a K step (the conv stages' layout: lo half at f, hi half at f ^ 64)
  int fr_x[MB], fr_w[NB];
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    const int r = wm * (MB * 16) + j * 16 + (lane & 15);
    fr_x[j] = r * KC + ((g ^ ((r >> 1) & 7)) << 4);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int r = BM + wn * (NB * 16) + i * 16 + (lane & 15);
    fr_w[i] = r * KC + ((g ^ ((r >> 1) & 7)) << 4);
  }

  // one tile; FIRST (a constant): the first tile, whose K steps wait for their own loads. The first tile is peeled off
  // the loop so that the loop's K steps follow only the counted wait at the end of the previous tile: with the first
  // tile's waits under a branch inside the loop, the compiler's own wait before the LDS reads merged both paths and
  // became a full vmcnt(0), which also waited for the previous tile's output stores
  auto run_tile = [&](int t, auto first_c) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first_c)::value;
    v4i acc_i[NB][MB];
    v4f acc_f[NB][MB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        acc_i[i][j] = v4i{0, 0, 0, 0};
        acc_f[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      if constexpr (FIRST) {  // step st of the first tile (and, at step 0, the staged epilogue operands) landed
        wait_vm_at_most((KS - 1 - st) * PER_STEP);
        asm volatile("s_barrier" ::: "memory");
      }
      const uint8_t* cur = stage_of(st);
      v8i xf[MB], wf[NB];
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const v4i lo = *reinterpret_cast<const v4i*>(cur + fr_x[j]);
        const v4i hi = *reinterpret_cast<const v4i*>(cur + (fr_x[j] ^ 64));
        xf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const v4i lo = *reinterpret_cast<const v4i*>(cur + fr_w[i]);
        const v4i hi = *reinterpret_cast<const v4i*>(cur + (fr_w[i] ^ 64));
        wf[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          if constexpr (KIND == KIND_INT8) {
            acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(wf[i], wf[i], 0, 1, 2, 3),
                                                                __builtin_shufflevector(xf[j], xf[j], 0, 1, 2, 3),
                                                                acc_i[i][j], 0, 0, 0);
            acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(wf[i], wf[i], 4, 5, 6, 7),
                                                                __builtin_shufflevector(xf[j], xf[j], 4, 5, 6, 7),
                                                                acc_i[i][j], 0, 0, 0);
          } else {
            acc_f[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[i], xf[j], acc_f[i][j], 0, 0, 0,
                                                                           sw[st][i], 0, sx[st]);
          }
        }
    }
    // the accumulators pinned (else the MFMAs sink into the epilogue, past the barrier, with their operands live)
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        if constexpr (KIND == KIND_INT8)
          asm volatile("" : "+v"(acc_i[i][j]));
        else
          asm volatile("" : "+v"(acc_f[i][j]));
      }
    lds_barrier();  // every wavefront has read this tile's activations
    const int next = t + stride;
    if (next < total) {
#pragma unroll
      for (int st = 0; st < KS; ++st) load_a_step(next, st);
    }
    {  // the fast epilogue (the host launches this kernel only where it applies)
      int mrow[MB];
#pragma unroll
      for (int j = 0; j < MB; ++j) mrow[j] = (t / a.n_tiles) * BM + wm * (MB * 16) + j * 16 + (lane & 15);
      conv_epilogue_rows<KIND, OUT, MB, NB>(a, acc_i, acc_f, mrow, n0, wn * (NB * 16), ep_scale, ep_bias, ep_osc);
    }
    // the next tile's activations landed in every wavefront's chunks before any wavefront reads them. A full vmcnt(0):
    // the epilogue's stores, issued after the activation loads, may complete before them (the counter makes no order
    // between loads and stores), so no smaller count proves the loads done. Unconditional (also after the last tile),
    // so that the compiler's own accounting sees this wait on every path into the next tile's LDS reads
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    asm volatile("s_barrier" ::: "memory");
  };
  run_tile(first, std::true_type{});
  for (int t = first + stride; t < total; t += stride) run_tile(t, std::false_type{});
}

// Whether the resident-K pointwise kernel applies: the pointwise kernel's shape conditions (1 x 1, stride 1, no
// padding, Cin % 128 == 0 up to 512, 16-byte aligned operands and output), the fast epilogue and at least one
// 160-pixel tile per CU.
static int res_ks(const ConvArgs& a, int lw, bool fast_ok) {
  // the fast epilogue only: the kernel's waits count its stores (the general epilogue's shapes take the other kernels)
  if (lw != 16 || !fast_ok || a.pool_out != nullptr || a.a_scale_rows != nullptr || a.x_swz != nullptr) return 0;
  if (a.kh != 1 || a.kw != 1 || a.sh != 1 || a.sw != 1 || a.ph != 0 || a.pw != 0) return 0;
  if (a.Cin % KC != 0 || a.Cin > 4 * KC || a.Cout < 128) return 0;
  if ((int64_t)a.M * a.Cin >= (1LL << 31) - 16 || (int64_t)a.Cout * a.Cin >= (1LL << 31)) return 0;
  if (cdiv((int64_t)a.M, RES_BM) * cdiv((int64_t)a.Cout, RES_BN) < device_cus()) return 0;
  return a.Cin / KC;
}

template <int KIND, int OUT>
static void launch_res_ks(const ConvArgs& a, int ks, dim3 grid, hipStream_t stream) {
  switch (ks) {
    case 1: conv_1x1_resident_kernel<KIND, OUT, 1><<<grid, dim3(512), 0, stream>>>(a); break;
    case 2: conv_1x1_resident_kernel<KIND, OUT, 2><<<grid, dim3(512), 0, stream>>>(a); break;
    case 3: conv_1x1_resident_kernel<KIND, OUT, 3><<<grid, dim3(512), 0, stream>>>(a); break;
    default: conv_1x1_resident_kernel<KIND, OUT, 4><<<grid, dim3(512), 0, stream>>>(a); break;
  }
}

template <int KIND>
static int launch_res(ConvArgs a, int ks, hipStream_t stream) {
  a.n_tiles = (int)cdiv(a.Cout, RES_BN);
  const int64_t tiles = cdiv((int64_t)a.M, RES_BM) * a.n_tiles;
  const dim3 grid((unsigned)patch_grid(tiles, a.n_tiles));
  constexpr int QOUT = KIND == KIND_INT8 ? OUT_INT8 : OUT_E4M3;
  if (a.out_mode == OUT_BF16)
    launch_res_ks<KIND, OUT_BF16>(a, ks, grid, stream);
  else
    launch_res_ks<KIND, QOUT>(a, ks, grid, stream);
  return launch_status();
}

template <int KIND, int WM>
static void launch_wide(const ConvArgs& a, dim3 grid, hipStream_t stream) {
  constexpr int QOUT = KIND == KIND_INT8 ? OUT_INT8 : OUT_E4M3;
  if (a.out_mode == OUT_BF16)
    conv_igemm_wide_kernel<KIND, WM, OUT_BF16><<<grid, dim3(512), 0, stream>>>(a);
  else
    conv_igemm_wide_kernel<KIND, WM, QOUT><<<grid, dim3(512), 0, stream>>>(a);
}

// 64 x 64 tiles (2 x 2 blocks per wavefront) on the plain path: the tail of a split launch, and launches too small to
// reach every CU with 128-row tiles. With a.tps > 1 (Cin 16, 32, 64; 16-byte loads) the packed-tap variant.
template <int KIND>
static void launch_tail(const ConvArgs& a, int lw, dim3 grid, hipStream_t stream) {
  constexpr int QOUT = KIND == KIND_INT8 ? OUT_INT8 : OUT_E4M3;
  const bool pack = a.tps > 1 && lw == 16;
  if (a.out_mode == OUT_BF16) {
    if (pack)
      conv_igemm_kernel<KIND, 64, 16, OUT_BF16, 0, 0, 2, true><<<grid, dim3(256), 0, stream>>>(a);
    else if (lw == 16)
      conv_igemm_kernel<KIND, 64, 16, OUT_BF16, 0, 0, 2><<<grid, dim3(256), 0, stream>>>(a);
    else
      conv_igemm_kernel<KIND, 64, 1, OUT_BF16, 0, 0, 2><<<grid, dim3(256), 0, stream>>>(a);
  } else {
    if (pack)
      conv_igemm_kernel<KIND, 64, 16, QOUT, 0, 0, 2, true><<<grid, dim3(256), 0, stream>>>(a);
    else if (lw == 16)
      conv_igemm_kernel<KIND, 64, 16, QOUT, 0, 0, 2><<<grid, dim3(256), 0, stream>>>(a);
    else
      conv_igemm_kernel<KIND, 64, 1, QOUT, 0, 0, 2><<<grid, dim3(256), 0, stream>>>(a);
  }
}

template <int KIND, int BN, int OUT, int XS, int POOL = 0>
static void launch_lw(const ConvArgs& a, int lw, dim3 grid, hipStream_t stream) {
  if constexpr (XS == 0 && POOL == 0) {
    if (lw == 16 && a.kh * a.kw * a.kchunks == 1) {
      conv_igemm_kernel<KIND, BN, 16, OUT, 0, 0, 4, false, true><<<grid, dim3(256), 0, stream>>>(a);
      return;
    }
  }
  if (lw == 16)
    conv_igemm_kernel<KIND, BN, 16, OUT, XS, POOL><<<grid, dim3(256), 0, stream>>>(a);
  else
    conv_igemm_kernel<KIND, BN, 1, OUT, XS, POOL><<<grid, dim3(256), 0, stream>>>(a);
}

template <int KIND, int BN, int XS>
static void launch_bn(const ConvArgs& a, int lw, dim3 grid, hipStream_t stream) {
  constexpr int QOUT = KIND == KIND_INT8 ? OUT_INT8 : OUT_E4M3;
  if (a.out_mode == OUT_BF16)
    launch_lw<KIND, BN, OUT_BF16, XS>(a, lw, grid, stream);
  else
    launch_lw<KIND, BN, QOUT, XS>(a, lw, grid, stream);
}

template <int KIND, int BN>
static void launch_xs(const ConvArgs& a, int lw, dim3 grid, hipStream_t stream) {
  if constexpr (KIND == KIND_INT8) {
    if (a.pool_out != nullptr) {
      launch_lw<KIND, BN, OUT_BF16, 0, 1>(a, lw, grid, stream);
      return;
    }
  }
  if constexpr (KIND == KIND_MX) {
    if (a.x_swz != nullptr) {
      launch_bn<KIND, 64, 1>(a, lw, grid, stream);  // row scales take 8 more VGPRs: the 64-channel tile keeps them
      return;
    }
  }
  launch_bn<KIND, BN, 0>(a, lw, grid, stream);
}

// Wide tiles (conv_igemm_wide_kernel) when they apply and their tiles fill at least 85% of one round of one workgroup
// per CU; the wavefront grid is the one whose N tiles pad Cout the least (ties: 256-channel tiles).
// Returns WM (2: 160 x 256 tiles, 4: 320 x 128) or 0.
static int wide_wm(const ConvArgs& a, int lw) {
  if (lw != 16 || a.x_swz != nullptr || a.pool_out != nullptr || a.a_scale_rows != nullptr || a.Cout <= 64) return 0;
  if ((int64_t)a.B * a.H * a.W * a.Cin >= (1LL << 31) - 16 || (int64_t)a.Cout * a.kh * a.kw * a.Cin >= (1LL << 31))
    return 0;
  const int wm = cdiv((int64_t)a.Cout, 256) * 256 <= cdiv((int64_t)a.Cout, 128) * 128 ? 2 : 4;
  const int64_t tiles = cdiv((int64_t)a.M, wm * 80) * cdiv((int64_t)a.Cout, (8 / wm) * 64);
  const int64_t cus = device_cus();
  // One round only: over several rounds the one workgroup per CU runs its tiles back to back (each tile's epilogue
  // and the next tile's loads do not overlap), while two 128-row workgroups per CU overlap them (the refiner stack's
  // many-round 1x1 layers: 23.8 -> 22.2 ms with this rule, one-round configs 2 and 3 unchanged).
  if (tiles > cus) return 0;
  return tiles * 100 >= cus * 85 ? wm : 0;
}

// Small 3x3 INT8 convs (config 1: 1 x 128 x 128, 64 -> 64): stride 1, pad 1, Cin = 64, output width a multiple of 64,
// too few 128-row tiles to fill the CUs. A workgroup takes 64 consecutive output pixels (one row segment) x R3_TN
// output channels and loads everything it needs in one phase: the 3 x 66-pixel input patch (12.7 KB, zeros outside
// the image) and the N tile's whole weight (R3_TN rows x 576 B), then runs the 9 taps from LDS (one
// v_mfma_i32_16x16x64_i8 per tap and 16 x 16 block: wave w takes pixels 16 w .. 16 w + 15 x all the tile's channels)
// and the shared epilogue. Against the 64 x 64 tile kernel's five dependent K steps (each a round trip to L2), there is one
// load latency per workgroup. INT8 sums are exact, so the tap order does not change the result.
constexpr int R3_TW = 64, R3_CIN = 64, R3_PW = R3_TW + 2;
constexpr int R3_WROW = 9 * R3_CIN + 16;  // LDS bytes per weight row: 576 + 16 (rows 148 dwords apart: conflict-free)
constexpr int R3_TN = 32;  // output channels per workgroup (config 1: 5.15 us; 64 channels 5.6, 16 channels 5.5)

template <int OUT, int TN = R3_TN>
__global__ __launch_bounds__(256) void conv3x3_row_kernel(const ConvArgs a) {
  constexpr int NB = TN / 16;
  __shared__ __attribute__((aligned(16))) uint8_t patch[3 * R3_PW * R3_CIN];  // [row][col][64 B], 16-byte slots swizzled
  __shared__ __attribute__((aligned(16))) uint8_t wt[TN * R3_WROW];           // [n][tap][64 B]
  __shared__ __attribute__((aligned(16))) float ep_scale[TN], ep_bias[TN], ep_osc[TN];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int per_xcd = gridDim.x >> 3;
  const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (t >= a.n_tiles * a.m_tiles) return;
  const int n0 = (t % a.n_tiles) * TN;
  const int m0 = (t / a.n_tiles) * R3_TW;
  const int hw = a.Ho * a.Wo;
  const int img = m0 / hw, oh = (m0 - img * hw) / a.Wo, ow0 = m0 - img * hw - oh * a.Wo;

  // one load phase: the patch (792 16-byte units) and the weight tile (2304 units), all in flight together
  constexpr int PU = 3 * R3_PW * 4, WU = TN * 36;
  uint4 pv[(PU + 255) / 256], wv[(WU + 255) / 256];
#pragma unroll
  for (int i = 0; i < (PU + 255) / 256; ++i) {
    const int u = tid + 256 * i;
    const int r = u / (R3_PW * 4), rem = u - r * (R3_PW * 4), col = rem >> 2, seg = rem & 3;
    const int ih = oh - 1 + r, iw = ow0 - 1 + col;
    const bool ok = u < PU && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
    pv[i] = ok ? *reinterpret_cast<const uint4*>(a.x + ((int64_t)(img * a.H + ih) * a.W + iw) * R3_CIN + seg * 16)
               : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < (WU + 255) / 256; ++i) {
    const int u = tid + 256 * i;
    const int n = u / 36, s = u - n * 36;
    wv[i] = u < WU && n0 + n < a.Cout
                ? *reinterpret_cast<const uint4*>(a.w + (int64_t)(n0 + n) * (9 * R3_CIN) + s * 16)
                : make_uint4(0, 0, 0, 0);
  }
  if (tid < TN) {
    const int n = n0 + tid;
    const bool nok = n < a.Cout;
    ep_scale[tid] = nok ? *a.a_scale * a.w_scale[n] : 1.0f;
    float bias = -0.0f;  // x + (-0) == x for every x: the fast epilogue adds it unconditionally
    if (a.bias != nullptr && nok)
      bias = a.bias_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.bias)[n])
                                      : static_cast<const float*>(a.bias)[n];
    ep_bias[tid] = bias;
    ep_osc[tid] = 1.0f;
  }
#pragma unroll
  for (int i = 0; i < (PU + 255) / 256; ++i) {
    const int u = tid + 256 * i;
    const int r = u / (R3_PW * 4), rem = u - r * (R3_PW * 4), col = rem >> 2, seg = rem & 3;
    if (u < PU)
      *reinterpret_cast<uint4*>(&patch[(r * R3_PW + col) * R3_CIN + ((seg ^ ((col >> 2) & 3)) << 4)]) = pv[i];
  }
#pragma unroll
  for (int i = 0; i < (WU + 255) / 256; ++i) {
    const int u = tid + 256 * i;
    const int n = u / 36, s = u - n * 36;
    if (u < WU) *reinterpret_cast<uint4*>(&wt[n * R3_WROW + s * 16]) = wv[i];
  }
  __syncthreads();

  v4i acc_i[NB][1];
  v4f acc_f[NB][1];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    acc_i[i][0] = v4i{0, 0, 0, 0};
    acc_f[i][0] = v4f{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int ky = 0; ky < 3; ++ky)
#pragma unroll
    for (int kx = 0; kx < 3; ++kx) {
      const int col = 16 * wave + r16 + kx;
      const v4i xf = *reinterpret_cast<const v4i*>(&patch[(ky * R3_PW + col) * R3_CIN + ((g ^ ((col >> 2) & 3)) << 4)]);
      const int tap = ky * 3 + kx;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const v4i wf = *reinterpret_cast<const v4i*>(&wt[(16 * i + r16) * R3_WROW + tap * R3_CIN + 16 * g]);
        acc_i[i][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, xf, acc_i[i][0], 0, 0, 0);
      }
    }
  conv_epilogue<KIND_INT8, OUT, 0, 1, NB>(a, acc_i, acc_f, m0 + 16 * wave, n0, 0, ep_scale, ep_bias, ep_osc);
}

// Whether conv3x3_row_kernel takes this launch (see there); the caller has established that the 128-row tiles would
// not fill the CUs.
template <int KIND>
static bool row3_ok(const ConvArgs& a, int lw) {
  return KIND == KIND_INT8 && lw == 16 && a.kh == 3 && a.kw == 3 && a.sh == 1 && a.sw == 1 && a.ph == 1 && a.pw == 1 &&
         a.dh == 1 && a.dw == 1 && a.Cin == R3_CIN && a.Wo % R3_TW == 0 && a.Cout % R3_TN == 0 && a.x_swz == nullptr &&
         a.a_scale_rows == nullptr && a.pool_out == nullptr && a.out_mode != OUT_E4M3 &&
         (int64_t)a.B * a.H * a.W * R3_CIN < (1LL << 31);
}

template <int KIND>
static int launch_conv(ConvArgs a, hipStream_t stream) {
  if (a.B < 0 || a.H < 0 || a.W < 0 || a.Cin <= 0 || a.Cout <= 0 || a.kh <= 0 || a.kw <= 0 || a.sh <= 0 ||
      a.sw <= 0 || a.dh <= 0 || a.dw <= 0 || a.ph < 0 || a.pw < 0)
    return FIM_ERR_INVALID;
  a.Ho = (a.H + 2 * a.ph - a.dh * (a.kh - 1) - 1) / a.sh + 1;
  a.Wo = (a.W + 2 * a.pw - a.dw * (a.kw - 1) - 1) / a.sw + 1;
  if (a.Ho <= 0 || a.Wo <= 0) return FIM_ERR_INVALID;
  const int64_t M = (int64_t)a.B * a.Ho * a.Wo;
  if (M == 0) return FIM_OK;
  if (M >= (1LL << 31) - 256) return FIM_ERR_UNSUPPORTED;
  if (a.pool_out != nullptr &&
      (KIND != KIND_INT8 || (a.Ho | a.Wo) & 1 || a.out_mode != OUT_BF16 || a.out_scale == nullptr ||
       a.residual != nullptr || a.a_scale_rows != nullptr))
    return FIM_ERR_UNSUPPORTED;
  a.M = (int)M;
  a.kchunks = (a.Cin + KC - 1) / KC;
  a.tps = 1;
  int lw = 1;
  const uintptr_t both = (uintptr_t)a.x | (uintptr_t)a.w;
  if (a.Cin % 16 == 0 && both % 16 == 0) lw = 16;
  // Cin 16, 32 or 64: the 64 x 64-tile kernels pack 128 / Cin taps into each 128-byte K step instead of padding every
  // step with zeros (MXFP8 needs whole 32-channel scale blocks)
  if (lw == 16 && a.kh * a.kw > 1 && (a.Cin == 64 || a.Cin == 32 || (a.Cin == 16 && KIND == KIND_INT8)))
    a.tps = KC / a.Cin;
  const int bn = (a.Cout > 64 && a.x_swz == nullptr) ? 128 : 64;
  a.n_tiles = (a.Cout + bn - 1) / bn;
  const int64_t m_tiles = (a.M + BM_MAIN - 1) / BM_MAIN;
  const int64_t tiles = m_tiles * a.n_tiles;
  if (tiles > (1LL << 30)) return FIM_ERR_UNSUPPORTED;
  a.m_tiles = (int)m_tiles;
  a.m_base = 0;
  const bool fast_ok = a.out_mode == OUT_BF16 ? conv_fast_ok<OUT_BF16>(a) : conv_fast_ok<OUT_INT8>(a);
  if (patch_ok(a, lw, fast_ok)) return launch_patch<KIND>(a, stream);
  if (const int ks = pw_ks(a, lw, fast_ok)) return launch_pw<KIND>(a, ks, stream);
  if (const int ks = res_ks(a, lw, fast_ok)) return launch_res<KIND>(a, ks, stream);
  if (const int wm = wide_wm(a, lw)) {
    a.n_tiles = (int)cdiv((int64_t)a.Cout, (8 / wm) * 64);
    a.m_tiles = (int)cdiv((int64_t)a.M, wm * 80);
    const dim3 grid((unsigned)(cdiv((int64_t)a.n_tiles * a.m_tiles, 8) * 8));
    if (wm == 2)
      launch_wide<KIND, 2>(a, grid, stream);
    else
      launch_wide<KIND, 4>(a, grid, stream);
    return launch_status();
  }
  // Workgroups stay resident 2 per CU, so tiles run in rounds of 2 x CUs. When the last round would be less than half
  // full (e.g. config 2: 632 tiles on 512 slots), it would still take a full tile time: the whole M tiles that fill
  // complete rounds run as one launch and the remaining rows as a second launch of 64 x 64 tiles (4x as many, each
  // about a quarter of the work), which fills the last round instead.
  if (a.x_swz == nullptr && a.pool_out == nullptr) {
    // fewer 128-row tiles than CUs: 64 x 64 tiles instead, so the launch reaches every CU (e.g. config 1: 128 tiles
    // of 128 x 64 -> 256 of 64 x 64)
    if (tiles < device_cus()) {
      if (row3_ok<KIND>(a, lw)) {
        ConvArgs t = a;
        t.n_tiles = a.Cout / R3_TN;
        t.m_tiles = a.M / R3_TW;
        const dim3 grid((unsigned)(cdiv((int64_t)t.m_tiles * t.n_tiles, 8) * 8));
        if (a.out_mode == OUT_BF16)
          conv3x3_row_kernel<OUT_BF16><<<grid, dim3(256), 0, stream>>>(t);
        else
          conv3x3_row_kernel<OUT_INT8><<<grid, dim3(256), 0, stream>>>(t);
        return launch_status();
      }
      ConvArgs t = a;
      t.n_tiles = (a.Cout + 63) / 64;
      t.m_tiles = (int)cdiv(a.M, 64);
      launch_tail<KIND>(t, lw, dim3((unsigned)(cdiv((int64_t)t.m_tiles * t.n_tiles, 8) * 8)), stream);
      return launch_status();
    }
    const int64_t slots = 2LL * device_cus();
    const int64_t full = tiles / slots, rem = tiles - full * slots;
    const int64_t mt_main = full * slots / a.n_tiles;
    if (full > 0 && rem > 0 && rem * 2 < slots && mt_main > 0 && mt_main < m_tiles) {
      ConvArgs t = a;
      a.m_tiles = (int)mt_main;
      const dim3 g1((unsigned)(cdiv(mt_main * a.n_tiles, 8) * 8));
      if (bn == 128)
        launch_xs<KIND, 128>(a, lw, g1, stream);
      else
        launch_xs<KIND, 64>(a, lw, g1, stream);
      const int status = launch_status();
      if (status != FIM_OK) return status;
      t.m_base = (int)(mt_main * BM_MAIN);
      t.n_tiles = (a.Cout + 63) / 64;
      t.m_tiles = (int)cdiv(a.M - t.m_base, 64);
      launch_tail<KIND>(t, lw, dim3((unsigned)(cdiv((int64_t)t.m_tiles * t.n_tiles, 8) * 8)), stream);
      return launch_status();
    }
  }
  dim3 grid((unsigned)(cdiv(tiles, 8) * 8));  // a multiple of the 8 XCDs: the kernel maps pids to tiles per XCD
  if (bn == 128)
    launch_xs<KIND, 128>(a, lw, grid, stream);
  else
    launch_xs<KIND, 64>(a, lw, grid, stream);
  return launch_status();
}

static void fill_geometry(ConvArgs& a, int64_t B, int64_t H, int64_t W, int64_t Cin, int64_t Cout, int kh, int kw,
                          int sh, int sw, int ph, int pw, int dh, int dw) {
  a.B = (int)B; a.H = (int)H; a.W = (int)W; a.Cin = (int)Cin; a.Cout = (int)Cout;
  a.kh = kh; a.kw = kw; a.sh = sh; a.sw = sw; a.ph = ph; a.pw = pw; a.dh = dh; a.dw = dw;
}

static void fill_epilogue(ConvArgs& a, const void* bias, int bias_dtype, const void* residual, int res_dtype,
                          int64_t res_channels, const int64_t* res_strides, int relu, int gelu, void* out,
                          int relu_before_residual = 0) {
  a.bias = bias; a.bias_dtype = bias_dtype;
  a.residual = residual; a.res_dtype = res_dtype; a.res_channels = res_channels;
  if (residual != nullptr && res_strides != nullptr) {
    a.rs_b = res_strides[0]; a.rs_h = res_strides[1]; a.rs_w = res_strides[2]; a.rs_c = res_strides[3];
  } else {
    a.rs_b = a.rs_h = a.rs_w = a.rs_c = 0;
  }
  // conv semantics (ops/conv.py:193-203): ReLU before the BF16 rounding without a residual, after the residual add
  // with one; linear semantics (ops/gemm.py:91-97, relu_before_residual): always before, the residual added after
  a.relu_pre = relu && (residual == nullptr || relu_before_residual);
  a.relu_post = relu && residual != nullptr && !relu_before_residual;
  a.gelu = gelu; a.out = out; a.out_ld = a.Cout;
}

static bool dims_fit(int64_t B, int64_t H, int64_t W, int64_t Cin, int64_t Cout) {
  const int64_t lim = 2147483647LL;
  return B < lim && H < lim && W < lim && Cin < lim && Cout < lim && B * H * W < lim * 64;
}

// 2x2 / stride-2 max pool of BF16 [B, Ho, Wo, C] then INT8 quantize: one lane per 4 channels of a pooled pixel.
__global__ __launch_bounds__(256) void pool2x2_quantize_kernel(const uint16_t* __restrict__ in, int64_t B, int64_t Ho,
                                                               int64_t Wo, int64_t C, const float* scale_ptr,
                                                               int8_t* __restrict__ out) {
  const int64_t cq = (C + 3) >> 2;
  const int64_t ho2 = Ho >> 1, wo2 = Wo >> 1;
  const int64_t total = B * ho2 * wo2 * cq;
  const float scale = *scale_ptr;
  const float inv = __fdiv_rn(1.0f, scale);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c0 = (i % cq) * 4;
    const int64_t p = i / cq;
    const int64_t x2 = p % wo2, q = p / wo2;
    const int64_t y2 = q % ho2, img = q / ho2;
    const uint16_t* base = in + ((img * Ho + 2 * y2) * Wo + 2 * x2) * C;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (c0 + v >= C) break;
      const uint16_t* s = base + c0 + v;
      const float m = fmaxf(fmaxf(bf16_to_f32(s[0]), bf16_to_f32(s[C])),
                            fmaxf(bf16_to_f32(s[Wo * C]), bf16_to_f32(s[Wo * C + C])));
      out[p * C + c0 + v] = quantize_int8_fast(m, scale, inv);
    }
  }
}

static int launch_pool2x2_quantize(const uint16_t* in, int64_t B, int64_t Ho, int64_t Wo, int64_t C,
                                   const float* scale, int8_t* out, hipStream_t stream) {
  const int64_t total = B * (Ho / 2) * (Wo / 2) * ((C + 3) / 4);
  if (total == 0) return FIM_OK;
  const int64_t blocks = std::min<int64_t>(cdiv(total, 256), 65536);
  pool2x2_quantize_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(in, B, Ho, Wo, C, scale, out);
  return launch_status();
}

}  // namespace fim

using namespace fim;

extern "C" {

int fim_int8_conv2d(const int8_t* x, int64_t B, int64_t H, int64_t W, int64_t Cin, const int8_t* weight, int64_t Cout,
                    const float* a_scale, const float* w_scale, const void* bias, int bias_dtype, int kh, int kw,
                    int sh, int sw, int ph, int pw, int dh, int dw, int relu, int gelu, const void* residual,
                    int res_dtype, int64_t res_channels, const int64_t* res_strides, const float* out_scale,
                    void* out, hipStream_t stream) {
  if (x == nullptr || weight == nullptr || a_scale == nullptr || w_scale == nullptr || out == nullptr)
    return FIM_ERR_INVALID;
  if (!dims_fit(B, H, W, Cin, Cout)) return FIM_ERR_UNSUPPORTED;
  ConvArgs a = {};
  a.x = reinterpret_cast<const uint8_t*>(x);
  a.w = reinterpret_cast<const uint8_t*>(weight);
  a.a_scale = a_scale;
  a.w_scale = w_scale;
  fill_geometry(a, B, H, W, Cin, Cout, kh, kw, sh, sw, ph, pw, dh, dw);
  fill_epilogue(a, bias, bias_dtype, residual, res_dtype, res_channels, res_strides, relu, gelu, out);
  a.out_scale = out_scale;
  a.out_mode = out_scale != nullptr ? OUT_INT8 : OUT_BF16;
  return launch_conv<KIND_INT8>(a, stream);
}

int fim_mxfp8_conv2d(const uint8_t* x, int64_t B, int64_t H, int64_t W, int64_t Cin, const int8_t* channel_exponent,
                     const uint8_t* weight, int64_t Cout, const int8_t* weight_exponent, const void* bias,
                     int bias_dtype, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, int relu, int gelu,
                     const void* residual, int res_dtype, int64_t res_channels, const int64_t* res_strides,
                     const int8_t* out_exponent, void* out, hipStream_t stream) {
  if (x == nullptr || channel_exponent == nullptr || weight == nullptr || weight_exponent == nullptr ||
      out == nullptr)
    return FIM_ERR_INVALID;
  if (Cin % 32 != 0) return FIM_ERR_UNSUPPORTED;
  if (out_exponent != nullptr && Cout % 32 != 0) return FIM_ERR_UNSUPPORTED;
  if (!dims_fit(B, H, W, Cin, Cout)) return FIM_ERR_UNSUPPORTED;
  ConvArgs a = {};
  a.x = x;
  a.w = weight;
  a.x_expo = channel_exponent;
  a.w_expo = weight_exponent;
  fill_geometry(a, B, H, W, Cin, Cout, kh, kw, sh, sw, ph, pw, dh, dw);
  fill_epilogue(a, bias, bias_dtype, residual, res_dtype, res_channels, res_strides, relu, gelu, out);
  a.out_expo = out_exponent;
  a.out_mode = out_exponent != nullptr ? OUT_E4M3 : OUT_BF16;
  return launch_conv<KIND_MX>(a, stream);
}

// int8_conv2d then MaxPool2d(2) quantized for the next conv (ops/conv.py:209-222): out BF16 [B, Ho, Wo, Cout] as
// fim_int8_conv2d writes it, pooled int8 [B, Ho/2, Wo/2, Cout] = quantize_int8(max_pool2d(out, 2), out_scale). Even
// Ho and Wo: from the conv's epilogue (pool-ordered rows); odd: a separate pool pass over out (a trailing odd row /
// column dropped, as F.max_pool2d does).
int fim_int8_conv2d_maxpool(const int8_t* x, int64_t B, int64_t H, int64_t W, int64_t Cin, const int8_t* weight,
                            int64_t Cout, const float* a_scale, const float* w_scale, const void* bias,
                            int bias_dtype, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, int relu,
                            const float* out_scale, void* out, int8_t* pooled, hipStream_t stream) {
  if (x == nullptr || weight == nullptr || a_scale == nullptr || w_scale == nullptr || out == nullptr ||
      out_scale == nullptr || pooled == nullptr)
    return FIM_ERR_INVALID;
  if (!dims_fit(B, H, W, Cin, Cout)) return FIM_ERR_UNSUPPORTED;
  if (kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 || dh <= 0 || dw <= 0 || ph < 0 || pw < 0) return FIM_ERR_INVALID;
  const int64_t Ho = (H + 2 * ph - (int64_t)dh * (kh - 1) - 1) / sh + 1;
  const int64_t Wo = (W + 2 * pw - (int64_t)dw * (kw - 1) - 1) / sw + 1;
  ConvArgs a = {};
  a.x = reinterpret_cast<const uint8_t*>(x);
  a.w = reinterpret_cast<const uint8_t*>(weight);
  a.a_scale = a_scale;
  a.w_scale = w_scale;
  fill_geometry(a, B, H, W, Cin, Cout, kh, kw, sh, sw, ph, pw, dh, dw);
  fill_epilogue(a, bias, bias_dtype, nullptr, 0, 0, nullptr, relu, 0, out);
  a.out_scale = out_scale;
  a.out_mode = OUT_BF16;
  if (Ho > 0 && Wo > 0 && Ho % 2 == 0 && Wo % 2 == 0) {
    a.pool_out = pooled;
    return launch_conv<KIND_INT8>(a, stream);
  }
  const int rc = launch_conv<KIND_INT8>(a, stream);
  if (rc != FIM_OK) return rc;
  return launch_pool2x2_quantize(static_cast<const uint16_t*>(out), B, Ho, Wo, Cout, out_scale, pooled, stream);
}

// INT8 GEMM [M, K] x [N, K]^T with int8_linear's epilogue (ops/gemm.py:78-98): a 1x1 conv over a 1 x M "image".
// a_scale_rows (may be null) holds per-row activation scales [M] in place of the per-tensor a_scale; ReLU comes
// before the BF16 rounding and the residual ([M, res_channels], row stride res_row_stride) is added after it.
int fim_int8_linear(const int8_t* a, int64_t M, int64_t K, const int8_t* weight, int64_t N, const float* a_scale,
                    const float* a_scale_rows, const float* w_scale, const void* bias, int bias_dtype, int relu, int gelu,
                    const void* residual, int res_dtype, int64_t res_channels, int64_t res_row_stride,
                    const float* out_scale, void* out, hipStream_t stream) {
  if (a == nullptr || weight == nullptr || (a_scale == nullptr && a_scale_rows == nullptr) || w_scale == nullptr ||
      out == nullptr)
    return FIM_ERR_INVALID;
  if (!dims_fit(1, 1, M, K, N)) return FIM_ERR_UNSUPPORTED;
  ConvArgs c = {};
  c.x = reinterpret_cast<const uint8_t*>(a);
  c.w = reinterpret_cast<const uint8_t*>(weight);
  c.a_scale = a_scale != nullptr ? a_scale : a_scale_rows;
  c.a_scale_rows = a_scale_rows;
  c.w_scale = w_scale;
  fill_geometry(c, 1, 1, M, K, N, 1, 1, 1, 1, 0, 0, 1, 1);
  const int64_t strides[4] = {0, 0, res_row_stride, 1};
  fill_epilogue(c, bias, bias_dtype, residual, res_dtype, res_channels, strides, relu, gelu, out, 1);
  c.out_scale = out_scale;
  c.out_mode = out_scale != nullptr ? OUT_INT8 : OUT_BF16;
  return launch_conv<KIND_INT8>(c, stream);
}

// int8_linear's BF16 result statically quantized again for the next INT8 consumer, written into rows out_row_stride
// bytes apart (e.g. one half of a concatenation buffer): ops/gemm.py:104-116.
int fim_int8_linear_quantize(const int8_t* a, int64_t M, int64_t K, const int8_t* weight, int64_t N,
                             const float* a_scale, const float* a_scale_rows, const float* w_scale, const void* bias,
                             int bias_dtype, const float* out_scale, int8_t* out, int64_t out_row_stride,
                             hipStream_t stream) {
  if (a == nullptr || weight == nullptr || (a_scale == nullptr && a_scale_rows == nullptr) || w_scale == nullptr ||
      out_scale == nullptr || out == nullptr)
    return FIM_ERR_INVALID;
  if (out_row_stride < N) return FIM_ERR_INVALID;
  if (!dims_fit(1, 1, M, K, N) || out_row_stride > 2147483647LL) return FIM_ERR_UNSUPPORTED;
  ConvArgs c = {};
  c.x = reinterpret_cast<const uint8_t*>(a);
  c.w = reinterpret_cast<const uint8_t*>(weight);
  c.a_scale = a_scale != nullptr ? a_scale : a_scale_rows;
  c.a_scale_rows = a_scale_rows;
  c.w_scale = w_scale;
  fill_geometry(c, 1, 1, M, K, N, 1, 1, 1, 1, 0, 0, 1, 1);
  fill_epilogue(c, bias, bias_dtype, nullptr, 0, 0, nullptr, 0, 0, out, 1);
  c.out_ld = out_row_stride;
  c.out_scale = out_scale;
  c.out_mode = OUT_INT8;
  return launch_conv<KIND_INT8>(c, stream);
}

// Block-scaled MXFP8 GEMM with per-(row, 32) scales on both operands (ops/gemm.py:40-49, F.scaled_mm's MXFP8 mode):
// a [M, K] E4M3 with its E8M0 scales in the 128x4 swizzled layout (a_scale_swizzled), weight [N, K] E4M3 with int8
// exponents [N, K/32]; out BF16 [M, N] = a @ weight^T (+ bias).
int fim_mxfp8_scaled_mm(const uint8_t* a, int64_t M, int64_t K, const uint8_t* a_scale_swizzled,
                        const uint8_t* weight, int64_t N, const int8_t* weight_exponent, int weight_scale_e8m0,
                        const void* bias, int bias_dtype, void* out, hipStream_t stream) {
  if (a == nullptr || a_scale_swizzled == nullptr || weight == nullptr || weight_exponent == nullptr || out == nullptr)
    return FIM_ERR_INVALID;
  if (K % 32 != 0) return FIM_ERR_UNSUPPORTED;
  if (!dims_fit(1, 1, M, K, N)) return FIM_ERR_UNSUPPORTED;
  ConvArgs c = {};
  c.x = a;
  c.w = weight;
  c.x_expo = weight_exponent;  // unused with row scales; any valid pointer
  c.x_swz = a_scale_swizzled;
  c.x_swz_tiles_k = (int)(((K / 32) + 3) / 4);
  c.w_expo = weight_exponent;
  c.w_expo_e8m0 = weight_scale_e8m0 != 0;
  fill_geometry(c, 1, 1, M, K, N, 1, 1, 1, 1, 0, 0, 1, 1);
  fill_epilogue(c, bias, bias_dtype, nullptr, 0, 0, nullptr, 0, 0, out);
  c.out_mode = OUT_BF16;
  return launch_conv<KIND_MX>(c, stream);
}

}  // extern "C"

// ----- im2col gather (byte tensors) ----------------------------------------------------------------------------

namespace fim {

// [B, H, W, C] bytes -> [B*Ho*Wo, T*C] in (ky, kx, c) order, zero padding (ops/conv.py:144-165). One lane per 16
// bytes of a (pixel, tap) segment when C % 16 == 0, else per byte.
template <int VEC>
__global__ __launch_bounds__(256) void im2col_kernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ out, int B,
                                                     int H, int W, int C, int Ho, int Wo, int kh, int kw, int sh,
                                                     int sw, int ph, int pw, int dh, int dw) {
  const int64_t segs = C / VEC;
  const int64_t per_row = (int64_t)kh * kw * segs;
  const int64_t total = (int64_t)B * Ho * Wo * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / per_row;
    const int64_t rest = i - m * per_row;
    const int tap = (int)(rest / segs);
    const int sg = (int)(rest - (int64_t)tap * segs);
    const int ow = (int)(m % Wo);
    const int64_t q = m / Wo;
    const int oh = (int)(q % Ho);
    const int b = (int)(q / Ho);
    const int ky = tap / kw, kx = tap - ky * kw;
    const int ih = oh * sh - ph + ky * dh, iw = ow * sw - pw + kx * dw;
    const bool ok = ih >= 0 && ih < H && iw >= 0 && iw < W;
    const uint8_t* src = x + (((int64_t)b * H + ih) * W + iw) * C + (int64_t)sg * VEC;
    uint8_t* dst = out + i * VEC;
    if (VEC == 16) {
      *reinterpret_cast<uint4*>(dst) = ok ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
    } else {
      *dst = ok ? *src : (uint8_t)0;
    }
  }
}

}  // namespace fim

extern "C" int fim_im2col_gather(const uint8_t* x, int64_t B, int64_t H, int64_t W, int64_t C, int kh, int kw, int sh,
                                 int sw, int ph, int pw, int dh, int dw, uint8_t* out, hipStream_t stream) {
  if (x == nullptr || out == nullptr || B < 0 || H < 0 || W < 0 || C <= 0 || kh <= 0 || kw <= 0 || sh <= 0 ||
      sw <= 0 || dh <= 0 || dw <= 0 || ph < 0 || pw < 0)
    return FIM_ERR_INVALID;
  if (!dims_fit(B, H, W, C, 1)) return FIM_ERR_UNSUPPORTED;
  const int Ho = (int)((H + 2 * ph - dh * (kh - 1) - 1) / sh + 1), Wo = (int)((W + 2 * pw - dw * (kw - 1) - 1) / sw + 1);
  if (Ho <= 0 || Wo <= 0) return FIM_ERR_INVALID;
  const bool vec = C % 16 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)out % 16) == 0;
  const int64_t elems = B * Ho * Wo * (int64_t)kh * kw * (vec ? C / 16 : C);
  if (elems == 0) return FIM_OK;
  int64_t blocks = cdiv(elems, 256);
  if (blocks > 65536) blocks = 65536;
  if (vec)
    im2col_kernel<16><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(x, out, (int)B, (int)H, (int)W, (int)C, Ho, Wo,
                                                                          kh, kw, sh, sw, ph, pw, dh, dw);
  else
    im2col_kernel<1><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(x, out, (int)B, (int)H, (int)W, (int)C, Ho, Wo,
                                                                         kh, kw, sh, sw, ph, pw, dh, dw);
  return launch_status();
}
