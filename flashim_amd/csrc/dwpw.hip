// Depthwise 5x5 + bias + ReLU -> quantize -> pointwise GEMM + bias in one kernel, the fused refiner blocks of
// flashim/backends/triton/conv.py (ops flashim/ops/conv.py:93-138), for C = 128 input channels and a 128 x 128
// pointwise weight (the reference's fused shape):
//   MXFP8 (_dw5x5_relu_mx_pointwise_kernel, :310-420): relu(dwconv + bias) in FP32 -> dynamic per-(pixel, 32-channel)
//   MXFP8 -> block-scaled GEMM with the weight's E8M0 bytes (+ bias) -> BF16; bit for bit the two-launch composite
//   (depthwise producer, then fim_mxfp8_scaled_mm) with the same MFMA per 16 x 16 output block;
//   INT8 (_dw5x5_relu_int8_pointwise_kernel, :417-475): dwconv + bias rounded to BF16 -> static INT8 (ReLU folded into
//   the saturation) -> INT8 GEMM with per-channel weight scales (+ bias) -> BF16; bit for bit the composite
//   (depthwise producer, then fim_int8_linear): exact int32 sums and the same FP32 epilogue.
// The quantized activations never leave the CU.
//
// Persistent workgroups of 256 lanes (2 per CU by LDS) keep the pointwise weight in LDS and take tiles of 32 columns x
// 8 rows of one image, all 128 channels:
//   depthwise, per 32-channel slice: the 12 x 36-pixel input window (loaded into registers one slice ahead, with the
//   slice's depthwise weights) is staged channel-planar in LDS and the taps run on v_mfma_f32_4x4x4_16b_bf16 exactly
//   as in depthwise.hip (Toeplitz weight rows, 10 MFMAs per 16 channels x 4 x 4 outputs). MXFP8: the activated FP32
//   values go through LDS in two 4-row halves and a per-pixel pass (8 channels per lane, 4 lanes per pixel) quantizes
//   them into the workgroup's activation tile [256 pixels][128 B] (XOR-swizzled 16-byte slots, as the conv kernels'
//   stages) with the MX exponents beside it; INT8: each lane quantizes its own values and a 4 x 4 byte transpose across
//   lanes writes them to the tile as 32-bit words;
//   pointwise: wave w takes pixels [64 w, 64 w + 64) x 128 output channels in two 64-channel passes, weights as the
//   MFMA's A operand so each lane ends with 4 consecutive output channels of one pixel; the BF16 results are staged in
//   the wave's part of the activation tile and leave as whole 128-byte lines.
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
  const void* dw_b;         // FP32 or BF16 [128]
  int dw_b_bf16;
  const uint8_t* pw_w;      // E4M3 or INT8 [128, 128]
  const uint8_t* pw_e8m0;   // MXFP8: [128, 4] E8M0 bytes
  const float* act_scale;   // INT8: the static activation scale (one value)
  const float* pw_wscale;   // INT8: [128] per-output-channel weight scales
  const void* pw_b;         // [128] or null
  int pw_b_dtype;
  uint16_t* out;            // BF16 [B, H, W, 128]
  int B, H, W;
  int tiles_x, tiles_y;
  int ntiles;               // tiles_x * tiles_y * B
};

typedef __bf16 v4bf16 __attribute__((ext_vector_type(4)));

constexpr int DP_MX = 0, DP_INT8 = 1;

template <int KIND>
__global__ __launch_bounds__(256, 2) void dw_pw_kernel(const DwPwArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t sm[DP_STAGE];           // input window / FP32 output half
  __shared__ __attribute__((aligned(16))) uint8_t act[DP_PX * DP_C];       // quantized activations [px][128 B]
  __shared__ __attribute__((aligned(16))) uint8_t wts[DP_N * DP_C];        // pointwise weight [n][128 B]
  __shared__ int8_t aexp[DP_PX * 4];                                        // MX exponents [px][32-channel block]
  __shared__ float pb[DP_N];                                                // pointwise bias
  __shared__ uint8_t pe[DP_N * 4];                                          // MX weight E8M0 [n][block]
  __shared__ float pcs[DP_N];                                               // INT8: act_scale * w_scale[n]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Persistent, XCD-aware: workgroup p runs on XCD p % 8, and each XCD takes a contiguous run of tiles (column tiles
  // fastest), dealt round-robin to its workgroups, so the tiles in flight on one XCD are neighbours that share halo
  // rows through its L2.
  const int per_xcd = (a.ntiles + 7) >> 3;
  const int xcd = blockIdx.x & 7, wg_in_xcd = blockIdx.x >> 3, wgs_per_xcd = gridDim.x >> 3;
  const int t_end = min((xcd + 1) * per_xcd, a.ntiles);
  int tile = xcd * per_xcd + wg_in_xcd;
  if (tile >= t_end) return;

  // ---- the depthwise operands of one (tile, 32-channel slice), loaded into registers one slice ahead ------------
  // staging unit u (row r of the 12-row window, 4-column group q, channel octet o): 4 pixels x 8 channels, loaded
  // from the first in-image window row with buffer loads; pixels outside the image get an offset past the buffer's
  // range, which the hardware returns as zeros. Units past the 432 are loaded again (clamped) but not written.
  constexpr int UNITS = (DP_TH + 4) * 9 * 4, NU = (UNITS + 255) / 256;
  const int cg = wave & 1, rq = wave >> 1;  // 16-channel group of the slice; output row quad (rows 4 rq .. 4 rq + 3)
  const int bch = lane >> 2, r4 = lane & 3;
  uint4 pre[NU][4];
  uint32_t wpre[25];
  float bpre;
  // tile t -> (first column, first row, image), wave-uniform
  auto origin = [&](int t, int& x0, int& y0, int& b) {
    const int tx = t % a.tiles_x, rest = t / a.tiles_x;
    x0 = __builtin_amdgcn_readfirstlane(tx * DP_TW);
    y0 = __builtin_amdgcn_readfirstlane((rest % a.tiles_y) * DP_TH);
    b = __builtin_amdgcn_readfirstlane(rest / a.tiles_y);
  };
  auto issue = [&](int x0, int y0, int b, int s) {
    const int ybase = max(y0 - 2, 0);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.x + ((int64_t)b * a.H + ybase) * a.W * DP_C + s * DP_CS), (short)0, 0x7fffffff,
        0x00020000);
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      const int u = min(tid + 256 * j, UNITS - 1);
      const int o = u & 3, rr = u >> 2;
      const int r = rr / 9, q = rr - r * 9;
      const int iy = y0 - 2 + r;
      const bool row_ok = iy >= 0 && iy < a.H;
      // byte offsets below 2^31 (the host bounds 12 W C)
      const uint32_t row_off = (uint32_t)(((iy - ybase) * a.W + x0 - 2 + 4 * q) * DP_C + 8 * o) * 2u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int ix = x0 - 2 + 4 * q + k;
        const bool ok = row_ok && ix >= 0 && ix < a.W;
        const uint32_t off = ok ? row_off + (uint32_t)(k * DP_C * 2) : 0x80000000u;
        pre[j][k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
      }
    }
    const int ch = s * DP_CS + 16 * cg + bch;
#pragma unroll
    for (int k = 0; k < 25; ++k) wpre[k] = a.dw_w[k * DP_C + ch];
    bpre = a.dw_b_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(a.dw_b)[ch]) : static_cast<const float*>(a.dw_b)[ch];
  };
  int cx0, cy0, cb;
  origin(tile, cx0, cy0, cb);
  issue(cx0, cy0, cb, 0);  // in flight while the pointwise operands are staged

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
    if (KIND == DP_MX)
      *reinterpret_cast<uint32_t*>(&pe[4 * tid]) = reinterpret_cast<const uint32_t*>(a.pw_e8m0)[tid];
    else
      pcs[tid] = *a.act_scale * a.pw_wscale[tid];  // int8_linear's combined scale, one FP32 product
  }
  // INT8: the producer's static quantizer (depthwise5x5 with an INT8 output): BF16 rounding, then round(v / scale)
  // saturated to [0, 127] (the ReLU folded into the lower bound)
  const float qscale = KIND == DP_INT8 ? *a.act_scale : 1.0f;
  const float qinv = KIND == DP_INT8 ? __fdiv_rn(1.0f, qscale) : 1.0f;
  float* st = reinterpret_cast<float*>(sm);

  for (; tile < t_end; tile += wgs_per_xcd) {
    const int x0 = cx0, y0 = cy0, b = cb;
    const int rows = min(DP_TH, a.H - y0), cols = min(DP_TW, a.W - x0);
    // the next tile's origin (this tile's again after the last one: its loads are then issued but never used, which
    // keeps the prefetch unconditional, so no register copies wait on loads in flight)
    const int next = tile + wgs_per_xcd;
    int nx0 = x0, ny0 = y0, nb = b;
    if (next < t_end) origin(next, nx0, ny0, nb);

    // ---- depthwise, one 32-channel slice at a time ----------------------------------------------------------------
#pragma unroll 1
    for (int s = 0; s < DP_C / DP_CS; ++s) {
      __syncthreads();  // the previous slice's output pass (or the previous tile's pointwise) is done with sm / act
      // stage the prefetched window: each unit's 4 pixels x 8 channels transposed (v_perm) into 8 channel rows of 4
#pragma unroll
      for (int j = 0; j < NU; ++j) {
        const int u = tid + 256 * j;
        if (j < NU - 1 || u < UNITS) {
          const int o = u & 3, rr = u >> 2;
          const int r = rr / 9, q = rr - r * 9;
          const uint32_t P[4][4] = {{pre[j][0].x, pre[j][0].y, pre[j][0].z, pre[j][0].w},
                                    {pre[j][1].x, pre[j][1].y, pre[j][1].z, pre[j][1].w},
                                    {pre[j][2].x, pre[j][2].y, pre[j][2].z, pre[j][2].w},
                                    {pre[j][3].x, pre[j][3].y, pre[j][3].z, pre[j][3].w}};
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
      }
      // this lane's Toeplitz weight rows (segment 0: v shifted up by r4 BF16 elements, segment 1: u shifted down by
      // 3 - r4, with v = w[ky][0..3], u = w[ky][1..4] packed 16 bits apart)
      v4bf16 wa[5][2];
#pragma unroll
      for (int ky = 0; ky < 5; ++ky) {
        uint64_t w5[5];
#pragma unroll
        for (int kx = 0; kx < 5; ++kx) w5[kx] = wpre[ky * 5 + kx];
        const uint64_t v = w5[0] | (w5[1] << 16) | (w5[2] << 32) | (w5[3] << 48);
        const uint64_t u = w5[1] | (w5[2] << 16) | (w5[3] << 32) | (w5[4] << 48);
        wa[ky][0] = __builtin_bit_cast(v4bf16, v << (16 * r4));
        wa[ky][1] = __builtin_bit_cast(v4bf16, u >> (16 * (3 - r4)));
      }
      const float dbias = bpre;
      __syncthreads();  // window staged
      // the next window's loads fly during this slice's taps, output pass and (after the last slice) the pointwise
      // (issued before this barrier they measured slower: they then compete with the other waves' staging)
      {
        const bool last = s == DP_C / DP_CS - 1;
        issue(last ? nx0 : x0, last ? ny0 : y0, last ? nb : b, last ? 0 : s + 1);
      }

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
            acc[cq] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(wa[ky][sg], __builtin_bit_cast(v4bf16, raw), acc[cq],
                                                             0, 0, 0);
          }
      }
      if constexpr (KIND == DP_INT8) {
        // static quantization in registers; the codes go straight into the activation tile, one byte per value
        float v[32];
#pragma unroll
        for (int cq = 0; cq < 8; ++cq)
#pragma unroll
          for (int i = 0; i < 4; ++i) v[4 * cq + i] = acc[cq][i];
#pragma unroll
        for (int k = 0; k < 16; ++k) round_bf16x2(v[2 * k], v[2 * k + 1]);
        int qi[32];
        quantize_int8_fast_n<32, 0>(v, qscale, qinv, qi);
        // a lane holds one channel (bch) at 4 columns per column quad: a 4 x 4 byte transpose across the lanes of
        // channels 4 k .. 4 k + 3 (lanes 16 k + r4 + 4 m, m = bch & 3) leaves lane m with column 4 cq + m of those 4
        // channels, one 32-bit LDS write per column quad
        const int seg = 2 * s + cg;  // 16-byte slot of channels [32 s + 16 cg, + 16)
        const int m = bch & 3;
#pragma unroll
        for (int cq = 0; cq < 8; ++cq) {
          const uint32_t dq = __builtin_amdgcn_perm(__builtin_amdgcn_perm(qi[4 * cq + 3], qi[4 * cq + 2], 0x0c0c0400u),
                                                    __builtin_amdgcn_perm(qi[4 * cq + 1], qi[4 * cq], 0x0c0c0400u),
                                                    0x05040100u);  // bytes: columns 0..3
          const uint32_t t1 = (uint32_t)__shfl_xor((int)dq, 4);
          // m even: [own 0, partner 0, own 2, partner 2]; m odd: [partner 1, own 1, partner 3, own 3]
          const uint32_t d1 = (m & 1) ? __builtin_amdgcn_perm(dq, t1, 0x07030501u) : __builtin_amdgcn_perm(t1, dq, 0x06020400u);
          const uint32_t t2 = (uint32_t)__shfl_xor((int)d1, 8);
          // m < 2: [own 0, own 1, partner 0, partner 1]; m >= 2: [partner 2, partner 3, own 2, own 3]
          const uint32_t d2 = (m & 2) ? __builtin_amdgcn_perm(d1, t2, 0x07060302u) : __builtin_amdgcn_perm(t2, d1, 0x05040100u);
          const int p = (4 * rq + r4) * DP_TW + 4 * cq + m;
          *reinterpret_cast<uint32_t*>(&act[p * DP_C + ((seg ^ ((p >> 1) & 7)) << 4) + 4 * (bch >> 2)]) = d2;
        }
      } else {
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
            const float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
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
            const uint2 codes = make_uint2(pack_e4m3x4(q[0], q[1], q[2], q[3]), pack_e4m3x4(q[4], q[5], q[6], q[7]));
            if (part == 0) aexp[p * 4 + s] = (int8_t)ex;
            const int seg = 2 * s + (part >> 1);  // 16-byte slot of channels [32 s + 8 part, + 8)
            *reinterpret_cast<uint2*>(&act[p * DP_C + ((seg ^ ((p >> 1) & 7)) << 4) + 8 * (part & 1)]) = codes;
          }
        }
      }
    }
    __syncthreads();  // activation tile complete

    // ---- pointwise: wave w, pixels [64 w, 64 w + 64), output channels in two passes of 64 ------------------------
    const int g = lane >> 4, r16 = lane & 15;
    v8i xf[4];
    int sx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = 64 * wave + 16 * j + r16;
      const v4i lo = *reinterpret_cast<const v4i*>(&act[p * DP_C + ((g ^ ((p >> 1) & 7)) << 4)]);
      const v4i hi = *reinterpret_cast<const v4i*>(&act[p * DP_C + (((g + 4) ^ ((p >> 1) & 7)) << 4)]);
      xf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      sx[j] = KIND == DP_MX ? (int)aexp[p * 4 + g] + 127 : 0;  // lane group g scales K block g = channel slice g
    }
    __syncthreads();  // every wave holds its operands: act becomes the output staging area
    // each wave stages its 64 pixels x 64 channels of a pass in its own 8 KB of act (16-byte chunks XOR-swizzled by
    // row), then writes them back as whole 128-byte lines: 8 stores per pass, each 8 pixels x 128 B (scattered
    // 8-byte stores from the MFMA layout touch 16 lines per instruction and bound the epilogue)
    uint8_t* const stg = act + wave * 8192;
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
          if constexpr (KIND == DP_MX) {
            const v8i wf = __builtin_shufflevector(wl, wh, 0, 1, 2, 3, 4, 5, 6, 7);
            acc_f[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf, xf[j], v4f{0.f, 0.f, 0.f, 0.f}, 0,
                                                                           0, 0, (int)pe[n * 4 + g], 0, sx[j]);
          } else {  // the same 16-byte K slots from both operands: exact int32 sums in any K order
            const v4i xlo = __builtin_shufflevector(xf[j], xf[j], 0, 1, 2, 3);
            const v4i xhi = __builtin_shufflevector(xf[j], xf[j], 4, 5, 6, 7);
            v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl, xlo, v4i{0, 0, 0, 0}, 0, 0, 0);
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh, xhi, c, 0, 0, 0);
            acc_f[i][j] = v4f{(float)c[0], (float)c[1], (float)c[2], (float)c[3]};
          }
        }
      }
      // epilogue: + bias, BF16; lane (g, r16) holds channels 16 i + 4 g .. + 3 of pixel row 16 j + r16
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = 16 * j + r16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n0 = 64 * pass + 16 * i + 4 * g;
          float yv[4];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            yv[v] = __fadd_rn(KIND == DP_MX ? acc_f[i][j][v] : __fmul_rn(acc_f[i][j][v], pcs[n0 + v]), pb[n0 + v]);
          const int chunk = (2 * i + (g >> 1)) ^ (row & 7);
          *reinterpret_cast<uint2*>(&stg[row * 128 + chunk * 16 + 8 * (g & 1)]) =
              make_uint2(pack_bf16x2(yv[0], yv[1]), pack_bf16x2(yv[2], yv[3]));
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int row = 8 * k + (lane >> 3), c = lane & 7;
        const uint4 val = *reinterpret_cast<const uint4*>(&stg[row * 128 + ((c ^ (row & 7)) << 4)]);
        const int p = 64 * wave + row;
        const int py = p >> 5, pxx = p & 31;
        if (py < rows && pxx < cols)
          *reinterpret_cast<uint4*>(a.out + (((int64_t)b * a.H + y0 + py) * a.W + x0 + pxx) * DP_N + 64 * pass +
                                    8 * c) = val;
      }
    }
    cx0 = nx0;
    cy0 = ny0;
    cb = nb;
  }
}

}  // namespace fim

using namespace fim;

static int dwpw_launch(const DwPwArgs& a, int kind, int64_t C, int64_t N, hipStream_t stream) {
  if (a.x == nullptr || a.dw_w == nullptr || a.dw_b == nullptr || a.pw_w == nullptr || a.out == nullptr)
    return FIM_ERR_INVALID;
  if (a.B < 0 || a.H < 0 || a.W < 0) return FIM_ERR_INVALID;
  if (C != DP_C || N != DP_N) return FIM_ERR_UNSUPPORTED;
  if (((uintptr_t)a.x % 16) != 0 || ((uintptr_t)a.pw_w % 16) != 0 || ((uintptr_t)a.out % 16) != 0 ||
      ((uintptr_t)a.dw_w % 2) != 0)
    return FIM_ERR_UNSUPPORTED;
  if ((int64_t)a.B * a.H * a.W == 0) return FIM_OK;
  DwPwArgs t = a;
  t.tiles_x = (int)cdiv(a.W, DP_TW);
  t.tiles_y = (int)cdiv(a.H, DP_TH);
  const int64_t ntiles = (int64_t)t.tiles_x * t.tiles_y * a.B;
  if (ntiles > (1LL << 31) - 64) return FIM_ERR_UNSUPPORTED;  // tile indices (and their XCD runs) in int
  t.ntiles = (int)ntiles;
  if ((int64_t)(DP_TH + 4) * a.W * DP_C * 2 >= (1LL << 31)) return FIM_ERR_UNSUPPORTED;  // window byte offsets
  // persistent: two workgroups per CU (the LDS bound), a multiple of the 8 XCDs, no more than the tiles need
  const int64_t slots = (int64_t)device_cus() * 2 / 8 * 8;
  const dim3 grid((unsigned)min(slots, cdiv(ntiles, 8) * 8));
  if (kind == DP_MX)
    dw_pw_kernel<DP_MX><<<grid, dim3(256), 0, stream>>>(t);
  else
    dw_pw_kernel<DP_INT8><<<grid, dim3(256), 0, stream>>>(t);
  return launch_status();
}

static bool dwpw_dims_ok(int64_t B, int64_t H, int64_t W, int64_t C) {
  return B <= 2147483647LL && H <= 2147483647LL && W <= 2147483647LL && B * H * W * C < (1LL << 40);
}

extern "C" {

int fim_depthwise5x5_relu_pointwise_mxfp8(const uint16_t* x, int64_t B, int64_t H, int64_t W, int64_t C,
                                          const uint16_t* dw_weight, const void* dw_bias, int dw_bias_dtype,
                                          const uint8_t* pw_weight, int64_t N, const uint8_t* pw_scale_e8m0,
                                          const void* pw_bias, int pw_bias_dtype, uint16_t* out, hipStream_t stream) {
  if (pw_scale_e8m0 == nullptr || ((uintptr_t)pw_scale_e8m0 % 4) != 0) return FIM_ERR_INVALID;
  if (dw_bias_dtype != FIM_F32 && dw_bias_dtype != FIM_BF16) return FIM_ERR_INVALID;
  if (!dwpw_dims_ok(B, H, W, C)) return FIM_ERR_UNSUPPORTED;
  DwPwArgs a{x, dw_weight, dw_bias, dw_bias_dtype == FIM_BF16, pw_weight, pw_scale_e8m0, nullptr, nullptr, pw_bias, pw_bias_dtype, out,
             (int)B, (int)H, (int)W, 0, 0, 0};
  return dwpw_launch(a, DP_MX, C, N, stream);
}

int fim_depthwise5x5_relu_pointwise_int8(const uint16_t* x, int64_t B, int64_t H, int64_t W, int64_t C,
                                         const uint16_t* dw_weight, const void* dw_bias, int dw_bias_dtype,
                                         const float* act_scale, const int8_t* pw_weight, int64_t N,
                                         const float* pw_wscale, const void* pw_bias, int pw_bias_dtype, uint16_t* out,
                                         hipStream_t stream) {
  if (act_scale == nullptr || pw_wscale == nullptr) return FIM_ERR_INVALID;
  if (dw_bias_dtype != FIM_F32 && dw_bias_dtype != FIM_BF16) return FIM_ERR_INVALID;
  if (!dwpw_dims_ok(B, H, W, C)) return FIM_ERR_UNSUPPORTED;
  DwPwArgs a{x, dw_weight, dw_bias, dw_bias_dtype == FIM_BF16, reinterpret_cast<const uint8_t*>(pw_weight), nullptr, act_scale, pw_wscale,
             pw_bias, pw_bias_dtype, out, (int)B, (int)H, (int)W, 0, 0, 0};
  return dwpw_launch(a, DP_INT8, C, N, stream);
}

}  // extern "C"
