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
#include "common.h"

namespace fim {

enum { KIND_INT8 = 0, KIND_MX = 1 };
enum { OUT_BF16 = 0, OUT_INT8 = 1, OUT_E4M3 = 2 };

struct ConvArgs {
  const uint8_t* x;        // [B, H, W, Cin] int8 / e4m3
  const uint8_t* w;        // [Cout, T*Cin]
  const int8_t* x_expo;    // MX: [Cin / 32]
  const int8_t* w_expo;    // MX: [Cout, T*Cin / 32]
  const float* a_scale;    // INT8: scalar
  const float* w_scale;    // INT8: [Cout]
  const void* bias;        // [Cout] or null
  int bias_dtype;          // FIM_F32 / FIM_BF16
  const void* residual;    // [B, Ho, Wo, res_channels] with strides, or null
  int res_dtype;
  int64_t res_channels, rs_b, rs_h, rs_w, rs_c;
  const float* out_scale;  // OUT_INT8
  const int8_t* out_expo;  // OUT_E4M3: [Cout / 32]
  void* out;               // [B, Ho, Wo, Cout]
  int out_mode, relu, gelu;
  int B, H, W, Cin, Ho, Wo, Cout;
  int kh, kw, sh, sw, ph, pw, dh, dw;
  int64_t M;
  int kchunks;             // ceil(Cin / 128)
  int n_tiles;
};

constexpr int BM = 128;
constexpr int KC = 128;          // bytes of K per step
constexpr int LDS_PITCH = KC + 16;  // row pitch in LDS: 16 rows of a fragment read hit distinct banks

__device__ __forceinline__ float gelu_erf(float x) { return x * 0.5f * (1.0f + erff(x * 0.70710678118654752440f)); }

// 16 bytes of one row segment, channel-masked. LW = widest load the layout allows (16: Cin % 16 == 0; 4; 1).
template <int LW>
__device__ __forceinline__ uint4 load_seg(const uint8_t* p, bool row_ok, int cvalid) {
  uint4 v = make_uint4(0, 0, 0, 0);
  if (!row_ok || cvalid <= 0) return v;
  if (LW == 16) {
    v = *reinterpret_cast<const uint4*>(p);
  } else if (LW == 4) {
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

template <int KIND, int BN, int LW>
__global__ __launch_bounds__(256, 2) void conv_igemm_kernel(const ConvArgs a) {
  constexpr int NT = BN / 32;            // 16-column blocks per wavefront
  constexpr int MT = 4;                  // 16-row blocks per wavefront (64 rows)
  constexpr int A_PASSES = BM / 32;      // 256 lanes x 16 B cover 32 rows x 128 B per pass
  constexpr int B_PASSES = BN / 32;
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][BM * LDS_PITCH];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][BN * LDS_PITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int pid = blockIdx.x;
  const int n_tile = pid % a.n_tiles;
  const int64_t m0 = (int64_t)(pid / a.n_tiles) * BM;
  const int n0 = n_tile * BN;

  const int seg = tid & 7;   // 16-byte segment of the 128-byte chunk
  const int rsub = tid >> 3; // row within a 32-row pass
  const int T = a.kh * a.kw;
  const int64_t wrow = (int64_t)T * a.Cin;

  // per-lane gather geometry of its A rows
  int a_img[A_PASSES], a_h[A_PASSES], a_w[A_PASSES];
  bool a_ok[A_PASSES];
#pragma unroll
  for (int j = 0; j < A_PASSES; ++j) {
    int64_t m = m0 + rsub + 32 * j;
    a_ok[j] = m < a.M;
    int64_t mm = a_ok[j] ? m : 0;
    int ow = (int)(mm % a.Wo);
    int64_t t = mm / a.Wo;
    int oh = (int)(t % a.Ho);
    int b = (int)(t / a.Ho);
    a_img[j] = b;
    a_h[j] = oh * a.sh - a.ph;
    a_w[j] = ow * a.sw - a.pw;
  }

  const int nk = T * a.kchunks;
  uint4 ra[A_PASSES], rb[B_PASSES];

  auto gload = [&](int kt) {
    const int tap = kt / a.kchunks;
    const int c0 = (kt - tap * a.kchunks) * KC;
    const int ky = tap / a.kw, kx = tap - ky * a.kw;
    const int cseg = c0 + seg * 16;
    const int cvalid = a.Cin - cseg;
#pragma unroll
    for (int j = 0; j < A_PASSES; ++j) {
      int ih = a_h[j] + ky * a.dh, iw = a_w[j] + kx * a.dw;
      bool ok = a_ok[j] && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
      const uint8_t* p = a.x + ((((int64_t)a_img[j] * a.H + (ok ? ih : 0)) * a.W + (ok ? iw : 0)) * a.Cin + cseg);
      ra[j] = load_seg<LW>(p, ok, cvalid);
    }
#pragma unroll
    for (int j = 0; j < B_PASSES; ++j) {
      int n = n0 + rsub + 32 * j;
      bool ok = n < a.Cout;
      const uint8_t* p = a.w + ((int64_t)(ok ? n : 0) * wrow + (int64_t)tap * a.Cin + cseg);
      rb[j] = load_seg<LW>(p, ok, cvalid);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < A_PASSES; ++j)
      *reinterpret_cast<uint4*>(&lds_a[buf][(rsub + 32 * j) * LDS_PITCH + seg * 16]) = ra[j];
#pragma unroll
    for (int j = 0; j < B_PASSES; ++j)
      *reinterpret_cast<uint4*>(&lds_b[buf][(rsub + 32 * j) * LDS_PITCH + seg * 16]) = rb[j];
  };

  // accumulators
  v4i acc_i[MT][NT];
  v4f acc_f[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      acc_i[i][j] = v4i{0, 0, 0, 0};
      acc_f[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    }

  const int frag_row = lane & 15;
  const int frag_off = (lane >> 4) * 16;  // this lane's K bytes: [frag_off, +16) and [64 + frag_off, +16)
  const int wexp_stride = (int)(wrow >> 5);

  gload(0);
  sstore(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);

    int sa = 127, sb[NT];
    if (KIND == KIND_MX) {
      const int tap = kt / a.kchunks;
      const int c0 = (kt - tap * a.kchunks) * KC;
      const int blk = (c0 >> 5) + (lane >> 4);
      const bool bok = blk < (a.Cin >> 5);
      sa = bok ? (int)a.x_expo[blk] + 127 : 127;
      const int wblk = tap * (a.Cin >> 5) + blk;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        int n = n0 + wn * (BN / 2) + j * 16 + (lane & 15);
        sb[j] = (bok && n < a.Cout) ? (int)a.w_expo[(int64_t)n * wexp_stride + wblk] + 127 : 127;
      }
    }

    v8i bf[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const uint8_t* p = &lds_b[buf][(wn * (BN / 2) + j * 16 + frag_row) * LDS_PITCH + frag_off];
      v4i lo = *reinterpret_cast<const v4i*>(p);
      v4i hi = *reinterpret_cast<const v4i*>(p + 64);
      bf[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const uint8_t* p = &lds_a[buf][(wm * 64 + i * 16 + frag_row) * LDS_PITCH + frag_off];
      v4i lo = *reinterpret_cast<const v4i*>(p);
      v4i hi = *reinterpret_cast<const v4i*>(p + 64);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (KIND == KIND_INT8) {
          v4i blo = v4i{bf[j][0], bf[j][1], bf[j][2], bf[j][3]};
          v4i bhi = v4i{bf[j][4], bf[j][5], bf[j][6], bf[j][7]};
          acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(lo, blo, acc_i[i][j], 0, 0, 0);
          acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(hi, bhi, acc_i[i][j], 0, 0, 0);
        } else {
          v8i af = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          acc_f[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af, bf[j], acc_f[i][j], 0, 0, 0, sa, 0,
                                                                         sb[j]);
        }
      }
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  // ----- epilogue -----
  const float a_scale = KIND == KIND_INT8 ? *a.a_scale : 1.0f;
  const float out_scale = a.out_mode == OUT_INT8 ? *a.out_scale : 1.0f;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int n = n0 + wn * (BN / 2) + j * 16 + (lane & 15);
    if (n >= a.Cout) continue;
    float cscale = 1.0f;
    if (KIND == KIND_INT8) cscale = a_scale * a.w_scale[n];
    float bias = 0.0f;
    const bool has_bias = a.bias != nullptr;
    if (has_bias)
      bias = a.bias_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.bias)[n])
                                      : static_cast<const float*>(a.bias)[n];
    float oinv = 1.0f;
    if (a.out_mode == OUT_E4M3) oinv = exp2_int(-(int)a.out_expo[n >> 5]);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + v;
        if (m >= a.M) continue;
        float y;
        if (KIND == KIND_INT8) {
          y = __fmul_rn((float)acc_i[i][j][v], cscale);
        } else {
          y = acc_f[i][j][v];
        }
        if (has_bias) y = __fadd_rn(y, bias);
        const bool res = a.residual != nullptr;
        if (a.relu && !res) y = fmaxf(y, 0.0f);
        y = round_bf16(y);
        if (a.gelu) y = round_bf16(gelu_erf(y));
        if (res && n < a.res_channels) {
          int ow = (int)(m % a.Wo);
          int64_t t = m / a.Wo;
          int oh = (int)(t % a.Ho);
          int64_t b = t / a.Ho;
          int64_t off = b * a.rs_b + oh * a.rs_h + ow * a.rs_w + n * a.rs_c;
          float r = a.res_dtype == FIM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(a.residual)[off])
                                            : static_cast<const float*>(a.residual)[off];
          y = __fadd_rn(y, r);
          if (a.relu) y = fmaxf(y, 0.0f);
          y = round_bf16(y);
        } else if (res && a.relu) {
          y = fmaxf(y, 0.0f);
        }
        const int64_t o = m * a.Cout + n;
        if (a.out_mode == OUT_BF16) {
          static_cast<uint16_t*>(a.out)[o] = f32_to_bf16(y);
        } else if (a.out_mode == OUT_INT8) {
          static_cast<int8_t*>(a.out)[o] = quantize_int8_value(y, out_scale);
        } else {
          static_cast<uint8_t*>(a.out)[o] = e4m3(mx_scale_clamp(y, oinv));
        }
      }
    }
  }
}

template <int KIND, int BN>
static void launch_bn(const ConvArgs& a, int lw, dim3 grid, hipStream_t stream) {
  if (lw == 16)
    conv_igemm_kernel<KIND, BN, 16><<<grid, dim3(256), 0, stream>>>(a);
  else if (lw == 4)
    conv_igemm_kernel<KIND, BN, 4><<<grid, dim3(256), 0, stream>>>(a);
  else
    conv_igemm_kernel<KIND, BN, 1><<<grid, dim3(256), 0, stream>>>(a);
}

template <int KIND>
static int launch_conv(ConvArgs a, hipStream_t stream) {
  if (a.B < 0 || a.H < 0 || a.W < 0 || a.Cin <= 0 || a.Cout <= 0 || a.kh <= 0 || a.kw <= 0 || a.sh <= 0 ||
      a.sw <= 0 || a.dh <= 0 || a.dw <= 0 || a.ph < 0 || a.pw < 0)
    return FIM_ERR_INVALID;
  a.Ho = (a.H + 2 * a.ph - a.dh * (a.kh - 1) - 1) / a.sh + 1;
  a.Wo = (a.W + 2 * a.pw - a.dw * (a.kw - 1) - 1) / a.sw + 1;
  if (a.Ho <= 0 || a.Wo <= 0) return FIM_ERR_INVALID;
  a.M = (int64_t)a.B * a.Ho * a.Wo;
  if (a.M == 0) return FIM_OK;
  a.kchunks = (a.Cin + KC - 1) / KC;
  const int bn = a.Cout > 64 ? 128 : 64;
  a.n_tiles = (a.Cout + bn - 1) / bn;
  const int64_t m_tiles = (a.M + BM - 1) / BM;
  if (m_tiles * a.n_tiles > 2147483647LL) return FIM_ERR_UNSUPPORTED;
  int lw = 1;
  const uintptr_t both = (uintptr_t)a.x | (uintptr_t)a.w;
  if (a.Cin % 16 == 0 && both % 16 == 0)
    lw = 16;
  else if (a.Cin % 4 == 0 && both % 4 == 0)
    lw = 4;
  dim3 grid((unsigned)(m_tiles * a.n_tiles));
  if (bn == 128)
    launch_bn<KIND, 128>(a, lw, grid, stream);
  else
    launch_bn<KIND, 64>(a, lw, grid, stream);
  return launch_status();
}

static void fill_geometry(ConvArgs& a, int64_t B, int64_t H, int64_t W, int64_t Cin, int64_t Cout, int kh, int kw,
                          int sh, int sw, int ph, int pw, int dh, int dw) {
  a.B = (int)B; a.H = (int)H; a.W = (int)W; a.Cin = (int)Cin; a.Cout = (int)Cout;
  a.kh = kh; a.kw = kw; a.sh = sh; a.sw = sw; a.ph = ph; a.pw = pw; a.dh = dh; a.dw = dw;
}

static void fill_epilogue(ConvArgs& a, const void* bias, int bias_dtype, const void* residual, int res_dtype,
                          int64_t res_channels, const int64_t* res_strides, int relu, int gelu, void* out) {
  a.bias = bias; a.bias_dtype = bias_dtype;
  a.residual = residual; a.res_dtype = res_dtype; a.res_channels = res_channels;
  if (residual != nullptr && res_strides != nullptr) {
    a.rs_b = res_strides[0]; a.rs_h = res_strides[1]; a.rs_w = res_strides[2]; a.rs_c = res_strides[3];
  } else {
    a.rs_b = a.rs_h = a.rs_w = a.rs_c = 0;
  }
  a.relu = relu; a.gelu = gelu; a.out = out;
}

static bool dims_fit(int64_t B, int64_t H, int64_t W, int64_t Cin, int64_t Cout) {
  const int64_t lim = 2147483647LL;
  return B < lim && H < lim && W < lim && Cin < lim && Cout < lim && B * H * W < lim * 64;
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

}  // extern "C"
