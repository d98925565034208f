// Activation / weight quantizers of the quantized conv path (all HBM-bound byte work):
//   fim_quantize_int8          static per-tensor INT8      flashim/ops/quantize.py:91-100, quant/tensor.py:148-151
//   fim_quantize_mxfp8         static block-32 MXFP8       flashim/ops/quantize.py:80-85, quant/tensor.py:97-121
//   fim_gelu_quantize_mxfp8 / _int8   GELU in the input dtype, then either   flashim/ops/quantize.py:63-74, 128-131
//   fim_quantize_mxfp8_dynamic per-(row, 32) MXFP8 (+ the 128x4 swizzled E8M0 scales)  quant/formats/mx.py:50-86
//   fim_quantize_int8_rows     per-row INT8 weights / tokens   quant/formats/int8.py:19-27, ops/quantize.py:148-157
//   fim_calibrate_block32      static exponents from an amax over rows  quant/formats/mx.py:41-47
//   fim_calibrate_block32_noalloc  the same without a caller workspace (file-scope device scratch; no allocation)
//
// Inputs are 4-D [B, H, W, C] with element strides, so both a packed NHWC tensor and the NHWC view of NCHW memory are
// read in place. Three read paths:
//   * channel-contiguous (sc == 1): each lane owns 8 consecutive channels of one pixel (one 16-byte BF16 load);
//   * width-contiguous (sw == 1, the NCHW view): a 64-pixel x 64-channel tile transposed through LDS, so both the
//     read (along W) and the write (along C) are coalesced;
//   * anything else: one element per lane.
#include <mutex>

#include "common.h"

namespace fim {

struct Geometry4 {
  int64_t B, H, W, C;
  int64_t sb, sh, sw, sc;
};

// ----- output element functions --------------------------------------------------------------------------------

// MODE_INT8: round(x * cs[c] / scale) (IEEE division); MODE_MX: clamp(x / 2^e[c/32], +-448) -> E4M3 (zero padding).
// gelu != 0 first applies GELU in the input's dtype (the gelu_quantize producers, flashim/ops/quantize.py:63-74,
// 128-131): x (+ in_bias[c] in FP32) -> GELU (erf or tanh form) in FP32 -> rounded to the dtype code `rnd` (FP32:
// unrounded).
enum { MODE_INT8 = 0, MODE_MX = 1 };

template <int MODE>
struct Quantizer {
  float scale;            // INT8 scale
  float inv;              // INT8 1 / scale
  const float* cs;        // INT8 optional per-channel pre-multiplier (SmoothQuant's 1/s)
  const int8_t* expo;     // MX static exponents [Cpad / 32]
  int gelu;               // GELU first (uniform): 0 none, 1 erf form, 2 tanh form
  int rnd;                // dtype code the GELU result is rounded to
  const float* in_bias;   // GELU's optional FP32 input bias [C]

  __device__ __forceinline__ uint8_t operator()(float v, int64_t c) const {
    if (gelu) {
      if (in_bias != nullptr) v = __fadd_rn(v, in_bias[c]);
      v = gelu == 2 ? gelu_tanh(v) : gelu_erf(v);
      if (rnd == FIM_BF16) v = round_bf16_hw(v);
      else if (rnd == FIM_F16) v = (float)(_Float16)v;
    }
    if (MODE == MODE_INT8) {
      if (cs != nullptr) v = v * cs[c];
      return (uint8_t)quantize_int8_fast(v, scale, inv);
    } else {
      float inv = exp2_int(-(int)expo[c >> 5]);
      return e4m3(mx_scale_clamp(v, inv));
    }
  }
};

template <int DT>
__device__ __forceinline__ void load8(const void* x, int64_t off, float* v) {
  if (DT == FIM_BF16) {
    uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + off);
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = u2f(w[i] << 16);
      v[2 * i + 1] = u2f(w[i] & 0xffff0000u);
    }
  } else if (DT == FIM_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + off);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const _Float16* p = static_cast<const _Float16*>(x) + off;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)p[i];
  }
}

// Channel-contiguous path. One lane = 8 output channels of one pixel; Cout = C (INT8) or Cpad (MX, zero padded).
template <int DT, int MODE>
__global__ __launch_bounds__(256) void quantize_rows_vec8(const void* __restrict__ x, Geometry4 g, int packed,
                                                          Quantizer<MODE> qz, const float* __restrict__ scale_ptr,
                                                          uint8_t* __restrict__ out, int64_t Cout) {
  if (MODE == MODE_INT8) {
    qz.scale = *scale_ptr;
    qz.inv = __fdiv_rn(1.0f, qz.scale);
  }
  const int64_t groups = Cout >> 3;
  const int64_t total = g.B * g.H * g.W * groups;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = i / groups;
    int64_t c0 = (i - r * groups) << 3;
    uint32_t lo = 0, hi = 0;
    if (c0 < g.C) {
      int64_t off;
      if (packed) {
        off = r * g.C + c0;
      } else {
        int64_t w = r % g.W, t = r / g.W;
        int64_t h = t % g.H, b = t / g.H;
        off = b * g.sb + h * g.sh + w * g.sw + c0;
      }
      float v[8];
      load8<DT>(x, off, v);
      uint8_t q[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] = qz(v[j], c0 + j);
      lo = q[0] | (q[1] << 8) | (q[2] << 16) | ((uint32_t)q[3] << 24);
      hi = q[4] | (q[5] << 8) | (q[6] << 16) | ((uint32_t)q[7] << 24);
    }
    *reinterpret_cast<uint2*>(out + r * Cout + c0) = make_uint2(lo, hi);
  }
}

// Width-contiguous path (NCHW view): block = 64 pixels of one image row x 64 output channels.
template <int DT, int MODE>
__global__ __launch_bounds__(256) void quantize_rows_transpose(const void* __restrict__ x, Geometry4 g,
                                                               Quantizer<MODE> qz, const float* __restrict__ scale_ptr,
                                                               uint8_t* __restrict__ out, int64_t Cout) {
  __shared__ float tile[64][65];
  if (MODE == MODE_INT8) {
    qz.scale = *scale_ptr;
    qz.inv = __fdiv_rn(1.0f, qz.scale);
  }
  const int64_t w0 = (int64_t)blockIdx.x * 64;
  const int64_t c0 = (int64_t)blockIdx.y * 64;
  const int64_t bh = blockIdx.z;
  const int64_t b = bh / g.H, h = bh % g.H;
  const int tid = threadIdx.x;
  // read: lane -> (w = tid % 64, c = tid / 64 + 4 k)
  {
    const int wl = tid & 63;
    const int64_t w = w0 + wl;
#pragma unroll 4
    for (int k = 0; k < 16; ++k) {
      int cl = (tid >> 6) + 4 * k;
      int64_t c = c0 + cl;
      float v = 0.0f;
      if (w < g.W && c < g.C) v = load_elem<DT>(x, b * g.sb + h * g.sh + w * g.sw + c * g.sc);
      tile[cl][wl] = v;
    }
  }
  __syncthreads();
  // write: lane -> (pixel = tid / 4, 16 channels = (tid % 4) * 16)
  {
    const int pl = tid >> 2, cq = (tid & 3) * 16;
    const int64_t w = w0 + pl;
    const int64_t cbase = c0 + cq;
    if (w < g.W && cbase < Cout) {
      uint8_t q[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int64_t c = cbase + j;
        q[j] = (c < g.C) ? qz(tile[cq + j][pl], c) : (uint8_t)0;
      }
      uint8_t* dst = out + ((b * g.H + h) * g.W + w) * Cout + cbase;
      int64_t n = Cout - cbase < 16 ? Cout - cbase : 16;
      if (n == 16 && ((uintptr_t)dst & 15) == 0) {
        uint4 pk;
        pk.x = q[0] | (q[1] << 8) | (q[2] << 16) | ((uint32_t)q[3] << 24);
        pk.y = q[4] | (q[5] << 8) | (q[6] << 16) | ((uint32_t)q[7] << 24);
        pk.z = q[8] | (q[9] << 8) | (q[10] << 16) | ((uint32_t)q[11] << 24);
        pk.w = q[12] | (q[13] << 8) | (q[14] << 16) | ((uint32_t)q[15] << 24);
        *reinterpret_cast<uint4*>(dst) = pk;
      } else {
        for (int j = 0; j < n; ++j) dst[j] = q[j];
      }
    }
  }
}

// Generic path: one output element per lane.
template <int DT, int MODE>
__global__ __launch_bounds__(256) void quantize_rows_scalar(const void* __restrict__ x, Geometry4 g,
                                                            Quantizer<MODE> qz, const float* __restrict__ scale_ptr,
                                                            uint8_t* __restrict__ out, int64_t Cout) {
  if (MODE == MODE_INT8) {
    qz.scale = *scale_ptr;
    qz.inv = __fdiv_rn(1.0f, qz.scale);
  }
  const int64_t total = g.B * g.H * g.W * Cout;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = i / Cout, c = i - r * Cout;
    uint8_t q = 0;
    if (c < g.C) {
      int64_t w = r % g.W, t = r / g.W;
      int64_t h = t % g.H, b = t / g.H;
      q = qz(load_elem<DT>(x, b * g.sb + h * g.sh + w * g.sw + c * g.sc), c);
    }
    out[i] = q;
  }
}

// Packed fast path: contiguous [rows, C] input, no padding (Cout == C), C % 16 == 0, total < 2^31 elements. Lane i
// quantizes elements [16 i, 16 i + 16): two 16-byte BF16 loads (four for FP32) and one 16-byte store; the 16 channels
// share one MX exponent (c0 % 16 == 0 lies in one 32-channel block), so the exponent is read and converted once.
template <int DT>
__device__ __forceinline__ void load16(const void* x, uint32_t off, float* v) {
  load8<DT>(x, off, v);
  load8<DT>(x, off + 8, v + 8);
}

template <int DT, int MODE>
__global__ __launch_bounds__(256) void quantize_packed_vec16(const void* __restrict__ x, uint32_t n16, uint32_t C,
                                                             Quantizer<MODE> qz, const float* __restrict__ scale_ptr,
                                                             uint8_t* __restrict__ out) {
  // 16-element groups per lane, 256 groups apart (each load instruction stays coalesced): two loads in flight per lane
  // (config 3's quantizer: cold 8.3 -> 6.6 us, hot 5.3 -> 4.5 us; 4: cold 7.2 us; consecutive groups per lane, which
  // strides each instruction's lanes 64 bytes apart: 10.6 us)
  constexpr int U = 2;
  float scale = 1.0f, inv = 1.0f;
  if (MODE == MODE_INT8) {
    scale = *scale_ptr;
    inv = __fdiv_rn(1.0f, scale);
  }
  const uint32_t i0 = blockIdx.x * 256u * U + threadIdx.x;
  float v[U][16];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (i0 + 256u * u < n16) load16<DT>(x, 16u * (i0 + 256u * u), v[u]);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = i0 + 256u * u;
    if (i >= n16) break;
    const uint32_t c0 = (16u * i) % C;
    uint32_t w[4];
    if (MODE == MODE_MX) {
      const float einv = exp2_int(-(int)qz.expo[c0 >> 5]);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = pack_e4m3x4(mx_scale_clamp(v[u][4 * k], einv), mx_scale_clamp(v[u][4 * k + 1], einv),
                           mx_scale_clamp(v[u][4 * k + 2], einv), mx_scale_clamp(v[u][4 * k + 3], einv));
    } else {
      if (qz.cs != nullptr) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[u][j] = v[u][j] * qz.cs[c0 + j];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t q = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) q |= (uint32_t)(uint8_t)quantize_int8_fast(v[u][4 * k + j], scale, inv) << (8 * j);
        w[k] = q;
      }
    }
    // streaming store: the codes are read once, by the next kernel
    __builtin_nontemporal_store(v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]}, reinterpret_cast<v4i*>(out + 16u * i));
  }
}

template <int DT, int MODE>
static int launch_quantize(const void* x, Geometry4 g, Quantizer<MODE> qz, const float* scale, uint8_t* out,
                           int64_t Cout, hipStream_t stream) {
  const int64_t rows = g.B * g.H * g.W;
  if (rows == 0 || Cout == 0) return FIM_OK;
  const int esize = DT == FIM_F32 ? 4 : 2;
  const bool aligned = ((uintptr_t)x % 16) == 0 && ((uintptr_t)out % 8) == 0;
  const bool packed_all = g.sc == 1 && g.sw == g.C && g.sh == g.W * g.C && g.sb == g.H * g.W * g.C;
  if (!qz.gelu && packed_all && Cout == g.C && g.C % 16 == 0 && ((uintptr_t)out % 16) == 0 && aligned &&
      rows * g.C < (1LL << 31)) {
    const uint32_t n16 = (uint32_t)(rows * g.C / 16);
    quantize_packed_vec16<DT, MODE><<<dim3((unsigned)cdiv(n16, 512)), dim3(256), 0, stream>>>(
        x, n16, (uint32_t)g.C, qz, scale, out);
    return launch_status();
  }
  if (g.sc == 1 && g.C % 8 == 0 && Cout % 8 == 0 && aligned && (g.sb * esize) % 16 == 0 &&
      (g.sh * esize) % 16 == 0 && (g.sw * esize) % 16 == 0) {
    const int packed = (g.sw == g.C && g.sh == g.W * g.C && g.sb == g.H * g.W * g.C) ? 1 : 0;
    int64_t total = rows * (Cout / 8);
    int64_t blocks = cdiv(total, 256);
    if (blocks > 65536) blocks = 65536;
    quantize_rows_vec8<DT, MODE><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(x, g, packed, qz, scale, out, Cout);
  } else if (g.sw == 1 && g.W >= 16 && g.B * g.H <= 65535) {
    dim3 grid((unsigned)cdiv(g.W, 64), (unsigned)cdiv(Cout, 64), (unsigned)(g.B * g.H));
    quantize_rows_transpose<DT, MODE><<<grid, dim3(256), 0, stream>>>(x, g, qz, scale, out, Cout);
  } else {
    int64_t blocks = cdiv(rows * Cout, 256);
    if (blocks > 65536) blocks = 65536;
    quantize_rows_scalar<DT, MODE><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(x, g, qz, scale, out, Cout);
  }
  return launch_status();
}

template <int MODE>
static int dispatch_quantize(const void* x, int dtype, Geometry4 g, Quantizer<MODE> qz, const float* scale,
                             uint8_t* out, int64_t Cout, hipStream_t stream) {
  switch (dtype) {
    case FIM_F32: return launch_quantize<FIM_F32, MODE>(x, g, qz, scale, out, Cout, stream);
    case FIM_BF16: return launch_quantize<FIM_BF16, MODE>(x, g, qz, scale, out, Cout, stream);
    case FIM_F16: return launch_quantize<FIM_F16, MODE>(x, g, qz, scale, out, Cout, stream);
    default: return FIM_ERR_UNSUPPORTED;
  }
}

// ----- dynamic per-(row, 32) MXFP8 ------------------------------------------------------------------------------

// cuBLAS SWIZZLE_32_4_4 byte offset of scale (row r, group gi) for `tiles_k = ceil(groups / 4)`
// (flashim/quant/formats/mx.py:67-86; closed form at flashim/backends/triton/conv.py:118-124).
__device__ __forceinline__ int64_t swizzle_offset(int64_t r, int64_t gi, int64_t tiles_k) {
  int64_t rt = r & 127;
  return (((r >> 7) * tiles_k + (gi >> 2)) << 9) + (rt & 31) * 16 + (rt >> 5) * 4 + (gi & 3);
}

// Four lanes per 32-element block, 8 elements per lane; the block amax is a 4-lane butterfly.
template <int DT>
__global__ __launch_bounds__(256) void quantize_dynamic_kernel(const void* __restrict__ x, int64_t rows, int64_t K,
                                                               int64_t row_stride, uint8_t* __restrict__ out,
                                                               int8_t* __restrict__ expo_out,
                                                               uint8_t* __restrict__ swizzled) {
  const int64_t lanes_per_row = K >> 3;
  const int64_t total = rows * lanes_per_row;
  const int64_t groups = K >> 5;
  const int64_t tiles_k = (groups + 3) >> 2;
  // grid-stride in whole wavefronts so every lane of a 4-lane block is present in each iteration
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x; base < total; base += (int64_t)gridDim.x * blockDim.x) {
    int64_t i = base + threadIdx.x;
    bool live = i < total;
    int64_t r = live ? i / lanes_per_row : 0;
    int64_t c0 = live ? (i - r * lanes_per_row) << 3 : 0;
    float v[8];
    if (live) {
      const int64_t off = r * row_stride + c0;
      if (DT == FIM_BF16 || DT == FIM_F32) {
        load8<DT>(x, off, v);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = load_elem<DT>(x, off + j);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const int e = mx_exponent_wave(amax);  // (all lanes: the slow path's branch is wave-uniform)
    if (!live) continue;
    const float inv = exp2_int(-e);
    uint32_t lo = pack_e4m3x4(mx_scale_clamp(v[0], inv), mx_scale_clamp(v[1], inv), mx_scale_clamp(v[2], inv),
                              mx_scale_clamp(v[3], inv));
    uint32_t hi = pack_e4m3x4(mx_scale_clamp(v[4], inv), mx_scale_clamp(v[5], inv), mx_scale_clamp(v[6], inv),
                              mx_scale_clamp(v[7], inv));
    *reinterpret_cast<uint2*>(out + r * K + c0) = make_uint2(lo, hi);
    if ((c0 & 31) == 0) {
      const int64_t gi = c0 >> 5;
      if (expo_out != nullptr) expo_out[r * groups + gi] = (int8_t)e;
      if (swizzled != nullptr) swizzled[swizzle_offset(r, gi, tiles_k)] = (uint8_t)(e + 127);
    }
  }
}

// ----- per-row INT8 ------------------------------------------------------------------------------------------

// One workgroup per row: amax -> scale -> quantize. RECIPROCAL = 0: scale = amax / 127 (weight_scales, an IEEE
// division); 1: scale = amax * (1 / 127) (quantize_int8_rows). Then safe_scale: non-finite or <= FLT_EPSILON -> eps.
template <int DT>
__global__ __launch_bounds__(256) void quantize_int8_rows_kernel(const void* __restrict__ x, int64_t K,
                                                                 int64_t row_stride, int reciprocal,
                                                                 int8_t* __restrict__ out,
                                                                 float* __restrict__ scale_out) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int64_t base = r * row_stride;
  float amax = 0.0f;
  for (int64_t c = threadIdx.x; c < K; c += 256) amax = fmaxf(amax, fabsf(load_elem<DT>(x, base + c)));
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float s = reciprocal ? amax * (1.0f / 127.0f) : __fdiv_rn(amax, 127.0f);
  const float eps = 1.1920928955078125e-07f;
  if (!(s > eps) || !__builtin_isfinite(s)) s = eps;
  if (threadIdx.x == 0) scale_out[r] = s;
  const float inv = __fdiv_rn(1.0f, s);
  for (int64_t c = threadIdx.x; c < K; c += 256) out[r * K + c] = quantize_int8_fast(load_elem<DT>(x, base + c), s, inv);
}

// ----- static exponent calibration (amax over rows per 32-channel block) -------------------------------------

__global__ void fill_u32(uint32_t* p, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Non-negative FP32 values order like their bit patterns, so the block amax is an integer atomicMax on the bits.
template <int DT>
__global__ __launch_bounds__(256) void block_amax_kernel(const void* __restrict__ x, int64_t rows, int64_t C,
                                                         int64_t row_stride, int64_t rows_per_block,
                                                         uint32_t* __restrict__ amax_bits) {
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one channel per lane
  float a = 0.0f;
  if (c < C) {
    int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    for (int64_t r = r0; r < r1; ++r) a = fmaxf(a, fabsf(load_elem<DT>(x, r * row_stride + c)));
  }
  // lanes 32 apart share nothing; reduce within each aligned group of 32 channels (one MX block)
  for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
  if ((threadIdx.x & 31) == 0 && c < C) atomicMax(amax_bits + (c >> 5), f2u(a));
}

__global__ void block_exponent_kernel(const uint32_t* __restrict__ amax_bits, int64_t groups,
                                      int8_t* __restrict__ expo) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < groups) expo[i] = (int8_t)mx_exponent_from_amax(u2f(amax_bits[i]));
}

// The launch sequence of the static-exponent calibration: clear the per-block amax words (a kernel, not a memset, so
// the sequence can be captured in a graph), one atomicMax per 32-channel block and row slab, then the exponent rule.
static int calibrate_launch(const void* x, int dtype, int64_t rows, int64_t C, int64_t row_stride, uint32_t* workspace,
                            int8_t* exponent, hipStream_t stream) {
  const int64_t groups = (C + 31) / 32;
  fill_u32<<<dim3((unsigned)cdiv(groups, 256)), dim3(256), 0, stream>>>(workspace, groups);
  if (rows > 0) {
    int64_t rows_per_block = 64;
    int64_t yb = cdiv(rows, rows_per_block);
    while (yb > 65535) {
      rows_per_block *= 2;
      yb = cdiv(rows, rows_per_block);
    }
    dim3 grid((unsigned)cdiv(C, 256), (unsigned)yb);
    switch (dtype) {
      case FIM_F32:
        block_amax_kernel<FIM_F32><<<grid, dim3(256), 0, stream>>>(x, rows, C, row_stride, rows_per_block, workspace);
        break;
      case FIM_BF16:
        block_amax_kernel<FIM_BF16><<<grid, dim3(256), 0, stream>>>(x, rows, C, row_stride, rows_per_block, workspace);
        break;
      default:
        block_amax_kernel<FIM_F16><<<grid, dim3(256), 0, stream>>>(x, rows, C, row_stride, rows_per_block, workspace);
        break;
    }
  }
  block_exponent_kernel<<<dim3((unsigned)cdiv(groups, 256)), dim3(256), 0, stream>>>(workspace, groups, exponent);
  return launch_status();
}

// Scratch of the allocation-free calibration entry point: the per-block amax words live in this file-scope device
// array (every GPU the library runs on holds its own copy, 16 KiB, until the process ends). Its device address is
// looked up once per device with that device current and cached; host code passes only that address to kernels.
constexpr int64_t FIM_CALIBRATE_MAX_GROUPS = 4096;  // C <= 131072 channels
static __device__ __align__(256) uint32_t scratch[FIM_CALIBRATE_MAX_GROUPS];
constexpr int FIM_MAX_DEVICES = 64;
static uint32_t* scratch_ptr[FIM_MAX_DEVICES];
static std::mutex scratch_mutex;

static int calibrate_scratch(uint32_t** ptr) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return (int)err;
  if (device < 0 || device >= FIM_MAX_DEVICES) return FIM_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_ptr[device] == nullptr) {
    void* addr = nullptr;
    err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return (int)err;
    scratch_ptr[device] = static_cast<uint32_t*>(addr);
  }
  *ptr = scratch_ptr[device];
  return FIM_OK;
}

}  // namespace fim

using namespace fim;

extern "C" {

int fim_quantize_int8(const void* x, int dtype, int64_t B, int64_t H, int64_t W, int64_t C, int64_t sb, int64_t sh,
                      int64_t sw, int64_t sc, const float* scale, const float* channel_scale, int8_t* out,
                      hipStream_t stream) {
  if (x == nullptr || scale == nullptr || out == nullptr || B < 0 || H < 0 || W < 0 || C < 0) return FIM_ERR_INVALID;
  Geometry4 g{B, H, W, C, sb, sh, sw, sc};
  Quantizer<MODE_INT8> qz{0.0f, 1.0f, channel_scale, nullptr, 0, 0, nullptr};
  return dispatch_quantize<MODE_INT8>(x, dtype, g, qz, scale, reinterpret_cast<uint8_t*>(out), C, stream);
}

int fim_quantize_mxfp8(const void* x, int dtype, int64_t B, int64_t H, int64_t W, int64_t C, int64_t sb, int64_t sh,
                       int64_t sw, int64_t sc, const int8_t* exponent, uint8_t* out, int64_t Cpad,
                       hipStream_t stream) {
  if (x == nullptr || exponent == nullptr || out == nullptr || B < 0 || H < 0 || W < 0 || C < 0) return FIM_ERR_INVALID;
  if (Cpad % 32 != 0 || Cpad < C || Cpad - C >= 32) return FIM_ERR_INVALID;
  Geometry4 g{B, H, W, C, sb, sh, sw, sc};
  Quantizer<MODE_MX> qz{0.0f, 1.0f, nullptr, exponent, 0, 0, nullptr};
  return dispatch_quantize<MODE_MX>(x, dtype, g, qz, nullptr, out, Cpad, stream);
}

int fim_gelu_quantize_mxfp8(const void* x, int dtype, int64_t B, int64_t H, int64_t W, int64_t C, int64_t sb,
                            int64_t sh, int64_t sw, int64_t sc, int approximate, const float* input_bias,
                            const int8_t* exponent, uint8_t* out, int64_t Cpad, hipStream_t stream) {
  if (x == nullptr || exponent == nullptr || out == nullptr || B < 0 || H < 0 || W < 0 || C < 0) return FIM_ERR_INVALID;
  if (approximate != 0 && approximate != 1) return FIM_ERR_INVALID;
  if (Cpad % 32 != 0 || Cpad < C || Cpad - C >= 32) return FIM_ERR_INVALID;
  Geometry4 g{B, H, W, C, sb, sh, sw, sc};
  Quantizer<MODE_MX> qz{0.0f, 1.0f, nullptr, exponent, 1 + approximate, dtype, input_bias};
  return dispatch_quantize<MODE_MX>(x, dtype, g, qz, nullptr, out, Cpad, stream);
}

int fim_gelu_quantize_int8(const void* x, int dtype, int64_t B, int64_t H, int64_t W, int64_t C, int64_t sb,
                           int64_t sh, int64_t sw, int64_t sc, int approximate, const float* scale, int8_t* out,
                           hipStream_t stream) {
  if (x == nullptr || scale == nullptr || out == nullptr || B < 0 || H < 0 || W < 0 || C < 0) return FIM_ERR_INVALID;
  if (approximate != 0 && approximate != 1) return FIM_ERR_INVALID;
  Geometry4 g{B, H, W, C, sb, sh, sw, sc};
  Quantizer<MODE_INT8> qz{0.0f, 1.0f, nullptr, nullptr, 1 + approximate, dtype, nullptr};
  return dispatch_quantize<MODE_INT8>(x, dtype, g, qz, scale, reinterpret_cast<uint8_t*>(out), C, stream);
}

int fim_quantize_mxfp8_dynamic(const void* x, int dtype, int64_t rows, int64_t K, int64_t row_stride, uint8_t* out,
                               int8_t* exponent, uint8_t* swizzled, hipStream_t stream) {
  if (x == nullptr || out == nullptr || rows < 0 || K < 0) return FIM_ERR_INVALID;
  if (K % 32 != 0) return FIM_ERR_UNSUPPORTED;
  if (rows == 0 || K == 0) return FIM_OK;
  const int esize = dtype == FIM_F32 ? 4 : 2;
  if (((uintptr_t)x % 16) != 0 || (row_stride * esize) % 16 != 0 || ((uintptr_t)out % 8) != 0) return FIM_ERR_UNSUPPORTED;
  int64_t total = rows * (K / 8);
  int64_t blocks = cdiv(total, 256);
  if (blocks > 65536) blocks = 65536;
  switch (dtype) {
    case FIM_F32:
      quantize_dynamic_kernel<FIM_F32><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(x, rows, K, row_stride, out,
                                                                                         exponent, swizzled);
      break;
    case FIM_BF16:
      quantize_dynamic_kernel<FIM_BF16><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(x, rows, K, row_stride, out,
                                                                                          exponent, swizzled);
      break;
    case FIM_F16:
      quantize_dynamic_kernel<FIM_F16><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(x, rows, K, row_stride, out,
                                                                                         exponent, swizzled);
      break;
    default: return FIM_ERR_UNSUPPORTED;
  }
  return launch_status();
}

int fim_quantize_int8_rows(const void* x, int dtype, int64_t rows, int64_t K, int64_t row_stride, int reciprocal,
                           int8_t* out, float* scale, hipStream_t stream) {
  if (x == nullptr || out == nullptr || scale == nullptr || rows < 0 || K < 0) return FIM_ERR_INVALID;
  if (rows == 0) return FIM_OK;
  if (rows > 2147483647LL) return FIM_ERR_UNSUPPORTED;
  dim3 grid((unsigned)rows);
  switch (dtype) {
    case FIM_F32:
      quantize_int8_rows_kernel<FIM_F32><<<grid, dim3(256), 0, stream>>>(x, K, row_stride, reciprocal, out, scale);
      break;
    case FIM_BF16:
      quantize_int8_rows_kernel<FIM_BF16><<<grid, dim3(256), 0, stream>>>(x, K, row_stride, reciprocal, out, scale);
      break;
    case FIM_F16:
      quantize_int8_rows_kernel<FIM_F16><<<grid, dim3(256), 0, stream>>>(x, K, row_stride, reciprocal, out, scale);
      break;
    default: return FIM_ERR_UNSUPPORTED;
  }
  return launch_status();
}

int fim_calibrate_block32(const void* x, int dtype, int64_t rows, int64_t C, int64_t row_stride, uint32_t* workspace,
                          int8_t* exponent, hipStream_t stream) {
  if (x == nullptr || workspace == nullptr || exponent == nullptr || rows < 0 || C <= 0) return FIM_ERR_INVALID;
  if (dtype != FIM_F32 && dtype != FIM_BF16 && dtype != FIM_F16) return FIM_ERR_UNSUPPORTED;
  return calibrate_launch(x, dtype, rows, C, row_stride, workspace, exponent, stream);
}

int fim_calibrate_block32_noalloc(const void* x, int dtype, int64_t rows, int64_t C, int64_t row_stride,
                                  int8_t* exponent, hipStream_t stream) {
  if (x == nullptr || exponent == nullptr || rows < 0 || C <= 0) return FIM_ERR_INVALID;
  if (dtype != FIM_F32 && dtype != FIM_BF16 && dtype != FIM_F16) return FIM_ERR_UNSUPPORTED;
  if ((C + 31) / 32 > FIM_CALIBRATE_MAX_GROUPS) return FIM_ERR_UNSUPPORTED;
  uint32_t* workspace = nullptr;
  const int status = calibrate_scratch(&workspace);
  if (status != FIM_OK) return status;
  return calibrate_launch(x, dtype, rows, C, row_stride, workspace, exponent, stream);
}

}  // extern "C"
