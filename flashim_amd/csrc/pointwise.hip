// BF16 pointwise (1x1) GEMM of the BF16 refiner block: out[m, n] = bf16(sum_k x[m, k] w[n, k] + bias[n]) with FP32
// accumulation, the second half of depthwise5x5_relu_pointwise (flashim/ops/conv.py:67-81: the depthwise result is
// rounded to BF16, then F.conv2d with the [C_out, C_in] weight and an FP32 bias, then BF16). The first half is the
// depthwise producer's ReLU + BF16 mode (depthwise.hip).
//
// Layout: x BF16 [M, K] (pixels x channels, NHWC rows), w BF16 [N, K], bias FP32 [N] or null, out BF16 [M, N].
// K in {32, 64, 96, 128}, N a multiple of 16 up to 128: the refiner blocks' channel counts (the reference fuses
// 16..128 channels, flashim/ops/conv.py:82-84).
//
// The op is HBM-bound (K, N <= 128: at most 128 FLOP per byte moved), so the kernel is a stream: each wavefront takes
// 16-pixel blocks in a grid-strided loop, loads the next block's operands while it multiplies the current one, and
// keeps the weight in LDS (staged once per workgroup, rows padded by 16 bytes: the 16 rows one MFMA operand reads
// start 4 banks apart, so a 16-byte read of 16 lanes covers all 64 banks once).
// Matrix unit: v_mfma_f32_16x16x32_bf16, A = 16 output channels of the weight, B = 16 pixels; lane l supplies row l % 16
// of A and column l % 16 of B over the same 8 K values (K group l / 16), so any assignment of K groups inside the
// instruction multiplies matching pairs. Lane l receives D[4 (l / 16) + i][l % 16]: 4 consecutive output channels of
// pixel l % 16, written to a wavefront-private LDS row; the block's 16 output rows, contiguous in memory, then leave as
// 16-byte stores of consecutive lanes. The bias is the accumulator's initial value (-0 without bias: x + (-0) == x).
#include "common.h"

namespace fim {

typedef __bf16 v8bf16 __attribute__((ext_vector_type(8)));

constexpr int PW_WAVES = 4;

template <int KS, int NB>
__global__ __launch_bounds__(256) void pw_bf16_kernel(const uint16_t* __restrict__ x, int64_t M,
                                                      const uint16_t* __restrict__ w, const void* __restrict__ bias,
                                                      int bias_bf16, uint16_t* __restrict__ out, int64_t nblocks) {
  constexpr int K = 32 * KS, N = 16 * NB;
  constexpr int WROW = K + 8;  // BF16 elements per staged weight row
  __shared__ __align__(16) uint16_t sw[N * WROW];
  __shared__ float sb[N];
  // per wavefront: its 16 pixels' outputs, rows of N BF16 padded by 16 bytes (the 4-lane groups of one row land in
  // other banks than the next row's)
  constexpr int SROW = 2 * N + 16;
  __shared__ __align__(16) uint8_t stage[PW_WAVES][16 * SROW];
  for (int i = threadIdx.x; i < N * (K / 8); i += 256) {
    const int r = i / (K / 8), c = i % (K / 8);
    *reinterpret_cast<uint4*>(&sw[r * WROW + 8 * c]) = *reinterpret_cast<const uint4*>(&w[(int64_t)r * K + 8 * c]);
  }
  for (int i = threadIdx.x; i < N; i += 256)
    sb[i] = bias == nullptr ? -0.0f
            : bias_bf16     ? bf16_to_f32(static_cast<const uint16_t*>(bias)[i])
                            : static_cast<const float*>(bias)[i];
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t nwaves = (int64_t)gridDim.x * PW_WAVES;
  int64_t blk = (int64_t)blockIdx.x * PW_WAVES + (threadIdx.x >> 6);

  auto load = [&](int64_t b, v8bf16 (&v)[KS]) {
    const int64_t row = b * 16 + r16;
    if (row < M) {
#pragma unroll
      for (int s = 0; s < KS; ++s) v[s] = *reinterpret_cast<const v8bf16*>(&x[row * K + 32 * s + 8 * g]);
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) v[s] = v8bf16{};
    }
  };

  v8bf16 cur[KS];
  if (blk < nblocks) load(blk, cur);
  for (; blk < nblocks; blk += nwaves) {
    v8bf16 nxt[KS];
    if (blk + nwaves < nblocks) load(blk + nwaves, nxt);
    v4f acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      acc[nb] = *reinterpret_cast<const v4f*>(&sb[16 * nb + 4 * g]);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const v8bf16 a = *reinterpret_cast<const v8bf16*>(&sw[(16 * nb + r16) * WROW + 32 * s + 8 * g]);
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, cur[s], acc[nb], 0, 0, 0);
      }
    }
    // outputs through LDS: lane l writes 4 channels of pixel l % 16, then the block (16 rows of 2 N bytes, contiguous
    // in the output) leaves as 16-byte stores of consecutive lanes, whole lines per instruction
    uint8_t* const st = stage[threadIdx.x >> 6];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      uint2 v;
      v.x = pack_bf16x2(acc[nb][0], acc[nb][1]);
      v.y = pack_bf16x2(acc[nb][2], acc[nb][3]);
      *reinterpret_cast<uint2*>(st + r16 * SROW + 2 * (16 * nb + 4 * g)) = v;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0) (vmcnt, expcnt untouched): this wavefront's LDS writes
    constexpr int CPR = 2 * N / 16;       // 16-byte chunks per pixel row
    const int64_t rows_left = M - blk * 16;
#pragma unroll
    for (int i = 0; i < (16 * CPR + 63) / 64; ++i) {
      const int c = lane + 64 * i;
      const int r = c / CPR, q = c % CPR;
      if (c < 16 * CPR && r < rows_left) {
        const uint4 v = *reinterpret_cast<const uint4*>(st + r * SROW + 16 * q);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(out) + ((blk * 16 + r) * N) * 2 + 16 * q) = v;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // the staged rows read before the next block overwrites them
#pragma unroll
    for (int s = 0; s < KS; ++s) cur[s] = nxt[s];
  }
}

template <int KS>
static void pw_launch_n(int nb, dim3 grid, hipStream_t s, const uint16_t* x, int64_t M, const uint16_t* w,
                        const void* bias, int bias_bf16, uint16_t* out, int64_t nblocks) {
  switch (nb) {
    case 1: pw_bf16_kernel<KS, 1><<<grid, dim3(256), 0, s>>>(x, M, w, bias, bias_bf16, out, nblocks); break;
    case 2: pw_bf16_kernel<KS, 2><<<grid, dim3(256), 0, s>>>(x, M, w, bias, bias_bf16, out, nblocks); break;
    case 3: pw_bf16_kernel<KS, 3><<<grid, dim3(256), 0, s>>>(x, M, w, bias, bias_bf16, out, nblocks); break;
    case 4: pw_bf16_kernel<KS, 4><<<grid, dim3(256), 0, s>>>(x, M, w, bias, bias_bf16, out, nblocks); break;
    case 5: pw_bf16_kernel<KS, 5><<<grid, dim3(256), 0, s>>>(x, M, w, bias, bias_bf16, out, nblocks); break;
    case 6: pw_bf16_kernel<KS, 6><<<grid, dim3(256), 0, s>>>(x, M, w, bias, bias_bf16, out, nblocks); break;
    case 7: pw_bf16_kernel<KS, 7><<<grid, dim3(256), 0, s>>>(x, M, w, bias, bias_bf16, out, nblocks); break;
    default: pw_bf16_kernel<KS, 8><<<grid, dim3(256), 0, s>>>(x, M, w, bias, bias_bf16, out, nblocks); break;
  }
}

}  // namespace fim

using namespace fim;

extern "C" {

int fim_pointwise_bf16(const uint16_t* x, int64_t M, int64_t K, const uint16_t* weight, int64_t N, const void* bias,
                       int bias_dtype, uint16_t* out, hipStream_t stream) {
  if (x == nullptr || weight == nullptr || out == nullptr || M < 0 || K <= 0 || N <= 0) return FIM_ERR_INVALID;
  if (bias_dtype != FIM_F32 && bias_dtype != FIM_BF16) return FIM_ERR_INVALID;
  const int bias_bf16 = bias_dtype == FIM_BF16;
  if (K % 32 != 0 || K > 128 || N % 16 != 0 || N > 128) return FIM_ERR_UNSUPPORTED;
  if (((uintptr_t)x % 16) != 0 || ((uintptr_t)weight % 16) != 0 || ((uintptr_t)out % 16) != 0) return FIM_ERR_UNSUPPORTED;
  if (M == 0) return FIM_OK;
  const int64_t nblocks = cdiv(M, 16);
  // Enough waves to keep every CU streaming (8 workgroups of 4 waves per CU on 256 CUs), each wave several blocks.
  const int64_t wgs = std::min<int64_t>(cdiv(nblocks, PW_WAVES), 2048);
  const dim3 grid((unsigned)wgs);
  switch (K / 32) {
    case 1: pw_launch_n<1>((int)(N / 16), grid, stream, x, M, weight, bias, bias_bf16, out, nblocks); break;
    case 2: pw_launch_n<2>((int)(N / 16), grid, stream, x, M, weight, bias, bias_bf16, out, nblocks); break;
    case 3: pw_launch_n<3>((int)(N / 16), grid, stream, x, M, weight, bias, bias_bf16, out, nblocks); break;
    default: pw_launch_n<4>((int)(N / 16), grid, stream, x, M, weight, bias, bias_bf16, out, nblocks); break;
  }
  return launch_status();
}

}  // extern "C"
