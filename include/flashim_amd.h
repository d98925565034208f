/* flashim_amd: C ABI of the MI355X (gfx950) quantized implicit-GEMM convolution path.
 *
 * Every entry point enqueues its kernels on `stream` and returns without synchronizing. Pointers are device pointers
 * (borrowed for the duration of the launch; the library allocates nothing). Sizes are element counts, strides are in
 * elements. The return value is 0 on success, FIM_ERR_INVALID (98) for a null pointer or inconsistent size,
 * FIM_ERR_UNSUPPORTED (99) for a shape or alignment this library has no kernel for, or a hipError_t code from the
 * launch. This mirrors the CUDA C++ backend's launch convention (flashim/backends/cuda/csrc/depthwise.cu:407-412 and
 * its ctypes caller flashim/backends/cuda/conv.py:135-145): plain pointers, ints and the stream, nonzero = failure.
 *
 * Floating activation dtype codes: 0 = float32, 1 = bfloat16, 2 = float16.
 * Byte formats: int8 (two's complement), E4M3 = OCP float8_e4m3fn, MX exponents = unbiased int8 (2^e), E8M0 = e + 127.
 */
#ifndef FLASHIM_AMD_H
#define FLASHIM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

#define FIM_OK 0
#define FIM_ERR_INVALID 98
#define FIM_ERR_UNSUPPORTED 99

/* Library version (major * 10000 + minor * 100 + patch). */
int fim_version(void);

/* ---- quantizers -------------------------------------------------------------------------------------------- */

/* Static per-tensor INT8: out[b,h,w,c] = clamp(round_half_even(x[b,h,w,c] * channel_scale[c] / *scale), +-127).
 * x is [B, H, W, C] with element strides (sb, sh, sw, sc): the NHWC view of NCHW memory is read in place; out is
 * packed [B, H, W, C]. channel_scale may be NULL. Replaces the impl of ops.quantize_int8
 * (flashim/ops/quantize.py:91-100; reference quant/tensor.py:148-151, quant/formats/int8.py:24-27). */
int fim_quantize_int8(const void* x, int dtype, int64_t B, int64_t H, int64_t W, int64_t C, int64_t sb, int64_t sh,
                      int64_t sw, int64_t sc, const float* scale, const float* channel_scale, int8_t* out,
                      hipStream_t stream);

/* Static block-32 MXFP8: out[r, c] = e4m3(clamp(x[r, c] / 2^exponent[c / 32], +-448)) for c < C, 0 for
 * C <= c < Cpad (Cpad = C rounded up to 32). Same input geometry as fim_quantize_int8; out is [B*H*W, Cpad].
 * Replaces ops.quantize_mxfp8 (flashim/ops/quantize.py:80-85; reference quant/tensor.py:97-121). */
int fim_quantize_mxfp8(const void* x, int dtype, int64_t B, int64_t H, int64_t W, int64_t C, int64_t sb, int64_t sh,
                       int64_t sw, int64_t sc, const int8_t* exponent, uint8_t* out, int64_t Cpad,
                       hipStream_t stream);

/* GELU then static block-32 MXFP8, fim_quantize_mxfp8's geometry and output: v = x (+ input_bias[c] in FP32,
 * input_bias may be NULL), g = gelu(v) in FP32 rounded to x's dtype, out = e4m3(clamp(g / 2^exponent[c/32], +-448)).
 * approximate: 0 the erf form, 1 the tanh form (F.gelu's approximate="none" / "tanh"; else 98).
 * Replaces ops.gelu_quantize (flashim/ops/quantize.py:63-74). */
int fim_gelu_quantize_mxfp8(const void* x, int dtype, int64_t B, int64_t H, int64_t W, int64_t C, int64_t sb,
                            int64_t sh, int64_t sw, int64_t sc, int approximate, const float* input_bias,
                            const int8_t* exponent, uint8_t* out, int64_t Cpad, hipStream_t stream);

/* GELU (approximate as above) in x's dtype then static per-tensor INT8 with *scale, fim_quantize_int8's geometry and
 * output. Replaces ops.gelu_quantize_int8 (flashim/ops/quantize.py:128-131). */
int fim_gelu_quantize_int8(const void* x, int dtype, int64_t B, int64_t H, int64_t W, int64_t C, int64_t sb,
                           int64_t sh, int64_t sw, int64_t sc, int approximate, const float* scale, int8_t* out,
                           hipStream_t stream);

/* Dynamic per-(row, 32) MXFP8 of a [rows, K] matrix (K % 32 == 0, row stride in elements, 16-byte aligned rows):
 * E4M3 out [rows, K] (packed), exponent [rows, K/32] int8 (may be NULL), and the E8M0 scales in cuBLAS' 128x4
 * swizzled layout (may be NULL; its padding bytes are not written, the caller zero-fills them).
 * Replaces quant/formats/mx.py:50-60 (quantize_dynamic_2d) + :67-86 (swizzle_scales); also packs QuantizedWeight
 * (quant/tensor.py:77-87) from a padded weight. */
int fim_quantize_mxfp8_dynamic(const void* x, int dtype, int64_t rows, int64_t K, int64_t row_stride, uint8_t* out,
                               int8_t* exponent, uint8_t* swizzled, hipStream_t stream);

/* Per-row symmetric INT8: scale[r] = safe_scale(amax_r / 127) (reciprocal = 0, IEEE division: weight_scales,
 * quant/formats/int8.py:19-21) or safe_scale(amax_r * (1/127)) (reciprocal = 1: ops.quantize_int8_rows,
 * flashim/ops/quantize.py:148-157); out[r, k] = clamp(round_half_even(x[r, k] / scale[r]), +-127). out is packed
 * [rows, K]. */
int fim_quantize_int8_rows(const void* x, int dtype, int64_t rows, int64_t K, int64_t row_stride, int reciprocal,
                           int8_t* out, float* scale, hipStream_t stream);

/* Static exponent calibration: exponent[g] = scale_exponent_from_amax(max over rows and the 32 channels of block g
 * of |x|), g < ceil(C / 32) (quant/formats/mx.py:41-47). workspace: ceil(C/32) uint32 of caller memory. */
int fim_calibrate_block32(const void* x, int dtype, int64_t rows, int64_t C, int64_t row_stride, uint32_t* workspace,
                          int8_t* exponent, hipStream_t stream);

/* fim_calibrate_block32 without the caller's workspace: no counterpart in the reference. For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * per-block amax words live in a file-scope device array of FIM_CALIBRATE_MAX_GROUPS (4096) words, so C <= 131072
 * (larger C returns FIM_ERR_UNSUPPORTED). It runs on the calling thread's current device; every call on one device
 * shares that device's array (cleared at the start of each call), so calls that overlap on one device race. */
#define FIM_CALIBRATE_MAX_GROUPS 4096
int fim_calibrate_block32_noalloc(const void* x, int dtype, int64_t rows, int64_t C, int64_t row_stride,
                                  int8_t* exponent, hipStream_t stream);

/* ---- implicit-GEMM convolutions ----------------------------------------------------------------------------- */

/* INT8 conv2d, groups == 1: x int8 [B, H, W, Cin] packed; weight int8 [Cout, kh*kw*Cin] in (ky, kx, c) order;
 * a_scale one float, w_scale [Cout]; bias [Cout] (bias_dtype 0 f32 / 1 bf16) or NULL. Epilogue:
 * y = float(acc) * (a_scale * w_scale[n]) + bias[n] (two roundings); ReLU (when no residual); BF16; GELU if gelu;
 * residual [B, Ho, Wo, res_channels] with res_strides[4] added in FP32 (+ReLU) then BF16. out: BF16 [B, Ho, Wo, Cout],
 * or, when out_scale != NULL, that BF16 result statically quantized to INT8 with *out_scale.
 * Replaces ops.int8_conv2d (flashim/ops/conv.py:174-206; backend signature flashim/backends/triton/conv.py:816-833).
 * gelu has no counterpart in int8_conv2d: it is int8_linear's GELU epilogue (flashim/ops/gemm.py:94-95). */
int fim_int8_conv2d(const int8_t* x, int64_t B, int64_t H, int64_t W, int64_t Cin, const int8_t* weight, int64_t Cout,
                    const float* a_scale, const float* w_scale, const void* bias, int bias_dtype, int kh, int kw,
                    int sh, int sw, int ph, int pw, int dh, int dw, int relu, int gelu, const void* residual,
                    int res_dtype, int64_t res_channels, const int64_t* res_strides, const float* out_scale,
                    void* out, hipStream_t stream);

/* Static MXFP8 conv2d, groups == 1: x E4M3 [B, H, W, Cin] (Cin % 32 == 0) with channel_exponent [Cin/32] shared by
 * every tap; weight E4M3 [Cout, kh*kw*Cin] (ky, kx, c) with weight_exponent [Cout, kh*kw*Cin/32]. FP32 accumulation on
 * block-scaled MFMA; epilogue y = acc + bias, then as fim_int8_conv2d; out BF16 [B, Ho, Wo, Cout], or with
 * out_exponent [Cout/32] (Cout % 32 == 0) that BF16 result statically quantized to E4M3.
 * Replaces ops.mxfp8_conv2d (flashim/ops/conv.py:309-342; backend signature flashim/backends/triton/conv.py:1195-1238). */
int fim_mxfp8_conv2d(const uint8_t* x, int64_t B, int64_t H, int64_t W, int64_t Cin, const int8_t* channel_exponent,
                     const uint8_t* weight, int64_t Cout, const int8_t* weight_exponent, const void* bias,
                     int bias_dtype, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, int relu, int gelu,
                     const void* residual, int res_dtype, int64_t res_channels, const int64_t* res_strides,
                     const int8_t* out_exponent, void* out, hipStream_t stream);

/* int8_conv2d (no residual) followed by MaxPool2d(2) and the next conv's static INT8 quantize: out BF16 [B, Ho, Wo,
 * Cout] exactly as fim_int8_conv2d writes it, pooled int8 [B, Ho/2, Wo/2, Cout] = quantize(max_pool2d(out, 2),
 * out_scale) (a trailing odd row / column dropped). Even Ho, Wo: pooled in the conv's epilogue; odd: one extra pass.
 * Replaces ops.int8_conv2d_maxpool (flashim/ops/conv.py:209-222). */
int fim_int8_conv2d_maxpool(const int8_t* x, int64_t B, int64_t H, int64_t W, int64_t Cin, const int8_t* weight,
                            int64_t Cout, const float* a_scale, const float* w_scale, const void* bias,
                            int bias_dtype, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, int relu,
                            const float* out_scale, void* out, int8_t* pooled, hipStream_t stream);

/* INT8 GEMM a [M, K] x weight [N, K]^T with int8_linear's epilogue: acc * (a_scale * w_scale[n]) + bias[n] (two
 * roundings), ReLU, BF16, GELU if gelu, then + residual [M, res_channels] (row stride res_row_stride) in FP32 -> BF16.
 * a_scale_rows [M] (per-row dynamic activation scales) replaces *a_scale when non-NULL. out BF16 [M, N], or INT8 with
 * out_scale. Replaces ops.int8_linear (flashim/ops/gemm.py:78-101). */
int fim_int8_linear(const int8_t* a, int64_t M, int64_t K, const int8_t* weight, int64_t N, const float* a_scale,
                    const float* a_scale_rows, const float* w_scale, const void* bias, int bias_dtype, int relu, int gelu,
                    const void* residual, int res_dtype, int64_t res_channels, int64_t res_row_stride,
                    const float* out_scale, void* out, hipStream_t stream);

/* int8_linear (no ReLU, GELU or residual) statically quantized again to INT8 with *out_scale, written into out rows
 * out_row_stride bytes apart (out_row_stride >= N: e.g. one half of a concatenation buffer).
 * Replaces ops.int8_linear_quantize (flashim/ops/gemm.py:104-116). */
int fim_int8_linear_quantize(const int8_t* a, int64_t M, int64_t K, const int8_t* weight, int64_t N,
                             const float* a_scale, const float* a_scale_rows, const float* w_scale, const void* bias,
                             int bias_dtype, const float* out_scale, int8_t* out, int64_t out_row_stride,
                             hipStream_t stream);

/* Block-scaled MXFP8 GEMM: a [M, K] E4M3 with per-(row, 32) E8M0 scales in cuBLAS' 128x4 swizzled layout, weight
 * [N, K] E4M3 with scales [N, K/32]: int8 exponents (weight_scale_e8m0 0) or their E8M0 bytes, exponent + 127
 * (weight_scale_e8m0 1, the unswizzled pw_scale_u8 of the refiner-block ops) -> BF16 [M, N] (+ bias). Replaces
 * ops.mxfp8_scaled_mm (flashim/ops/gemm.py:40-52; the caller passes b_t^T and unswizzled b scales). */
int fim_mxfp8_scaled_mm(const uint8_t* a, int64_t M, int64_t K, const uint8_t* a_scale_swizzled,
                        const uint8_t* weight, int64_t N, const int8_t* weight_exponent, int weight_scale_e8m0,
                        const void* bias, int bias_dtype, void* out, hipStream_t stream);

/* Fused MLP, C = 64 -> H = 256 -> C = 64 rows of x [P, C] (hidden layer quantized into LDS, never written out).
 * kind 0 INT8 (x_scale, h_scale FP32 scalars; w1_scale FP32 [H], w2_scale FP32 [C]), 1 MXFP8 (x_scale int8 [C/32],
 * w1_scale int8 [H, C/32], h_scale int8 [H/32], w2_scale int8 [C, H/32]). w1 [H, C], w2 [C, H]; out BF16 [P, C].
 * semantics 1 (MXFP8, b2 and residual null) replaces ops.mxfp8_gelu_mlp (flashim/ops/gemm.py:146-157):
 *   bf16(quantize_static(bf16(gelu(bf16(x W1^T) + b1)), h) W2^T).
 * semantics 0 is the conv-refiner block's pointwise pair, identical to fim_int8_conv2d / fim_mxfp8_conv2d 1x1 with
 * (b1, GELU, quantized output h_scale) followed by 1x1 with (b2, + residual BF16 [P, C]): the two launches it
 * replaces (flashim/ops/conv.py:174-206, 309-342; quant/methods/conv2d.py:102-125). 99 for any other C or H. */
int fim_refiner_mlp(int kind, int semantics, const uint8_t* x, int64_t P, int64_t C, int64_t H, const void* x_scale,
                    const uint8_t* w1, const void* w1_scale, const void* b1, int b1_dtype, const void* h_scale,
                    const uint8_t* w2, const void* w2_scale, const void* b2, int b2_dtype, const uint16_t* residual,
                    uint16_t* out, hipStream_t stream);

/* The first conv of a VGG encoder with its epilogue: quantize_int8(relu(bf16(conv3x3(x)) + bias)), stride 1,
 * padding 1. x BF16 NCHW [B, Cin, H, W], Cin <= 8; w_packed BF16 [Cout, KP], KP = 32 ceil(9 Cin / 32), tap
 * k = 9 c + 3 ky + kx (the [Cout, Cin, 3, 3] weight flattened) and zero beyond 9 Cin; Cout a power of two in
 * [16, 128]; bias [Cout] (bias_dtype 1 BF16: the sum rounds to BF16; 0 FP32: it does not); scale FP32 scalar;
 * out INT8 NHWC [B, H, W, Cout]. Replaces ops.conv2d_small_cin_quantize_int8 (flashim/ops/conv.py:225-235). */
int fim_conv3x3_small_cin_quantize_int8(const uint16_t* x, int64_t B, int64_t Cin, int64_t H, int64_t W,
                                        const uint16_t* w_packed, int64_t Cout, const void* bias, int bias_dtype,
                                        const float* scale, int8_t* out, hipStream_t stream);

/* quantize_int8(relu(raw + bias)) of a bias-free conv output: raw BF16 NCHW [B, C, H, W] -> INT8 NHWC [B, H, W, C];
 * bias [C] BF16 (bias_dtype 1) or FP32 (0), scale FP32 scalar. Replaces ops.bias_relu_quantize_int8
 * (flashim/ops/quantize.py:134-142). */
int fim_bias_relu_quantize_int8(const uint16_t* raw, int64_t B, int64_t C, int64_t H, int64_t W, const void* bias,
                                int bias_dtype, const float* scale, int8_t* out, hipStream_t stream);

/* im2col of a 1-byte NHWC tensor: out [B*Ho*Wo, kh*kw*C] in (ky, kx, c) order with zero padding. Replaces
 * ops.im2col_gather (flashim/ops/conv.py:144-168). */
int fim_im2col_gather(const uint8_t* x, int64_t B, int64_t H, int64_t W, int64_t C, int kh, int kw, int sh, int sw,
                      int ph, int pw, int dh, int dw, uint8_t* out, hipStream_t stream);

/* ---- depthwise 5x5 producers -------------------------------------------------------------------------------- */

/* Depthwise 5x5, pad 2: x BF16 NHWC [B, H, W, C] (channels-last [B, C, H, W]), weight BF16 [25, C] (ky, kx major),
 * bias [C] FP32 (bias_dtype 0) or BF16 (1), C % 32 == 0. act 0: relu(conv + bias) in FP32; act 1: gelu(bf16(conv + bias)) rounded to BF16.
 * out_mode 0: dynamic per-(pixel, 32) MXFP8, E4M3 out [B*H*W, C] + exponent_out [B*H*W, C/32] and/or the swizzled
 * E8M0 bytes (either may be NULL); 1: static INT8 of the BF16-rounded value with *scale; 2: BF16 out;
 * 3: static MXFP8 with exponent [C/32]. act 0 + mode 0 replaces ops.depthwise5x5_relu_mxfp8 (flashim/ops/conv.py:30-44),
 * act 0 + mode 1 replaces ops.depthwise5x5_relu_int8 (flashim/ops/conv.py:50-61; the CUDA launcher it mirrors is
 * launch_dw5x5_relu_int8, flashim/backends/cuda/csrc/depthwise.cu:407-412). */
int fim_depthwise5x5(const uint16_t* x, int64_t B, int64_t H, int64_t W, int64_t C, const uint16_t* weight,
                     const void* bias, int bias_dtype, int act, int out_mode, const float* scale,
                     const int8_t* exponent, void* out, int8_t* exponent_out, uint8_t* swizzled, hipStream_t stream);

/* The MXFP8 depthwise-then-pointwise refiner block in one kernel, for C = 128 and a 128 x 128 pointwise weight (the
 * reference's fused shape; other shapes return 99 and take the two-launch composite). Replaces the fused Triton kernel
 * _dw5x5_relu_mx_pointwise_kernel (flashim/backends/triton/conv.py:310-420) behind
 * ops.depthwise5x5_relu_pointwise_mxfp8 (flashim/ops/conv.py:93-117); bit for bit the composite (fim_depthwise5x5 then
 * fim_mxfp8_scaled_mm). x BF16 NHWC [B, H, W, 128] (16-byte aligned); dw_weight BF16 [25, 128]; dw_bias [128] FP32
 * (dw_bias_dtype 0) or BF16 (1);
 * pw_weight [128 (n), 128 (k)] E4M3; pw_scale_e8m0 [128, 4] E8M0 bytes; pw_bias [128] FP32 or BF16 (dtype code as
 * fim_int8_linear) or NULL; out BF16 NHWC [B, H, W, 128] (16-byte aligned). */
int fim_depthwise5x5_relu_pointwise_mxfp8(const uint16_t* x, int64_t B, int64_t H, int64_t W, int64_t C,
                                          const uint16_t* dw_weight, const void* dw_bias, int dw_bias_dtype,
                                          const uint8_t* pw_weight, int64_t N, const uint8_t* pw_scale_e8m0,
                                          const void* pw_bias, int pw_bias_dtype, uint16_t* out, hipStream_t stream);

/* The INT8 depthwise-then-pointwise refiner block in one kernel at C = N = 128: _dw5x5_relu_int8_pointwise_kernel
 * (flashim/backends/triton/conv.py:417-475, registered at :585-599) behind ops.depthwise5x5_relu_pointwise_int8
 * (flashim/ops/conv.py:119-138); bit for bit the composite (fim_depthwise5x5 with the INT8 output, then
 * fim_int8_linear). act_scale: the static activation scale (one FP32, device); pw_weight INT8 [128 (n), 128 (k)];
 * pw_wscale FP32 [128]; other operands as fim_depthwise5x5_relu_pointwise_mxfp8. */
int fim_depthwise5x5_relu_pointwise_int8(const uint16_t* x, int64_t B, int64_t H, int64_t W, int64_t C,
                                         const uint16_t* dw_weight, const void* dw_bias, int dw_bias_dtype,
                                         const float* act_scale, const int8_t* pw_weight, int64_t N,
                                         const float* pw_wscale, const void* pw_bias, int pw_bias_dtype, uint16_t* out,
                                         hipStream_t stream);

/* The BF16 refiner block's pointwise GEMM: out[m, n] = bf16(sum_k x[m, k] * w[n, k] + bias[n]) with FP32 accumulation.
 * x BF16 [M, K] (16-byte aligned), weight BF16 [N, K] (16-byte aligned), bias [N] FP32 (bias_dtype 0) or BF16 (1) or
 * NULL, out BF16 [M, N]
 * (16-byte aligned); K in {32, 64, 96, 128}, N a multiple of 16 up to 128 (else 99). With fim_depthwise5x5 (act 0, out_mode 2) it
 * replaces the fused BF16 block behind ops.depthwise5x5_relu_pointwise (flashim/ops/conv.py:67-84; the CUDA launcher
 * it stands for is launch_depthwise5x5_relu_pointwise, flashim/backends/cuda/conv.py:194-209). */
int fim_pointwise_bf16(const uint16_t* x, int64_t M, int64_t K, const uint16_t* weight, int64_t N, const void* bias,
                       int bias_dtype, uint16_t* out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHIM_AMD_H */
