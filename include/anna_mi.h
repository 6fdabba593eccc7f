/*
 * anna_mi.h -- C ABI of the MI355X (gfx950) implementation of Anna's quantized
 * decode path: group-wise int4 weight-only linear, TurboQuant KV-cache packing and
 * GQA decode attention over the packed cache.
 *
 * Conventions
 *   - Plain pointers and sizes only.  Every device pointer refers to HBM of the
 *     current HIP device; `stream` is a hipStream_t (NULL = default stream).
 *   - Calls are asynchronous on `stream` and never synchronize the host.
 *   - Return 0 on success, an ANNA_MI_E* code otherwise; anna_mi_last_error()
 *     returns the message of the last failure on the calling thread.  Argument
 *     checks happen before anything is launched.
 *   - Element strides are in elements, not bytes.
 *   - dtype codes: ANNA_MI_BF16, ANNA_MI_F16, ANNA_MI_F32.
 *
 * Each entry point names the reference interface it replaces (paths relative to
 * the funkpopo/Anna repository root; "sycl" = src/anna/model/custom_ops/
 * gated_delta_fused_op.sycl).
 */
#ifndef ANNA_MI_H_
#define ANNA_MI_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ANNA_MI_ABI_VERSION 1

#define ANNA_MI_OK 0
#define ANNA_MI_EINVAL 1 /* bad argument (shape, dtype, alignment, size) */
#define ANNA_MI_EHIP 2   /* HIP runtime error */

#define ANNA_MI_BF16 0
#define ANNA_MI_F16 1
#define ANNA_MI_F32 2

const char* anna_mi_last_error(void);
int anna_mi_abi_version(void);

/* ------------------------------------------------------------------ int4 linear
 * Weight layout (XPUInt4Linear buffers, src/anna/model/quantization.py:460-487):
 *   qweight int32 [N, Kp/8]  nibble k%8 of word k/8 at bits 4*(k%8)
 *   qscale        [G, N]     G = Kp/group_size, dtype scale_dtype (reference: fp32)
 *   qzeros  int8  [G, N]     w = (q - zero) * scale
 */

/* y[M, N] = x[M, K] * dequant(W)^T, fp32 accumulation, y in x_dtype.
 * Replaces torch.ops.anna.xpu_int4_gemv (schema sycl:7735-7743, host
 * xpu_int4_gemv_xpu sycl:3175-3270, checks sycl:1100-1130) and is the device path
 * of XPUInt4Linear.forward (quantization.py:686-710).  K = in_features <= Kp;
 * x_row_stride >= K.  M <= 16 runs the HBM-bound MFMA GEMV kernel, larger M the
 * LDS-tiled MFMA GEMM. */
int anna_mi_int4_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t x_row_stride,
                        const int32_t* qweight, int64_t N, int64_t packed_cols,
                        const void* qscale, int scale_dtype, const int8_t* qzeros,
                        int64_t group_count, int64_t group_size, void* y, void* stream);

/* w_out[N, K] = (q - zero) * scale rounded to out_dtype (the dequant strategy,
 * XPUInt4Linear._dequantize_weight, quantization.py:626-635). */
int anna_mi_int4_dequant(const int32_t* qweight, int64_t N, int64_t packed_cols,
                         const void* qscale, int scale_dtype, const int8_t* qzeros,
                         int64_t group_count, int64_t group_size, int64_t K, void* w_out,
                         int out_dtype, void* stream);

/* Symmetric int4 quantizer + packer: scale = amax/7 (1 if amax == 0),
 * q = clamp(round(w/scale + 8), 0, 15), zero = 8.  rounding 0 = half to even
 * (XPUInt4Linear._quantize_weight, quantization.py:597-624); rounding 1 = half away
 * from zero (the load-time packer quantize_linear_raw, crates/anna-rust/src/lib.rs:341-401).
 * w [N, K] of w_dtype (row stride K); Kp multiple of group_size and 8; columns K..Kp-1
 * quantize as zeros.  qscale out is fp32 [Kp/group, N], qzeros int8 [Kp/group, N]. */
int anna_mi_int4_quantize(const void* w, int w_dtype, int64_t N, int64_t K, int64_t Kp,
                          int64_t group_size, int rounding, int32_t* qweight, float* qscale,
                          int8_t* qzeros, void* stream);

/* AutoRound/GPTQ payload -> the layout above (AutoRoundGPTQLinear._to_xpu_int4_tensors,
 * quantization.py:348-375): gptq_qweight int32 [ceil(K/8), N], gptq_qzeros int32
 * [G, ceil(N/8)] storing zero-1, scales fp16 [G, N]. */
int anna_mi_autoround_to_int4(const int32_t* gptq_qweight, const int32_t* gptq_qzeros,
                              const uint16_t* scales_f16, int64_t K, int64_t N, int64_t group_size,
                              int64_t G, int64_t Kp, int32_t* qweight, float* qscale,
                              int8_t* qzeros, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ANNA_MI_H_ */
