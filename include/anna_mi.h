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
/* sha256 (hex) of the csrc/ and include/ files the library was built from; no
 * counterpart in the reference (provenance of the shipped binary). */
const char* anna_mi_source_hash(void);

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


/* ------------------------------------------------------------------ TurboQuant
 * Value format (reference quantize_turboquant_values, src/anna/model/turboquant.py:157-252):
 *   data uint8 [rows, D*sb/8] (sb = 2 for 2-bit, 4 for 3/4-bit; element i at bits
 *   sb*(i % (8/sb)) of byte i/(8/sb)), scales/zeros [rows, D/group] in the value dtype.
 * TQ-MSE format (this build's definition of the third-party TurboQuantMSE the reference
 *   calls at turboquant.py:75-82; the package is absent): y = R x, code_i = #{j : y_i >=
 *   thr_j * |x|}, norm |x| as fp16 bits, codes packed like the values; reconstruction
 *   |x| * R^T c[code]. */

/* Seeded rotation R (fp32 [D, D] row-major, host memory, y = R x): the randomized Hadamard
 * H diag(s) / sqrt(D) (signs of anna_mi_tq_hadamard_signs) for power-of-two D, a seeded Haar
 * matrix otherwise.  Replaces TurboQuantMSE(dim, bits, seed=42)'s rotation (turboquant.py:80). */
int anna_mi_tq_rotation(int64_t D, uint64_t seed, float* out_host);

/* Codebook of the MSE quantizer: 2^bits ascending centroids (Gaussian Lloyd-Max levels
 * scaled by 1/sqrt(D); the 2-bit pair is fp16-structured, see turboquant.hip) and the
 * 2^bits - 1 midpoint thresholds, host memory. */
/* Sign vector s (fp32 +-1, host) of the randomized Hadamard rotation R = H diag(s) / sqrt(D)
 * used by TQ-MSE for power-of-two head_dim: s_i = -1 where bit i % 64 of the (i / 64)-th
 * splitmix64 output of `seed` is set.  Stands in for the rotation of the absent `turboquant`
 * package's TurboQuantMSE (turboquant.py:75-82). */
int anna_mi_tq_hadamard_signs(int64_t D, uint64_t seed, float* out);

/* TQ-MSE quantize with the Hadamard rotation (D a power of two in [64, 1024]): codes and fp16
 * norms as anna_mi_tq_mse_quantize, computed by an in-register fast Walsh-Hadamard transform
 * (O(D log D) per vector instead of the dense D x D product).  signs, thresholds: device. */
int anna_mi_tq_hadamard_quantize(const void* x, int x_dtype, int64_t nvec, int64_t D, int64_t x_row_stride,
                                 const float* signs, const float* thresholds, int bits, uint8_t* codes,
                                 uint16_t* norms, void* stream);

int anna_mi_tq_codebook(int bits, int64_t D, float* centroids_host, float* thresholds_host);

/* MSE quantizer (the quantize step of TurboQuantTensorRow.append, turboquant.py:382-394):
 * x [nvec, D] (row stride x_row_stride) -> codes uint8 [nvec, D*sb/8], norms fp16 bits
 * [nvec].  rot_t = R^T (fp32 [D, D], device), thresholds fp32 (device). */
int anna_mi_tq_mse_quantize(const void* x, int x_dtype, int64_t nvec, int64_t D, int64_t x_row_stride,
                            const float* rot_t, const float* thresholds, int bits, uint8_t* codes,
                            uint16_t* norms, void* stream);

/* MSE reconstruction (TurboQuantTensorRow.materialize, turboquant.py:401-431):
 * out [nvec, D] (row stride out_row_stride, out_dtype) = norm * R^T c[codes].  rot = R. */
int anna_mi_tq_mse_dequant(const uint8_t* codes, const uint16_t* norms, int64_t nvec, int64_t D,
                           const float* rot, const float* centroids, int bits, void* out, int out_dtype,
                           int64_t out_row_stride, void* stream);

/* TurboQuant inner-product keys (TurboQuant_prod: MSE stage of bits-1 bits + 1-bit QJL sketch of
 * its residual), this build's definition of the absent package's TurboQuantIP that the reference
 * calls in _quantize_turboquant_keys / dequantize_turboquant_keys / turboquant_key_attention_scores
 * (src/anna/model/turboquant.py:84-92, 255-332).  D a power of two in [64, 1024].  State per vector:
 * mse_indices uint8 [D] (one code per byte), qjl_signs uint8 [D] (0/1), norms fp32, residual_norms
 * fp32 (|residual| / norm).  signs: the Hadamard sign vector (anna_mi_tq_hadamard_signs);
 * thresholds / centroids: anna_mi_tq_codebook(bits - 1, D); gaussian / gaussian_t: the QJL matrix G
 * of anna_mi_tq_ip_gaussian and its transpose, device fp32 [D, D]. */

/* G (fp32 [D, D] row-major, host): standard normals (splitmix64 + Box-Muller in fp64) of `seed`.
 * The reference's quantizer.S is G R (R the Hadamard rotation). */
int anna_mi_tq_ip_gaussian(int64_t D, uint64_t seed, float* out_host);

/* TurboQuantIP.quantize (turboquant.py:262-264): x [nvec, D] (row stride x_row_stride, bf16/f16/
 * f32) -> mse_indices, qjl_signs [nvec, D], norms, residual_norms [nvec]. */
int anna_mi_tq_ip_quantize(const void* x, int x_dtype, int64_t nvec, int64_t D, int64_t x_row_stride,
                           const float* signs, const float* thresholds, const float* centroids,
                           const float* gaussian_t, int bits, uint8_t* mse_indices, uint8_t* qjl_signs,
                           float* norms, float* residual_norms, void* stream);

/* TurboQuantIP.dequantize (dequantize_turboquant_keys, turboquant.py:275-287): out [nvec, D]
 * (row stride out_row_stride, out_dtype) = norm * R^T (c[idx] + sqrt(pi/2)/D * rn * G^T (2 qjl - 1)). */
int anna_mi_tq_ip_dequant(const uint8_t* mse_indices, const uint8_t* qjl_signs, const float* norms,
                          const float* residual_norms, int64_t nvec, int64_t D, const float* signs,
                          const float* centroids, const float* gaussian, int bits, void* out, int out_dtype,
                          int64_t out_row_stride, void* stream);

/* turboquant_key_attention_scores (turboquant.py:290-332): query [Hq, Lq, D] (strides q_stride_h,
 * q_stride_l, 1), key state [Hkv, T, D] / [Hkv, T] -> out fp32 [Hkv, Hq/Hkv, Lq, T] = scaling *
 * (MSE scores + QJL scores), without expanding the keys.  workspace: fp32 [2 * Hq * Lq * D]. */
int anna_mi_tq_ip_scores(const void* query, int q_dtype, int64_t Hq, int64_t Lq, int64_t D,
                         int64_t q_stride_h, int64_t q_stride_l, const uint8_t* mse_indices,
                         const uint8_t* qjl_signs, const float* norms, const float* residual_norms,
                         int64_t Hkv, int64_t T, const float* signs, const float* centroids,
                         const float* gaussian_t, int bits, float scaling, float* workspace, float* out,
                         void* stream);

/* quantize_turboquant_values + _pack_value_data (turboquant.py:164-175, 199-230):
 * values [H, T, D] with strides (stride_h, stride_t, 1) -> data/scales/zeros (contiguous). */
int anna_mi_tq_values_quantize(const void* values, int dtype, int64_t H, int64_t T, int64_t D,
                               int64_t stride_h, int64_t stride_t, int bits, int64_t group_size,
                               uint8_t* data, void* scales, void* zeros, void* stream);

/* dequantize_turboquant_values (turboquant.py:233-252): out [rows, D] = q * scale + zero. */
int anna_mi_tq_values_dequant(const uint8_t* data, const void* scales, const void* zeros, int dtype,
                              int64_t rows, int64_t D, int bits, int64_t group_size, void* out,
                              int out_dtype, void* stream);

/* ------------------------------------------------------------------ split-KV GQA decode */

/* A strided view; strides in elements. */
typedef struct {
  const void* ptr;
  int64_t s0, s1, s2, s3;
} anna_mi_view;

#define ANNA_MI_KEYS_DENSE 0
#define ANNA_MI_KEYS_TQ_MSE 1
#define ANNA_MI_VALUES_DENSE 0
#define ANNA_MI_VALUES_MINMAX 1
#define ANNA_MI_VALUES_TQ_MSE 2
#define ANNA_MI_GATE_NONE 0
#define ANNA_MI_GATE_FLAT 1  /* [B, 1, Hq*D]: s0 batch, s2 inner */
#define ANNA_MI_GATE_HEADS 2 /* [B, Hq, 1, D]: s0, s1, s3 */

typedef struct {
  int dtype; /* query, dense keys/values, value scales/zeros, residual, gate, output */
  int64_t batch, q_heads, kv_heads, head_dim;
  anna_mi_view query; /* [B, Hq, 1, D] */
  /* main segment of `len1` tokens (the quantized prefix, or every token) */
  int64_t len1;
  int key_format;          /* ANNA_MI_KEYS_* */
  anna_mi_view key;        /* dense [B, Hkv, len1, D] | MSE codes uint8 [B, Hkv, len1, bytes] */
  anna_mi_view key_norms;  /* MSE: fp16 bits [B, Hkv, len1] (s0, s1, s2) */
  int key_bits;
  int value_format;        /* ANNA_MI_VALUES_* */
  anna_mi_view value;      /* dense [B, Hkv, len1, D] | packed uint8 [B, Hkv, len1, bytes] */
  anna_mi_view value_scales; /* MINMAX: [B, Hkv, len1, groups]; MSE: norms fp16 bits [B, Hkv, len1] */
  anna_mi_view value_zeros;  /* MINMAX: [B, Hkv, len1, groups] */
  int value_bits;
  int64_t value_group_size;
  const float* rotation;   /* MSE formats: R and R^T (fp32 [D, D]) and the centroids */
  const float* rotation_t;
  const float* key_centroids;
  const float* value_centroids;
  float* query_rot;        /* MSE keys: workspace fp32 [B, Hq, D] */
  /* residual segment of `len2` dense tokens (may be 0) */
  int64_t len2;
  anna_mi_view residual_key, residual_value; /* [B, Hkv, len2, D] */
  float scaling;
  int64_t block_size;
  int gate_layout;         /* ANNA_MI_GATE_* */
  anna_mi_view gate;
  anna_mi_view out;        /* [B, Hq, 1, D] */
  anna_mi_view partial_stats;  /* fp32 [B, Hq, capacity, 2] */
  anna_mi_view partial_values; /* fp32 [B, Hq, capacity, D] */
  int64_t partial_capacity;
  /* Optional (NULL: every row holds len1 + len2 tokens).  Per-row token counts, device int32
   * [B]: row b holds n = seq_lengths[b] tokens, the newest min(n, len2) in the residual segment
   * (its first positions, in any order: a ring of capacity len2) and the min(max(n - len2, 0),
   * len1) before them in the main segment; len1 and len2 are then the segments' capacities.  The
   * batched form of the reference's per-row decode loop (ops.py:1055-1071). */
  const int32_t* seq_lengths;
  /* Optional (NULL: the dense rotation_t is used).  MSE keys with the randomized Hadamard
   * rotation R = H diag(s) / sqrt(D) (power-of-two D in [64, 1024]): the sign vector s, device
   * fp32 [D]; the query is then rotated by a fast Walsh-Hadamard transform, one wave per query,
   * instead of the D x D product. */
  const float* rotation_signs;
} anna_mi_decode_args;

/* sizeof(anna_mi_decode_args), so that bindings can check their struct layout. */
int64_t anna_mi_sizeof_decode_args(void);

/* Number of split blocks a call uses (the workspace must hold at least this many):
 * ceil(L / eb) with eb = min(max(block_size, 16), L) as in the reference
 * (sycl:1521-1556); with TQ-MSE keys or values the two segments are split separately. */
int64_t anna_mi_decode_num_blocks(const anna_mi_decode_args* args);

/* Single-token GQA decode over [main segment ++ residual], flash-decoding in two kernels
 * (per-block online softmax partials, then log-sum-exp merge, optional sigmoid gate).
 * With dense values and keys this is gqa_decode_splitkv_fused_out (schema sycl:7640-7651,
 * launch sycl:4494-4706); with min/max-packed values it is
 * gqa_decode_splitkv_turboquant_fused_out (schema sycl:7652-7668, launch sycl:4771-5094).
 * All q-heads of a KV group share one workgroup and one read of each K/V token. */
int anna_mi_gqa_decode_splitkv(const anna_mi_decode_args* args, void* stream);

/* Allocation-free form of anna_mi_gqa_decode_splitkv.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The partial_stats, partial_values,
 * partial_capacity and query_rot fields of args are ignored; that workspace lives in a static
 * device array of anna_mi_gqa_decode_splitkv_noalloc_capacity() bytes (32 MiB) per GPU, held
 * until the process ends.  The call fails with ANNA_MI_EINVAL when the workspace does not
 * fit: 4 * (up(B*Hq*nblk*2) + up(B*Hq*nblk*D) + up(B*Hq*D)) bytes, up(n) = n rounded up to a
 * multiple of 64 (each part 256-byte aligned), nblk = anna_mi_decode_num_blocks, the last term
 * only for TQ-MSE keys.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU race.  It
 * allocates nothing and launches the same kernels, so results equal anna_mi_gqa_decode_splitkv's. */
int anna_mi_gqa_decode_splitkv_noalloc(const anna_mi_decode_args* args, void* stream);
int64_t anna_mi_gqa_decode_splitkv_noalloc_capacity(void);

/* ------------------------------------------------------------------ batched TQ decode
 * Batched, variable-length single-token GQA decode over a 2-bit TQ-MSE K/V cache
 * (head_dim 256, Hadamard rotation): the batched replacement of the per-row loop of
 * Qwen3DynamicCache.turboquant_single_token_decode_attention (src/anna/model/ops.py:1024-1072)
 * over TurboQuantKVRow.decode_attention (turboquant.py:1181-1346), and of the per-row append of
 * _update_turboquant_layer (ops.py:618-661) over TurboQuantKVRow.append (turboquant.py:1027-1140).
 *
 * Cache per KV head: a pool of token slots (sequence b owns pool slots seq_offsets[b] ..
 * + its capacity, offsets multiples of 32) holding the quantized prefix, and per sequence a
 * ring of R dense bf16 tokens holding the newest min(length, R) tokens (token j at ring slot
 * j % R).  seq_lengths[b] (device) is the total token count; the quantized prefix is
 * max(0, length - R) tokens.  Layout details: tq_decode.hip. */
typedef struct {
  int64_t batch, q_heads, kv_heads, head_dim;
  int key_bits, value_bits;         /* 2, 2 */
  const uint16_t* query;            /* bf16 [B][Hq][D] */
  const uint16_t* gate;             /* bf16 [B][Hq][D] or NULL: out *= sigmoid(gate) */
  const uint8_t* key_codes;         /* [Hkv][pool][D/4] */
  const uint16_t* key_norms;        /* fp16 [Hkv][pool] */
  const uint8_t* value_codes;       /* [Hkv][pool/32][32*D/4] blocked */
  const uint16_t* value_norms;      /* fp16 [Hkv][pool] */
  int64_t pool_tokens;
  const uint16_t* residual_key;     /* bf16 [B][Hkv][R][D] ring */
  const uint16_t* residual_value_t; /* bf16 [B][Hkv][D][R] ring */
  int64_t residual_capacity;        /* R, multiple of 32 */
  const int32_t* seq_offsets;       /* device [B] */
  const int32_t* seq_lengths;       /* device [B] */
  const float* signs;               /* device [D]: the rotation's sign vector */
  float key_scale, value_scale;     /* centroid c = key_scale * fp16 LUT value */
  float scaling;
  int64_t blocks_per_item;          /* 32-token blocks per work item; 0 = sized to fill the GPU */
  int64_t num_workgroups;           /* grid size, from anna_mi_tq_decode_workgroups */
  float* partial_stats;             /* workspace [num_workgroups][16][2] */
  float* partial_values;            /* workspace, sized as float [num_workgroups][16][D] (internal layout) */
  int32_t* item_table;              /* workspace [2*B*Hkv] int32, [4*B*Hkv] for anna_mi_tq_append_decode
                                       (the split tells the merge its items) */
  uint16_t* out;                    /* bf16 [B][Hq][D] */
} anna_mi_tq_decode_args;

/* Grid size (workgroups) of anna_mi_tq_decode for sequences of at most pool_capacity[b]
 * quantized tokens (host array): B*Hkv window workgroups plus enough work-item workgroups for
 * any lengths up to those capacities. */
int64_t anna_mi_tq_decode_workgroups(int64_t batch, int64_t kv_heads, const int64_t* pool_capacity_host,
                                     int64_t blocks_per_item);

/* Two launches: every (b, kv head) is split into work items of 32-token blocks of its
 * quantized prefix plus one window item; the split is planned on the device from seq_lengths (no
 * host round trip, capturable in a graph).  Each item rotates q itself (FWHT), scores the 2-bit
 * codes by MFMA and writes log-sum-exp partials; the merge launch (one wave per q head) merges
 * them, rotates the result back, adds the window part, applies the gate and writes bf16.
 * Sequences of length 0 give zeros.  Calls that share workspaces must not overlap. */
int anna_mi_tq_decode(const anna_mi_tq_decode_args* args, void* stream);

typedef struct {
  int64_t batch, kv_heads, head_dim;
  const uint16_t* new_key;          /* bf16 [B][Hkv][D]: one token per sequence */
  const uint16_t* new_value;        /* bf16 [B][Hkv][D] */
  uint8_t* key_codes;               /* pool, as anna_mi_tq_decode_args */
  uint16_t* key_norms;
  uint8_t* value_codes;
  uint16_t* value_norms;
  int64_t pool_tokens;
  uint16_t* residual_key;           /* ring, as anna_mi_tq_decode_args */
  uint16_t* residual_value_t;
  int64_t residual_capacity;
  const int32_t* seq_offsets;       /* device [B] */
  const int32_t* seq_capacity;      /* device [B]: pool slots of each sequence */
  int32_t* seq_lengths;             /* device [B], incremented by one */
  int32_t* overflow;                /* device int32 or NULL: set to 1 when a sequence had no pool slot left */
  const float* signs;               /* device [D] */
  const float* thresholds;          /* device [3]: the 2-bit codebook's thresholds */
} anna_mi_tq_append_args;

/* Appends one token per sequence for all sequences in one launch: the token leaving the ring
 * (when length >= R) is quantized into the pool (key codes + norm, value codes in the 32-token
 * blocked layout + norm, bit-exact with anna_mi_tq_hadamard_quantize), the new token takes its
 * ring slot, and seq_lengths[b] grows by one. */
int anna_mi_tq_append(const anna_mi_tq_append_args* args, void* stream);

/* One decode step in two launches: the append above and the decode of anna_mi_tq_decode, with
 * the same results and the same cache state afterwards (pool codes, ring, lengths, overflow) as
 * anna_mi_tq_append followed by anna_mi_tq_decode, without the append's launch.  The split
 * launch plans on the lengths before the append; the window workgroup of each (b, kv head)
 * quantizes the token leaving its ring into the pool slot just past the planned items and
 * leaves that slot out of its window; the merge launch scores the leaving token (from its codes)
 * and the new one itself, then writes the new token into the ring and the new length.  Both
 * argument blocks must describe the one cache (checked); args->item_table holds 4 * batch *
 * kv_heads entries.  Replaces the pair of calls the reference makes per step and layer,
 * Qwen3DynamicCache._update_turboquant_layer (ops.py:618-661) and the decode (ops.py:1055-1071);
 * no single reference function does both. */
int anna_mi_tq_append_decode(const anna_mi_tq_decode_args* args, const anna_mi_tq_append_args* append,
                             void* stream);

/* The general batched cache (one region per sequence and KV head; any power-of-two head_dim in
 * [64, 1024], key bits 1..4, value bits 2..4): one token per sequence, the form of
 * Qwen3DynamicCache._update_turboquant_layer looping TurboQuantKVRow.append (ops.py:618-661,
 * turboquant.py:1027-1140) in one launch.  The token leaving the bf16 window (ring slot n % R)
 * is quantized into packed slot n - R: keys as Hadamard TQ-MSE codes + fp16 norm (as
 * anna_mi_tq_hadamard_quantize), values as min/max groups (as anna_mi_tq_values_quantize,
 * turboquant.py:199-230); the new token takes the ring slot and the length grows by one.  A
 * sequence whose packed region is full is left unchanged and sets *overflow.  Decode with
 * anna_mi_gqa_decode_splitkv and seq_lengths. */
typedef struct {
  int dtype; /* new tokens, ring, value scales/zeros */
  int64_t batch, kv_heads, head_dim;
  int64_t capacity;          /* packed slots per (sequence, KV head) */
  int64_t residual_capacity; /* R, ring slots per (sequence, KV head) */
  int key_bits, value_bits;
  int64_t value_group_size;
  const void* new_key;       /* [B, Hkv, D] contiguous */
  const void* new_value;
  uint8_t* key_codes;        /* [B, Hkv, capacity, D * sbits / 8] (sbits = 2 for 2-bit codes, else 4) */
  uint16_t* key_norms;       /* fp16 [B, Hkv, capacity] */
  uint8_t* value_data;       /* [B, Hkv, capacity, D * sbits / 8] */
  void* value_scales;        /* [B, Hkv, capacity, D / group] */
  void* value_zeros;
  void* residual_key;        /* [B, Hkv, R, D], token j of a sequence at slot j % R */
  void* residual_value;
  int32_t* seq_lengths;      /* device [B] */
  int32_t* overflow;         /* device, set to 1 when a sequence is full */
  const float* signs;        /* Hadamard signs [D] */
  const float* thresholds;   /* key codebook thresholds [2^key_bits - 1] */
} anna_mi_tq_rows_append_args;

int64_t anna_mi_sizeof_tq_rows_append_args(void);
int anna_mi_tq_rows_append(const anna_mi_tq_rows_append_args* args, void* stream);

typedef struct {
  int64_t kv_heads, head_dim, tokens;
  const uint16_t* keys;             /* bf16, element (h, t, d) at h * stride_head + t * stride_token + d */
  const uint16_t* values;           /* bf16, same strides */
  int64_t stride_head, stride_token;
  uint8_t* key_codes;               /* pool, as anna_mi_tq_decode_args */
  uint16_t* key_norms;
  uint8_t* value_codes;
  uint16_t* value_norms;
  int64_t pool_tokens;
  int64_t slot_offset;              /* first pool slot written (multiple of 32) */
  const float* signs;               /* device [D] */
  const float* thresholds;          /* device [3] */
} anna_mi_tq_pack_args;

/* Packs `tokens` tokens of K and V of every KV head into pool slots slot_offset .. + tokens in
 * one launch: Hadamard TQ-MSE codes (bit-exact with anna_mi_tq_hadamard_quantize), key codes
 * token-major, value codes in the 32-token blocked layout, fp16 norms.  The bulk (prefill)
 * counterpart of the per-token quantization in TurboQuantKVRow.append (turboquant.py:1027-1140)
 * and of TurboQuantTensorRow.append (turboquant.py:335-477) for BASELINE config 3. */
int anna_mi_tq_pack_kv(const anna_mi_tq_pack_args* args, void* stream);
int64_t anna_mi_sizeof_tq_pack_args(void);

/* Reorders natural 2-bit codes [tokens][64] (D = 256) of one KV head into the blocked value
 * layout [tokens/32][2048] read by anna_mi_tq_decode (tokens % 32 == 0).  Pure permutation. */
int anna_mi_tq_block_values(const uint8_t* codes, int64_t tokens, uint8_t* blocked, void* stream);

/* sizeof(anna_mi_tq_decode_args), for binding checks. */
int64_t anna_mi_sizeof_tq_decode_args(void);
int64_t anna_mi_sizeof_tq_append_args(void);

/* ------------------------------------------------------------------ tiled int4 GEMV, LM-head top-k */

/* xpu_int4_gemv_tiled (sycl:3272-3343; layout quantization.py:491-538): qweight int32
 * [tiles][packed_cols][tile] (tile 1, 2, 4 or 8; row n = tile*t_idx + t, word w at
 * [n / tile][w][n % tile]; tile 1 is the plain [N][Kp/8] layout); the scale / zero point of
 * (group g, row n) sits at g * scale_stride_group + n * scale_stride_row ([G][N] or [G][N/T][T]:
 * (N, 1); the LM-head top-k layout [N][G]: (1, G)).  y [M][N] (row stride given) is fp32 when
 * y_is_f32, else in the activation dtype. */
int anna_mi_int4_gemv_tiled(const void* x, int x_dtype, int64_t M, int64_t K, int64_t x_row_stride,
                            const int32_t* qweight, int64_t tiles, int64_t packed_cols, int64_t tile,
                            const void* qscale, int scale_dtype, const int8_t* qzeros, int64_t group_count,
                            int64_t scale_stride_group, int64_t scale_stride_row, int64_t group_size, int64_t N,
                            void* y, int y_is_f32, int64_t y_row_stride, void* stream);

/* Top-k of each row of fp32 values [rows][ld] (first V columns): values (in out_dtype) and
 * int64 indices [rows][top_k], descending, ties to the lower index.  top_k <= 32. */
int anna_mi_topk_rows(const float* values, int64_t rows, int64_t V, int64_t ld, int64_t top_k, void* out_values,
                      int out_dtype, int64_t* out_indices, void* stream);

/* lm_head_int4_topk_fused (sycl:2137-2572; caller qwen3_5_text_model.py:65-110): fp32 logits of
 * the int4 LM head into the workspace `logits` [rows][vocab], then their top-k (values in the
 * activation dtype).  `logits` is scratch: for few long rows the top-k writes its partial lists
 * over it, so it does not hold the logits afterwards. */
int anna_mi_lm_head_int4_topk(const void* x, int x_dtype, int64_t rows, int64_t K, int64_t x_row_stride,
                              const int32_t* qweight, int64_t tiles, int64_t packed_cols, int64_t tile,
                              const void* qscale, int scale_dtype, const int8_t* qzeros, int64_t group_count,
                              int64_t scale_stride_group, int64_t scale_stride_row, int64_t group_size, int64_t vocab,
                              int64_t top_k, float* logits, void* values, int64_t* indices, void* stream);

/* ------------------------------------------------------------------ MoE
 * Routing around the grouped expert MLP (Qwen3SparseMoeBlock, src/anna/model/ops.py:3280-3376). */

/* moe_router_fused (sycl:3731-3839; CPU path ops.py:3280-3299): per token, fp32 softmax over the
 * experts, top-k (ties: lower expert index first), renormalised when `normalize`; usage[e]
 * counts the routes of expert e (zeroed by the call).  logits [tokens][num_experts] (row
 * stride given), weights fp32 [tokens][top_k], selected int64 [tokens][top_k], usage int32
 * [num_experts].  num_experts <= 1024, top_k <= 64. */
int anna_mi_moe_router(const void* logits, int logits_dtype, int64_t tokens, int64_t num_experts,
                       int64_t logits_row_stride, int64_t top_k, int normalize, float* weights,
                       int64_t* selected, int32_t* usage, void* stream);

/* moe_dispatch_fused (sycl:3867-3965; CPU path ops.py:3301-3357): expert_offsets int64 [E+1]
 * (prefix sum of usage, int32 or int64), routes sorted by (expert, token, k) -- the CPU
 * path's order, deterministic: sorted_token_idx / sorted_route_idx int64 [tokens*top_k];
 * compact_hidden [routes][hidden] and compact_weights [routes] in the hidden dtype
 * (routing_weights [tokens][top_k] contiguous, dtype weights_dtype: the router's fp32 weights
 * are rounded to the hidden dtype here, as the reference's cast does).  route_pos (optional,
 * may be NULL) receives the compact position of route t*top_k + j.  items and slots (optional,
 * both or neither): the grouped MLP's list of experts with routes (see
 * anna_mi_moe_mlp_args.items) for bank slots slots[e] [E], written here so that the MLP can
 * take it prefilled. */
int anna_mi_moe_dispatch(const void* hidden, int dtype, int64_t tokens, int64_t hidden_dim,
                         int64_t hidden_row_stride, const void* routing_weights, int weights_dtype,
                         const int64_t* selected,
                         const void* usage, int usage_is_int64, int64_t num_experts, int64_t top_k,
                         int64_t* sorted_token_idx, int64_t* sorted_route_idx, int64_t* expert_offsets,
                         void* compact_hidden, void* compact_weights, int64_t* route_pos, const int64_t* slots,
                         int32_t* items, void* stream);

/* No single counterpart in the reference: moe_router_fused (sycl:3731-3865) followed by the
 * ordering half of moe_dispatch_fused (sycl:3867-3965), for small batches (tokens * top_k <=
 * 1024, num_experts <= 512), in one launch.  Outputs are those of anna_mi_moe_router
 * (weights, selected, usage as int32) and of the dispatch's ordering (expert_offsets [E+1],
 * sorted_token_idx, sorted_route_idx, route_pos [tokens*top_k]), identical to them, plus
 * items (int32 [4 + 4 E], the list the grouped MLP walks: see anna_mi_moe_mlp_args.items) with
 * bank slot slots[e] for expert e.  For callers such as an MoE block that run the whole chain. */
int anna_mi_moe_route_small(const void* logits, int logits_dtype, int64_t tokens, int64_t num_experts,
                            int64_t logits_row_stride, int64_t top_k, int normalize, float* weights,
                            int64_t* selected, int32_t* usage, int64_t* expert_offsets, int64_t* sorted_token_idx,
                            int64_t* sorted_route_idx, int64_t* route_pos, const int64_t* slots, int32_t* items,
                            void* stream);

/* The gathering half of moe_dispatch_fused (sycl:3867-3965): compact_hidden[p] =
 * hidden[sorted_route_idx[p] / top_k], compact_weights[p] = routing_weights[sorted_route_idx[p]]
 * (rounded to the hidden dtype from weights_dtype), after anna_mi_moe_route_small. */
int anna_mi_moe_gather(const void* hidden, int dtype, int64_t hidden_dim, int64_t hidden_row_stride,
                       const void* routing_weights, int weights_dtype, const int64_t* sorted_route_idx,
                       int64_t routes, int64_t top_k,
                       void* compact_hidden, void* compact_weights, void* stream);

/* moe_scatter_fused (sycl:3967-4037; CPU path ops.py:3359-3376): out[t] = sum of the compact
 * rows p with sorted_token_idx[p] == t, accumulated in fp32 (workspace accum [tokens][hidden]
 * fp32) and cast to the hidden dtype. */
int anna_mi_moe_scatter(const void* compact_outputs, int dtype, int64_t routes, int64_t hidden_dim,
                        const int64_t* sorted_token_idx, int64_t num_tokens, float* accum, void* out,
                        void* stream);

/* Deterministic form of the scatter for callers that kept route_pos from the dispatch:
 * out[t] = sum_j compact_outputs[route_pos[t*top_k + j]] in fp32, j ascending. */
int anna_mi_moe_combine(const void* compact_outputs, int dtype, int64_t hidden_dim, const int64_t* route_pos,
                        int64_t num_tokens, int64_t top_k, void* out, void* stream);

/* moe_grouped_int4_mlp_fused (sycl:4078-4324; caller ops.py:3405-3457; bank ops.py:73-89):
 * for each active expert e (bank slot active_slots[i]) and its compact routes
 * [expert_offsets[e], expert_offsets[e+1]):
 *   act = silu(x Wg^T) * (x Wu^T) (fp32), out = (act Wd^T) * routing weight (hidden dtype).
 * Bank layout (XPUInt4Linear buffers stacked over slots): gate/up qweight int32
 * [S][I][Kh/8], qscale [S][Gh][I], qzeros int8 [S][Gh][I]; down qweight [S][H][Ki/8], qscale
 * [S][Gi][H], qzeros [S][Gi][H].  hidden and intermediate dims: multiples of 128, <= 4096. */
typedef struct {
  int dtype;                      /* hidden dtype (bf16 / fp16 / fp32) */
  int scale_dtype;                /* qscale dtype of the bank */
  int64_t routes, hidden_dim, intermediate_dim;
  const void* compact_hidden;     /* [routes][hidden] */
  const void* compact_weights;    /* [routes], hidden dtype */
  void* compact_outputs;          /* [routes][hidden], hidden dtype; rows of inactive experts untouched */
  const int64_t* expert_offsets;  /* [E+1] */
  const int64_t* active_experts;  /* [active_count] */
  const int64_t* active_slots;    /* [active_count] */
  int64_t active_count;
  const int32_t* gate_qweight;
  const void* gate_qscale;
  const int8_t* gate_qzeros;
  const int32_t* up_qweight;
  const void* up_qscale;
  const int8_t* up_qzeros;
  const int32_t* down_qweight;
  const void* down_qscale;
  const int8_t* down_qzeros;
  int64_t hidden_packed_cols, hidden_groups, intermediate_packed_cols, intermediate_groups, group_size;
  float* activation;              /* workspace, routes * intermediate fp32 elements (the act
                                     between the two products; the wide form below keeps it as
                                     bf16 in the first half) */
  int sweep_chunks;               /* 1..4: a hint, ignored.  With 16-bit hidden states, group 128,
                                     hidden and intermediate dims multiples of 256 and at least 16
                                     routes per active expert on average, one 8-wave workgroup per
                                     CU takes up to 48 routes of an expert per sweep over its
                                     weights; otherwise sweeps are 16 routes (each form measured
                                     fastest where it is taken) */
  int32_t* items;                 /* optional workspace int32 [4 + 4 * active_count]: when set, the
                                     active experts that have routes are listed on the device
                                     first and the MLP launches walk that list (no workgroups
                                     for empty experts); NULL: one workgroup per expert and tile */
  int items_prefilled;            /* 1: items already holds the list (anna_mi_moe_route_small wrote
                                     it), so it is not rebuilt */
} anna_mi_moe_mlp_args;

int64_t anna_mi_sizeof_moe_mlp_args(void);
int anna_mi_moe_grouped_int4_mlp(const anna_mi_moe_mlp_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ANNA_MI_H_ */
