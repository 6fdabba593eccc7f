// Batched varlen GQA decode over a 2-bit TurboQuant-MSE KV cache (head_dim 256), MFMA.
//
// Cache layout (per KV head, a pool of `pool_tokens` token slots; sequence b owns slots
// [seq_offsets[b], seq_offsets[b] + capacity), offsets multiple of 32):
//   key_codes   uint8 [Hkv][pool][64]       token-major, dim i at bits 2(i%4) of byte i/4
//   key_norms   fp16  [Hkv][pool]
//   value_codes uint8 [Hkv][pool/32][2048]  32-token blocks, byte ((t%16)/4)*512 + dim*2 + t/16,
//                                           token t at bits 2(t%4) (see tq_block_values_kernel)
//   value_norms fp16  [Hkv][pool]
//   residual_key     bf16 [B][Hkv][R][256]  newest tokens, dense, token-major
//   residual_value_t bf16 [B][Hkv][256][R]  dense, dim-major
//
// Kernels (one call = three launches):
//   tq_rotate_query  q' = R q (MFMA, fp16 in / fp32 accumulate) for every (b, q-head).
//   tq_decode_split  one workgroup per work item (b, kv-head, <= tokens_per_item tokens or the
//     residual window).  4 waves take 32-token blocks.  Scores are formed transposed,
//     S^T = Khat Q'^T, by v_mfma_f32_16x16x32_f16 on codes turned into fp16 centroids with one
//     v_perm per pair (the 2-bit centroids are fp16 values sharing their low byte); S^T's
//     accumulator layout is exactly the B operand of O'^T = Vhat^T P^T, so probabilities
//     never leave registers.  Online softmax in base 2 with lazy rescaling (the running max
//     only moves when a block exceeds it by 2^4).  Output: per item and q-head
//     (max, denominator) and the unnormalized accumulator (rotated space for packed items).
//   tq_decode_merge  per (b, kv-head): log-sum-exp merge of the items, un-rotation of the
//     packed part (Y = A R, MFMA), plus the residual part, bf16 output.
#include <vector>

#include "common.hpp"

namespace anna {
namespace {

constexpr int TD = 256;              // head_dim
constexpr int TBT = 32;              // tokens per block
constexpr int TWAVES = 4;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LAZY = 4.0f;         // rescale threshold (log2 units)
constexpr float P_SCALE = 1.0f / 64.0f;  // keeps p * norm inside fp16 range; divided out at the end
constexpr float TQ2_A16 = 1.123046875f;

__device__ __forceinline__ uint32_t vconst(uint32_t c) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 2-bit codes at bits 8+2p (low half) and 24+2p (high half) of x -> 4 fp16 pairs.
// lut_hi holds the high bytes of the fp16 centroids {-b, -a, +a, +b}; lut_lo their common
// low byte; or_c = 0x04000400 (selector offset to the lut_hi bytes).
__device__ __forceinline__ u32x4 codes_to_f16(uint32_t x, uint32_t lut_hi, uint32_t lut_lo, uint32_t or_c) {
  u32x4 r;
  r.x = __builtin_amdgcn_perm(lut_hi, lut_lo, (x & 0x03000300u) | or_c);
  r.y = __builtin_amdgcn_perm(lut_hi, lut_lo, ((x >> 2) & 0x03000300u) | or_c);
  r.z = __builtin_amdgcn_perm(lut_hi, lut_lo, ((x >> 4) & 0x03000300u) | or_c);
  r.w = __builtin_amdgcn_perm(lut_hi, lut_lo, ((x >> 6) & 0x03000300u) | or_c);
  return r;
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}

// ------------------------------------------------------------------ q' = R q

// grid (B * Hkv), 256 threads.  Q [16 heads x 256] (bf16 -> fp16) times R^T -> fp16 q'.
__global__ __launch_bounds__(256) void tq_rotate_query_kernel(const anna_mi_tq_decode_args a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t bh = blockIdx.x, b = bh / a.kv_heads, h = bh % a.kv_heads;
  const int G = (int)(a.q_heads / a.kv_heads);
  const uint16_t* q = (const uint16_t*)a.query + (b * a.q_heads + h * G) * TD;
  const uint16_t* R = (const uint16_t*)a.rotation_f16;
  u32x4 af[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < G) v = *(const u32x4*)(q + r * TD + s * 32 + kq * 8);
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      o[w] = pack_f16x2(bf16_bits_to_f32((uint16_t)(v[w] & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(v[w] >> 16)));
    af[s] = o;
  }
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int tile = wave * 4 + tt;  // output dims i in [16 tile, 16 tile + 16)
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const u32x4 bfr = *(const u32x4*)(R + (int64_t)(tile * 16 + r) * TD + s * 32 + kq * 8);
      acc = mfma_f16(af[s], bfr, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 4 * kq + i;
      if (n < G) ((uint16_t*)a.query_rot)[(b * a.q_heads + h * G + n) * TD + tile * 16 + r] = f32_to_f16_bits(acc[i]);
    }
  }
}

// ------------------------------------------------------------------ split

__global__ __launch_bounds__(64 * TWAVES) void tq_decode_split_kernel(const anna_mi_tq_decode_args a) {
  __shared__ float s_m[TWAVES][16], s_l[TWAVES][16];
  __shared__ float s_acc[16 * TD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t item = blockIdx.x;
  const int32_t* it = a.items + item * 4;
  const int64_t b = it[0], h = it[1];
  const int64_t t0 = it[2], t1 = it[3];
  const bool resid = t0 < 0;
  const int G = (int)(a.q_heads / a.kv_heads);
  const int64_t T = a.pool_tokens;
  const int64_t Rc = a.residual_capacity;
  const int64_t tb0 = resid ? 0 : t0;
  const int64_t tend = resid ? (int64_t)a.residual_lens[b] : t1;
  const int64_t nblk = (tend - tb0 + TBT - 1) / TBT;

  for (int i = threadIdx.x; i < 16 * TD; i += blockDim.x) s_acc[i] = 0.f;

  const uint32_t lut_hi = vconst(0x433CBCC3u), lut_lo = vconst(0x7E7E7E7Eu), or_c = vconst(0x04000400u);

  // B operand of S^T = Khat Q'^T for the 8 dim-steps (lane: head n = r, k-group kq).
  u32x4 qf[8];
  if (!resid) {
    const uint16_t* qr = (const uint16_t*)a.query_rot + (b * a.q_heads + h * G + r) * TD;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int da = 64 * kq + 16 * (s >> 1) + 4 * (s & 1);
      uint2 lo = {0u, 0u}, hi = {0u, 0u};
      if (r < G) {
        lo = *(const uint2*)(qr + da);
        hi = *(const uint2*)(qr + da + 8);
      }
      qf[s].x = __builtin_amdgcn_perm(hi.x, lo.x, 0x05040100u);
      qf[s].y = __builtin_amdgcn_perm(hi.x, lo.x, 0x07060302u);
      qf[s].z = __builtin_amdgcn_perm(hi.y, lo.y, 0x05040100u);
      qf[s].w = __builtin_amdgcn_perm(hi.y, lo.y, 0x07060302u);
    }
  } else {
    const uint16_t* q = (const uint16_t*)a.query + (b * a.q_heads + h * G + r) * TD;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (r < G) v = *(const u32x4*)(q + s * 32 + kq * 8);
      qf[s] = v;
    }
  }

  const float kscale = a.key_scale * a.scaling * LOG2E;
  const float vscale = a.value_scale * P_SCALE;
  f32x4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  const int64_t off = resid ? 0 : a.seq_offsets[b];
  for (int64_t blk = wave; blk < nblk; blk += TWAVES) {
    const int64_t tb = tb0 + blk * TBT;  // first token of the block
    float s[8];
    float nv[8];
    u32x4 vraw[2];
    if (!resid) {
      const int64_t p0 = off + tb;
      const uint8_t* kc = a.key_codes + (h * T + p0) * 64;
      const u32x4 k0 = *(const u32x4*)(kc + r * 64 + kq * 16);
      const u32x4 k1 = *(const u32x4*)(kc + (16 + r) * 64 + kq * 16);
      const uint16_t* kn = a.key_norms + h * T + p0;
      const uint16_t* vn = a.value_norms + h * T + p0;
      const uint2 kn0 = *(const uint2*)(kn + 4 * kq), kn1 = *(const uint2*)(kn + 16 + 4 * kq);
      const uint2 vn0 = *(const uint2*)(vn + 4 * kq), vn1 = *(const uint2*)(vn + 16 + 4 * kq);
      const uint8_t* vc = a.value_codes + (h * (T / TBT) + p0 / TBT) * 2048 + kq * 512 + r * 32;
      vraw[0] = *(const u32x4*)(vc);
      vraw[1] = *(const u32x4*)(vc + 16);
      f32x4 st0 = {0.f, 0.f, 0.f, 0.f}, st1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const uint32_t w0 = k0[st >> 1], w1 = k1[st >> 1];
        const uint32_t x0 = (st & 1) ? w0 : (w0 << 8), x1 = (st & 1) ? w1 : (w1 << 8);
        st0 = mfma_f16(codes_to_f16(x0, lut_hi, lut_lo, or_c), qf[st], st0);
        st1 = mfma_f16(codes_to_f16(x1, lut_hi, lut_lo, or_c), qf[st], st1);
      }
      const uint32_t kw[4] = {kn0.x, kn0.y, kn1.x, kn1.y};
      const uint32_t vw[4] = {vn0.x, vn0.y, vn1.x, vn1.y};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float nk0 = f16_bits_to_f32((uint16_t)(kw[i >> 1] >> (16 * (i & 1))));
        const float nk1 = f16_bits_to_f32((uint16_t)(kw[2 + (i >> 1)] >> (16 * (i & 1))));
        s[i] = st0[i] * nk0 * kscale;
        s[4 + i] = st1[i] * nk1 * kscale;
        nv[i] = f16_bits_to_f32((uint16_t)(vw[i >> 1] >> (16 * (i & 1)))) * vscale;
        nv[4 + i] = f16_bits_to_f32((uint16_t)(vw[2 + (i >> 1)] >> (16 * (i & 1)))) * vscale;
      }
    } else {
      const uint16_t* rk = a.residual_key + ((b * a.kv_heads + h) * Rc + tb) * TD;
      f32x4 st0 = {0.f, 0.f, 0.f, 0.f}, st1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const u32x4 a0 = *(const u32x4*)(rk + r * TD + st * 32 + kq * 8);
        const u32x4 a1 = *(const u32x4*)(rk + (16 + r) * TD + st * 32 + kq * 8);
        st0 = mfma_bf16(a0, qf[st], st0);
        st1 = mfma_bf16(a1, qf[st], st1);
      }
      const float sc = a.scaling * LOG2E;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = st0[i] * sc;
        s[4 + i] = st1[i] * sc;
        nv[i] = P_SCALE;
        nv[4 + i] = P_SCALE;
      }
    }
    // mask tokens past the end (their memory may hold anything: select, never multiply)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t t = tb + (i >> 2) * 16 + 4 * kq + (i & 3);
      if (t >= tend) {
        s[i] = -INFINITY;
        nv[i] = 0.f;
      }
    }
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (__any(mx > m_run + LAZY)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] *= alpha;
      m_run = m_new;
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = exp2f(s[i] - m_run);
      l_run += p[i];
    }
    u32x4 pf;
    if (!resid) {
#pragma unroll
      for (int i = 0; i < 4; ++i) pf[i] = pack_f16x2(p[i] * nv[i], p[4 + i] * nv[4 + i]);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t w = vraw[j >> 3][(j >> 1) & 3];
        const uint32_t xv = __builtin_amdgcn_perm(w, w, (j & 1) ? 0x030C020Cu : 0x010C000Cu);
        acc[j] = mfma_f16(codes_to_f16(xv, lut_hi, lut_lo, or_c), pf, acc[j]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) pf[i] = pack_bf16x2(p[i] * nv[i], p[4 + i] * nv[4 + i]);
      const uint16_t* rv = a.residual_value_t + (b * a.kv_heads + h) * TD * Rc + tb;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t dim = r * 16 + j;
        const uint2 lo = *(const uint2*)(rv + dim * Rc + 4 * kq);
        const uint2 hi = *(const uint2*)(rv + dim * Rc + 16 + 4 * kq);
        u32x4 av;
        av.x = __builtin_amdgcn_perm(hi.x, lo.x, 0x05040100u);
        av.y = __builtin_amdgcn_perm(hi.x, lo.x, 0x07060302u);
        av.z = __builtin_amdgcn_perm(hi.y, lo.y, 0x05040100u);
        av.w = __builtin_amdgcn_perm(hi.y, lo.y, 0x07060302u);
        acc[j] = mfma_bf16(av, pf, acc[j]);
      }
    }
  }
  // lanes of one head: sum partial denominators
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (kq == 0) {
    s_m[wave][r] = m_run;
    s_l[wave][r] = l_run;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < TWAVES; ++w) M = fmaxf(M, s_m[w][r]);
  const float f = l_run > 0.f ? exp2f(m_run - M) : 0.f;
  if (r < G) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) atomicAdd(&s_acc[r * TD + (4 * kq + i) * 16 + j], acc[j][i] * f);
  }
  __syncthreads();
  float* pv = a.partial_values + item * 16 * TD;
  for (int i = threadIdx.x; i < G * TD; i += blockDim.x) pv[i] = s_acc[i] * (1.0f / P_SCALE);
  if (threadIdx.x < (unsigned)G) {
    const int n = threadIdx.x;
    float Mx = -INFINITY, L = 0.f;
    for (int w = 0; w < TWAVES; ++w) Mx = fmaxf(Mx, s_m[w][n]);
    for (int w = 0; w < TWAVES; ++w)
      if (s_l[w][n] > 0.f) L += s_l[w][n] * exp2f(s_m[w][n] - Mx);
    a.partial_stats[(item * 16 + n) * 2] = Mx;
    a.partial_stats[(item * 16 + n) * 2 + 1] = L;
  }
}

// ------------------------------------------------------------------ merge

// grid (B * Hkv), 256 threads.
__global__ __launch_bounds__(256) void tq_decode_merge_kernel(const anna_mi_tq_decode_args a) {
  __shared__ float s_w[64][16];          // per-item weight exp2(m - M) / L (<= 64 items per (b,h) cached)
  __shared__ float s_M[16], s_L[16];
  __shared__ __attribute__((aligned(16))) uint16_t s_rot[16 * TD];  // normalized rotated accumulators, fp16 [head][i]
  __shared__ float s_res[16 * TD];       // normalized residual accumulators
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t bh = blockIdx.x, b = bh / a.kv_heads, h = bh % a.kv_heads;
  const int G = (int)(a.q_heads / a.kv_heads);
  const int32_t i0 = a.item_ranges[bh], i1 = a.item_ranges[bh + 1];
  const int nit = i1 - i0;
  if (threadIdx.x < 16) {
    const int n = threadIdx.x;
    float M = -INFINITY, L = 0.f;
    if (n < G) {
      for (int it = i0; it < i1; ++it) M = fmaxf(M, a.partial_stats[((int64_t)it * 16 + n) * 2]);
      for (int it = i0; it < i1; ++it) {
        const float l = a.partial_stats[((int64_t)it * 16 + n) * 2 + 1];
        if (l > 0.f) L += l * exp2f(a.partial_stats[((int64_t)it * 16 + n) * 2] - M);
      }
    }
    s_M[n] = M;
    s_L[n] = L;
  }
  __syncthreads();
  for (int k = threadIdx.x; k < nit * 16 && k < 64 * 16; k += blockDim.x) {
    const int it = k / 16, n = k % 16;
    float w = 0.f;
    if (n < G && s_L[n] > 0.f) {
      const float l = a.partial_stats[((int64_t)(i0 + it) * 16 + n) * 2 + 1];
      if (l > 0.f) w = exp2f(a.partial_stats[((int64_t)(i0 + it) * 16 + n) * 2] - s_M[n]) / s_L[n];
    }
    s_w[it][n] = w;
  }
  __syncthreads();
  // thread = dim; accumulate the weighted partials per head
  const int d = threadIdx.x;
  for (int n = 0; n < 16; ++n) {
    float ar = 0.f, aq = 0.f;
    if (n < G) {
      for (int it = i0; it < i1; ++it) {
        const float w = (it - i0) < 64 ? s_w[it - i0][n] : 0.f;
        if (w == 0.f) continue;
        const float v = a.partial_values[((int64_t)it * 16 + n) * TD + d] * w;
        if (a.items[(int64_t)it * 4 + 2] < 0) aq += v; else ar += v;
      }
    }
    s_rot[n * TD + d] = f32_to_f16_bits(ar);
    s_res[n * TD + d] = aq;
  }
  __syncthreads();
  // Y[n][d] = sum_i rot[n][i] * R[i][d]: A = rot (lane: head r, 8 consecutive i), B from R^T rows.
  const uint16_t* RT = (const uint16_t*)a.rotation_t_f16;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int tile = wave * 4 + tt;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const u32x4 af = *(const u32x4*)(s_rot + r * TD + s * 32 + kq * 8);
      const u32x4 bfr = *(const u32x4*)(RT + (int64_t)(tile * 16 + r) * TD + s * 32 + kq * 8);
      acc = mfma_f16(af, bfr, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 4 * kq + i;
      const int dd = tile * 16 + r;
      if (n < G) ((uint16_t*)a.out)[(b * a.q_heads + h * G + n) * TD + dd] = f32_to_bf16_bits(acc[i] + s_res[n * TD + dd]);
    }
  }
}

// ------------------------------------------------------------------ value blocking

// natural codes [tokens][64] -> blocked [tokens/32][2048]; one thread per output byte.
__global__ __launch_bounds__(256) void tq_block_values_kernel(const uint8_t* __restrict__ nat, int64_t tokens,
                                                              uint8_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= tokens / TBT * 2048) return;
  const int64_t blk = idx / 2048;
  const int o = (int)(idx % 2048);
  const int kq = o / 512, dim = (o % 512) / 2, half = o % 2;
  uint32_t byte = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t t = blk * TBT + 16 * half + 4 * kq + e;
    const uint32_t c = (nat[t * 64 + dim / 4] >> (2 * (dim % 4))) & 3u;
    byte |= c << (2 * e);
  }
  out[idx] = (uint8_t)byte;
}

}  // namespace
}  // namespace anna

using namespace anna;

extern "C" int64_t anna_mi_sizeof_tq_decode_args(void) { return (int64_t)sizeof(anna_mi_tq_decode_args); }

extern "C" int anna_mi_tq_decode_plan(int64_t batch, int64_t kv_heads, const int64_t* quantized_lens,
                                      const int64_t* residual_lens, int64_t tokens_per_item, int32_t* items,
                                      int64_t items_capacity, int32_t* item_ranges, int64_t* num_items) {
  ANNA_CHECK(items && item_ranges && num_items && quantized_lens && residual_lens, "anna_mi_tq_decode_plan: null pointer");
  ANNA_CHECK(tokens_per_item > 0 && tokens_per_item % TBT == 0, "tokens_per_item must be a positive multiple of 32");
  int64_t n = 0;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t h = 0; h < kv_heads; ++h) {
      item_ranges[b * kv_heads + h] = (int32_t)n;
      for (int64_t t = 0; t < quantized_lens[b]; t += tokens_per_item) {
        ANNA_CHECK(n < items_capacity, "anna_mi_tq_decode_plan: items capacity too small");
        const int64_t e = t + tokens_per_item < quantized_lens[b] ? t + tokens_per_item : quantized_lens[b];
        int32_t* it = items + n * 4;
        it[0] = (int32_t)b, it[1] = (int32_t)h, it[2] = (int32_t)t, it[3] = (int32_t)e;
        ++n;
      }
      if (residual_lens[b] > 0) {
        ANNA_CHECK(n < items_capacity, "anna_mi_tq_decode_plan: items capacity too small");
        int32_t* it = items + n * 4;
        it[0] = (int32_t)b, it[1] = (int32_t)h, it[2] = -1, it[3] = -1;
        ++n;
      }
      ANNA_CHECK(n - item_ranges[b * kv_heads + h] <= 64, "more than 64 work items for one sequence: raise tokens_per_item");
    }
  item_ranges[batch * kv_heads] = (int32_t)n;
  *num_items = n;
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_decode(const anna_mi_tq_decode_args* ap, void* stream) {
  ANNA_CHECK(ap != nullptr, "anna_mi_tq_decode: null args");
  const anna_mi_tq_decode_args& a = *ap;
  ANNA_CHECK(a.head_dim == TD, "anna_mi_tq_decode: head_dim must be 256");
  ANNA_CHECK(a.key_bits == 2 && a.value_bits == 2, "anna_mi_tq_decode: 2-bit codes only (use anna_mi_gqa_decode_splitkv)");
  ANNA_CHECK(a.kv_heads > 0 && a.q_heads % a.kv_heads == 0 && a.q_heads / a.kv_heads <= 16,
             "anna_mi_tq_decode: need q_heads = G * kv_heads with G <= 16");
  ANNA_CHECK(a.pool_tokens % TBT == 0 && a.residual_capacity % TBT == 0, "pool and residual capacity must be multiples of 32");
  ANNA_CHECK(a.query && a.out && a.query_rot && a.partial_stats && a.partial_values && a.items && a.item_ranges,
             "anna_mi_tq_decode: null pointer");
  ANNA_CHECK(a.rotation_f16 && a.rotation_t_f16 && a.key_codes && a.key_norms && a.value_codes && a.value_norms,
             "anna_mi_tq_decode: null cache pointer");
  if (a.num_items <= 0) return ANNA_MI_OK;
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(tq_rotate_query_kernel, dim3((unsigned)(a.batch * a.kv_heads)), dim3(256), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_rotate_query_kernel");
  hipLaunchKernelGGL(tq_decode_split_kernel, dim3((unsigned)a.num_items), dim3(64 * TWAVES), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_decode_split_kernel");
  hipLaunchKernelGGL(tq_decode_merge_kernel, dim3((unsigned)(a.batch * a.kv_heads)), dim3(256), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_decode_merge_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_block_values(const uint8_t* codes, int64_t tokens, uint8_t* blocked, void* stream) {
  ANNA_CHECK(codes && blocked, "anna_mi_tq_block_values: null pointer");
  ANNA_CHECK(tokens % TBT == 0, "anna_mi_tq_block_values: tokens must be a multiple of 32");
  const int64_t n = tokens / TBT * 2048;
  if (n == 0) return ANNA_MI_OK;
  hipLaunchKernelGGL(tq_block_values_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), codes,
                     tokens, blocked);
  ANNA_LAUNCH_CHECK("tq_block_values_kernel");
  return ANNA_MI_OK;
}
