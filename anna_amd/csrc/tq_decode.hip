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
// Kernels (one call = four launches):
//   tq_rotate_query  q' = R q (MFMA, fp16 in / fp32 accumulate) for every (b, q-head).
//   tq_decode_split  one workgroup per work item (b, kv-head, <= tokens_per_item tokens or the
//     residual window).  8 waves take 32-token blocks (next block prefetched).  Scores are formed transposed,
//     S^T = Khat Q'^T, by v_mfma_f32_16x16x32_f16 on codes turned into fp16 centroids with one
//     v_perm per pair (the 2-bit centroids are fp16 values sharing their low byte); S^T's
//     accumulator layout is exactly the B operand of O'^T = Vhat^T P^T, so probabilities
//     never leave registers.  Online softmax in base 2 with lazy rescaling (the running max
//     only moves when a block exceeds it by 2^4).  Output: per item and q-head
//     (max, denominator) and the unnormalized accumulator (rotated space for packed items).
//   tq_decode_combine  per (b, q-head): log-sum-exp weights of the items, weighted sums of the
//     packed (rotated) and residual partial accumulators.
//   tq_decode_unrotate  out = (rotated sum) R + (residual sum), a [B*Hq x 256] x [256 x 256]
//     MFMA product, bf16 output.
#include <vector>

#include "common.hpp"

namespace anna {
namespace {

constexpr int TD = 256;              // head_dim
constexpr int TBT = 32;              // tokens per block
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

// grid (B * Hkv, 16 output tiles), one wave.  Q [16 heads x 256] (bf16 -> fp16) times R^T.
__global__ __launch_bounds__(64) void tq_rotate_query_kernel(const anna_mi_tq_decode_args a) {
  const int lane = threadIdx.x;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t bh = blockIdx.x, b = bh / a.kv_heads, h = bh % a.kv_heads;
  const int tile = blockIdx.y;  // output dims i in [16 tile, 16 tile + 16)
  const int G = (int)(a.q_heads / a.kv_heads);
  const uint16_t* q = (const uint16_t*)a.query + (b * a.q_heads + h * G) * TD;
  const uint16_t* R = (const uint16_t*)a.rotation_f16;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < G) v = *(const u32x4*)(q + r * TD + s * 32 + kq * 8);
    u32x4 af;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      af[w] = pack_f16x2(bf16_bits_to_f32((uint16_t)(v[w] & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(v[w] >> 16)));
    const u32x4 bfr = *(const u32x4*)(R + (int64_t)(tile * 16 + r) * TD + s * 32 + kq * 8);
    acc = mfma_f16(af, bfr, acc);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = 4 * kq + i;
    if (n < G) ((uint16_t*)a.query_rot)[(b * a.q_heads + h * G + n) * TD + tile * 16 + r] = f32_to_f16_bits(acc[i]);
  }
}

// ------------------------------------------------------------------ split

constexpr int SWAVES = 8;  // waves per work item

struct BlockRaw {
  u32x4 k0, k1, v0, v1;     // key codes (tokens r, 16 + r), value codes (dims 16 r .. 16 r + 15)
  uint2 kn0, kn1, vn0, vn1;  // norms of tokens 4 kq .. 4 kq + 3 and 16 + 4 kq ..
};

__device__ __forceinline__ void load_block(const anna_mi_tq_decode_args& a, int64_t h, int64_t p0, int r, int kq,
                                           BlockRaw& o) {
  const int64_t T = a.pool_tokens;
  const uint8_t* kc = a.key_codes + (h * T + p0) * 64;
  o.k0 = __builtin_nontemporal_load((const u32x4*)(kc + r * 64 + kq * 16));
  o.k1 = __builtin_nontemporal_load((const u32x4*)(kc + (16 + r) * 64 + kq * 16));
  const uint8_t* vc = a.value_codes + (h * (T / TBT) + p0 / TBT) * 2048 + kq * 512 + r * 32;
  o.v0 = __builtin_nontemporal_load((const u32x4*)(vc));
  o.v1 = __builtin_nontemporal_load((const u32x4*)(vc + 16));
  const uint16_t* kn = a.key_norms + h * T + p0;
  const uint16_t* vn = a.value_norms + h * T + p0;
  o.kn0 = *(const uint2*)(kn + 4 * kq);
  o.kn1 = *(const uint2*)(kn + 16 + 4 * kq);
  o.vn0 = *(const uint2*)(vn + 4 * kq);
  o.vn1 = *(const uint2*)(vn + 16 + 4 * kq);
}

__device__ __forceinline__ float half_of(uint2 v, int i) {
  const uint32_t w = (i >> 1) ? v.y : v.x;
  return f16_bits_to_f32((uint16_t)(w >> (16 * (i & 1))));
}

__global__ __launch_bounds__(64 * SWAVES) __attribute__((amdgpu_waves_per_eu(2, 8)))
void tq_decode_split_kernel(const anna_mi_tq_decode_args a) {
  __shared__ u32x4 s_qf[8][64];  // B operand of S^T = Khat Q'^T per dim-step and lane
  __shared__ float s_m[SWAVES][16], s_l[SWAVES][16];
  // s_acc[(i * 16 + j) * 64 + lane] holds head r, dim (4 kq + i) * 16 + j: the 64 lanes of
  // one atomic add hit 64 consecutive words (no bank conflict).
  __shared__ float s_acc[16 * TD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t item = blockIdx.x;
  const int32_t* it = a.items + item * 4;
  const int64_t b = it[0], h = it[1];
  const int64_t t0 = it[2], t1 = it[3];
  const bool resid = t0 < 0;
  const int G = (int)(a.q_heads / a.kv_heads);
  const int64_t Rc = a.residual_capacity;
  const int64_t tb0 = resid ? 0 : t0;
  const int64_t tend = resid ? (int64_t)a.residual_lens[b] : t1;
  const int64_t nblk = (tend - tb0 + TBT - 1) / TBT;

  for (int i = threadIdx.x; i < 16 * TD; i += blockDim.x) s_acc[i] = 0.f;
  const int64_t off = resid ? 0 : a.seq_offsets[b];
  BlockRaw cur;
  if (!resid && wave < nblk) load_block(a, h, off + tb0 + wave * TBT, r, kq, cur);  // in flight across the barrier
  if (wave == 0) {
    if (!resid) {
      // q' rows in the pair order of codes_to_f16 (see the K conversion below)
      const uint16_t* qr = (const uint16_t*)a.query_rot + (b * a.q_heads + h * G + r) * TD;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int da = 64 * kq + 16 * (s >> 1) + 4 * (s & 1);
        uint2 lo = {0u, 0u}, hi = {0u, 0u};
        if (r < G) {
          lo = *(const uint2*)(qr + da);
          hi = *(const uint2*)(qr + da + 8);
        }
        u32x4 f;
        f.x = __builtin_amdgcn_perm(hi.x, lo.x, 0x05040100u);
        f.y = __builtin_amdgcn_perm(hi.x, lo.x, 0x07060302u);
        f.z = __builtin_amdgcn_perm(hi.y, lo.y, 0x05040100u);
        f.w = __builtin_amdgcn_perm(hi.y, lo.y, 0x07060302u);
        s_qf[s][lane] = f;
      }
    } else {
      const uint16_t* q = (const uint16_t*)a.query + (b * a.q_heads + h * G + r) * TD;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (r < G) v = *(const u32x4*)(q + s * 32 + kq * 8);
        s_qf[s][lane] = v;
      }
    }
  }
  __syncthreads();

  const uint32_t lut_hi = vconst(0x433CBCC3u), lut_lo = vconst(0x7E7E7E7Eu), or_c = vconst(0x04000400u);
  const float kscale = a.key_scale * a.scaling * LOG2E;
  const float vscale = a.value_scale * P_SCALE;
  f32x4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int64_t blk = wave; blk < nblk; blk += SWAVES) {
    const int64_t tb = tb0 + blk * TBT;
    if (!resid && blk != wave) load_block(a, h, off + tb, r, kq, cur);
    float s[8], nv[8];
    f32x4 st0 = {0.f, 0.f, 0.f, 0.f}, st1 = {0.f, 0.f, 0.f, 0.f};
    if (!resid) {
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const u32x4 qf = s_qf[st][lane];
        const uint32_t w0 = cur.k0[st >> 1], w1 = cur.k1[st >> 1];
        const uint32_t x0 = (st & 1) ? w0 : (w0 << 8), x1 = (st & 1) ? w1 : (w1 << 8);
        st0 = mfma_f16(codes_to_f16(x0, lut_hi, lut_lo, or_c), qf, st0);
        st1 = mfma_f16(codes_to_f16(x1, lut_hi, lut_lo, or_c), qf, st1);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = st0[i] * half_of(cur.kn0, i) * kscale;
        s[4 + i] = st1[i] * half_of(cur.kn1, i) * kscale;
        nv[i] = half_of(cur.vn0, i) * vscale;
        nv[4 + i] = half_of(cur.vn1, i) * vscale;
      }
    } else {
      const uint16_t* rk = a.residual_key + ((b * a.kv_heads + h) * Rc + tb) * TD;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const u32x4 qf = s_qf[st][lane];
        const u32x4 a0 = *(const u32x4*)(rk + r * TD + st * 32 + kq * 8);
        const u32x4 a1 = *(const u32x4*)(rk + (16 + r) * TD + st * 32 + kq * 8);
        st0 = mfma_bf16(a0, qf, st0);
        st1 = mfma_bf16(a1, qf, st1);
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
    u32x4 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p0 = exp2f(s[i] - m_run), p1 = exp2f(s[4 + i] - m_run);
      l_run += p0 + p1;
      pf[i] = resid ? pack_bf16x2(p0 * nv[i], p1 * nv[4 + i]) : pack_f16x2(p0 * nv[i], p1 * nv[4 + i]);
    }
    if (!resid) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t w = (j >> 3) ? cur.v1[(j >> 1) & 3] : cur.v0[(j >> 1) & 3];
        const uint32_t xv = __builtin_amdgcn_perm(w, w, (j & 1) ? 0x030C020Cu : 0x010C000Cu);
        acc[j] = mfma_f16(codes_to_f16(xv, lut_hi, lut_lo, or_c), pf, acc[j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
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
  for (int w = 0; w < SWAVES; ++w) M = fmaxf(M, s_m[w][r]);
  const float f = l_run > 0.f ? exp2f(m_run - M) : 0.f;
  if (r < G && f != 0.f) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) atomicAdd(&s_acc[(i * 16 + j) * 64 + lane], acc[j][i] * f);
  }
  __syncthreads();
  float* pv = a.partial_values + item * 16 * TD;
  for (int e = threadIdx.x; e < G * TD; e += blockDim.x) {
    const int n = e / TD, d = e % TD;
    const int ekq = d >> 6, ei = (d >> 4) & 3, ej = d & 15;
    pv[e] = s_acc[(ei * 16 + ej) * 64 + ekq * 16 + n] * (1.0f / P_SCALE);
  }
  if (threadIdx.x < (unsigned)G) {
    const int n = threadIdx.x;
    float Mx = -INFINITY, L = 0.f;
    for (int w = 0; w < SWAVES; ++w) Mx = fmaxf(Mx, s_m[w][n]);
    for (int w = 0; w < SWAVES; ++w)
      if (s_l[w][n] > 0.f) L += s_l[w][n] * exp2f(s_m[w][n] - Mx);
    a.partial_stats[(item * 16 + n) * 2] = Mx;
    a.partial_stats[(item * 16 + n) * 2 + 1] = L;
  }
}

// ------------------------------------------------------------------ merge

// Phase 1, grid (B * Hq), 256 threads (thread = dim): weighted sum of the items of one
// (b, q-head); writes the normalized rotated part (fp16) and the residual part (fp32).
__global__ __launch_bounds__(256) void tq_decode_combine_kernel(const anna_mi_tq_decode_args a) {
  __shared__ float s_w[64];
  const int64_t bq = blockIdx.x, b = bq / a.q_heads, hq = bq % a.q_heads;
  const int G = (int)(a.q_heads / a.kv_heads);
  const int64_t h = hq / G, n = hq % G;
  const int32_t i0 = a.item_ranges[b * a.kv_heads + h], i1 = a.item_ranges[b * a.kv_heads + h + 1];
  if (threadIdx.x < 64) {
    const int it = i0 + (int)threadIdx.x;
    const float m = it < i1 ? a.partial_stats[((int64_t)it * 16 + n) * 2] : -INFINITY;
    const float l = it < i1 ? a.partial_stats[((int64_t)it * 16 + n) * 2 + 1] : 0.f;
    const float M = wave_max(l > 0.f ? m : -INFINITY);
    const float e = l > 0.f ? exp2f(m - M) : 0.f;
    const float L = wave_sum(l * e);
    s_w[threadIdx.x] = L > 0.f ? e / L : 0.f;
  }
  __syncthreads();
  const int d = threadIdx.x;
  // the residual item, when present, is the last of the range (anna_mi_tq_decode_plan)
  const bool has_res = i1 > i0 && a.items[(int64_t)(i1 - 1) * 4 + 2] < 0;
  const int ip = has_res ? i1 - 1 : i1;
  const float* pv = a.partial_values + n * TD + d;
  float ar = 0.f, aq = 0.f;
  int it = i0;
  for (; it + 4 <= ip; it += 4) {
    const float v0 = pv[(int64_t)it * 16 * TD], v1 = pv[(int64_t)(it + 1) * 16 * TD];
    const float v2 = pv[(int64_t)(it + 2) * 16 * TD], v3 = pv[(int64_t)(it + 3) * 16 * TD];
    ar += v0 * s_w[it - i0] + v1 * s_w[it + 1 - i0] + v2 * s_w[it + 2 - i0] + v3 * s_w[it + 3 - i0];
  }
  for (; it < ip; ++it) ar += pv[(int64_t)it * 16 * TD] * s_w[it - i0];
  if (has_res) aq = pv[(int64_t)(i1 - 1) * 16 * TD] * s_w[i1 - 1 - i0];
  ((uint16_t*)a.query_rot)[bq * TD + d] = f32_to_f16_bits(ar);  // q' is no longer needed: reuse
  ((float*)a.out_residual)[bq * TD + d] = aq;
}

// Phase 2, grid (ceil(B*Hq / 16), 16 output tiles), one wave: out = rot R + residual.
__global__ __launch_bounds__(64) void tq_decode_unrotate_kernel(const anna_mi_tq_decode_args a) {
  const int lane = threadIdx.x;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 16;
  const int tile = blockIdx.y;
  const int64_t rows = a.batch * a.q_heads;
  const uint16_t* rot = (const uint16_t*)a.query_rot;
  const uint16_t* RT = (const uint16_t*)a.rotation_t_f16;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    u32x4 af = {0u, 0u, 0u, 0u};
    if (row0 + r < rows) af = *(const u32x4*)(rot + (row0 + r) * TD + s * 32 + kq * 8);
    const u32x4 bfr = *(const u32x4*)(RT + (int64_t)(tile * 16 + r) * TD + s * 32 + kq * 8);
    acc = mfma_f16(af, bfr, acc);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + 4 * kq + i;
    const int dd = tile * 16 + r;
    if (row < rows) ((uint16_t*)a.out)[row * TD + dd] = f32_to_bf16_bits(acc[i] + ((const float*)a.out_residual)[row * TD + dd]);
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
  ANNA_CHECK(a.query && a.out && a.out_residual && a.query_rot && a.partial_stats && a.partial_values && a.items &&
             a.item_ranges,
             "anna_mi_tq_decode: null pointer");
  ANNA_CHECK(a.rotation_f16 && a.rotation_t_f16 && a.key_codes && a.key_norms && a.value_codes && a.value_norms,
             "anna_mi_tq_decode: null cache pointer");
  if (a.num_items <= 0) return ANNA_MI_OK;
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(tq_rotate_query_kernel, dim3((unsigned)(a.batch * a.kv_heads), 16), dim3(64), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_rotate_query_kernel");
  hipLaunchKernelGGL(tq_decode_split_kernel, dim3((unsigned)a.num_items), dim3(64 * SWAVES), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_decode_split_kernel");
  hipLaunchKernelGGL(tq_decode_combine_kernel, dim3((unsigned)(a.batch * a.q_heads)), dim3(256), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_decode_combine_kernel");
  hipLaunchKernelGGL(tq_decode_unrotate_kernel, dim3((unsigned)((a.batch * a.q_heads + 15) / 16), 16), dim3(64), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_decode_unrotate_kernel");
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
