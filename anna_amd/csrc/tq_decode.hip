// Batched varlen GQA decode over a 2-bit TurboQuant-MSE KV cache (head_dim 256), MFMA.
//
// Cache layout (per KV head, a pool of `pool_tokens` token slots; a sequence owns a range
// of slots starting at a multiple of 32):
//   key_codes   uint8 [Hkv][pool][64]       token-major, dim i at bits 2(i%4) of byte i/4
//   key_norms   fp16  [Hkv][pool]
//   value_codes uint8 [Hkv][pool/32][2048]  32-token blocks, byte ((t%16)/4)*512 + dim*2 + t/16,
//                                           token t at bits 2(t%4) (see tq_block_values_kernel)
//   value_norms fp16  [Hkv][pool]
//   residual_key     bf16 [B][Hkv][R][256]  newest tokens, dense, token-major
//   residual_value_t bf16 [B][Hkv][256][R]  dense, dim-major
//
// Three launches per call (work items come from anna_mi_tq_decode_plan):
//   tq_rotate_query   q' = R q for every (b, kv-head)'s G q-heads (MFMA, fp16), written in the
//     B-operand fragment order of the score product.
//   tq_decode_split   one 512-thread workgroup per work item (b, kv-head, pool range) or per
//     residual window.  8 waves take 32-token blocks (the next block prefetched).  Scores are
//     formed transposed, S^T = Khat Q'^T, by v_mfma_f32_16x16x32_f16 on codes turned into fp16
//     centroids with one v_perm per pair (the 2-bit centroids are fp16 values sharing their
//     low byte); S^T's accumulator layout is the B operand of O'^T = Vhat^T P^T, so the
//     probabilities never leave registers.  Online softmax in base 2 with lazy rescaling
//     (the running max only moves when a block exceeds it by 2^4).  The 8 waves' accumulators
//     are summed through LDS; per item and q-head the (max, denominator) and the unnormalized
//     accumulator go to the workspace.
//   tq_decode_combine 8 workgroups per (b, kv-head), one per 32 output dims: log-sum-exp merge
//     of the items over the rotated dims, R^T for the tile's dims (MFMA), plus the residual
//     window's part, written as bf16.
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

// ------------------------------------------------------------------ decode kernel

constexpr int SWAVES = 8;      // waves per work item

struct BlockRaw {
  u32x4 k0, k1, v0, v1;     // key codes (tokens r, 16 + r), value codes (dims 16 r .. 16 r + 15)
  uint2 kn0, kn1, vn0, vn1;  // norms of tokens 4 kq .. 4 kq + 3 and 16 + 4 kq ..
};

// p0: pool slot of the block's first token (multiple of 32)
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

__device__ __forceinline__ uint32_t f16x2_of_bf16x2(uint32_t v) {
  return pack_f16x2(bf16_bits_to_f32((uint16_t)(v & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(v >> 16)));
}

__device__ __forceinline__ uint32_t pkrtz(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// q' = R q for one tile of 16 dims of the G heads of one (b, kv-head), written into the B
// operand fragments of the score product: frag[step s][lane][e] (fp16) holds q'[head lane % 16][dim],
// dim = 64 (lane / 16) + 16 (s >> 1) + 4 (s & 1) + w', e = 2 (w' & 3) + (w' >> 3), w' in
// {0..3, 8..11} (the pair order of codes_to_f16).  One wave: A = R rows (16 dims x 32), B = q^T
// (32 x 16 heads, bf16 -> fp16); C lane: head r, dims 16 tile + 4 kq + i.
__device__ __forceinline__ void tq_rotate_fragment(const anna_mi_tq_decode_args& a, const uint16_t* qg, int G, int tile,
                                                   int lane, uint16_t* frag) {
  const int r = lane & 15, kq = lane >> 4;
  // unconditional loads (row clamped, value zeroed) so that they issue back to back
  const uint16_t* qrow = qg + (r < G ? r : 0) * TD + kq * 8;
  const uint32_t keep = r < G ? 0xFFFFFFFFu : 0u;
  u32x4 qv[8], rv[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    qv[st] = *(const u32x4*)(qrow + st * 32);
    rv[st] = *(const u32x4*)(a.rotation_f16 + (int64_t)(tile * 16 + r) * TD + st * 32 + kq * 8);
  }
  // no instruction moves above this point: every load is issued before the first conversion
  // waits for its data (the scheduler otherwise interleaves them, one round trip after another)
  __builtin_amdgcn_sched_barrier(0);
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    u32x4 qb;
#pragma unroll
    for (int w = 0; w < 4; ++w) qb[w] = f16x2_of_bf16x2(qv[st][w] & keep);
    c = mfma_f16(rv[st], qb, c);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int dim = tile * 16 + 4 * kq + i;
    const int kq2 = dim >> 6, rem = dim & 63, w = rem & 15;
    const int sx = 2 * (rem >> 4) + ((rem >> 2) & 1), e = 2 * (w & 3) + (w >> 3);
    frag[((sx * 64) + kq2 * 16 + r) * 8 + e] = f32_to_f16_bits(c[i]);
  }
}

// grid (B * Hkv, 16 dim tiles), one wave: q' fragments of every (b, kv-head) into
// query_frag[b][h] (4096 fp16 each).
__global__ __launch_bounds__(64) void tq_rotate_query_kernel(const anna_mi_tq_decode_args a) {
  const int64_t bh = blockIdx.x, b = bh / a.kv_heads, h = bh % a.kv_heads;
  const int G = (int)(a.q_heads / a.kv_heads);
  tq_rotate_fragment(a, a.query + (b * a.q_heads + h * G) * TD, G, blockIdx.y, threadIdx.x, a.query_frag + bh * 4096);
}

// One 32-token block of one wave (slot / window position tb): scores, online softmax, and
// the value product into acc.  RESID: the dense residual window (bf16 MFMAs, loads issued
// here); otherwise the 2-bit codes already loaded into cur.
// qf: the packed path's B fragments of the score product, held in registers for the whole item
// (the residual path reads s_qf and passes nullptr)
template <bool RESID>
__device__ __forceinline__ void block_step(const anna_mi_tq_decode_args& a, const u32x4 (*s_qf)[64], const u32x4* qf,
                                           int64_t b, int64_t h, int64_t tb, int64_t tend, int lane, const BlockRaw& cur,
                                           f32x4 (&acc)[16], float& m_run, float& l_run) {
  const int r = lane & 15, kq = lane >> 4;
  const int64_t Rc = a.residual_capacity;
  const uint32_t lut_hi = vconst(0x433CBCC3u), lut_lo = vconst(0x7E7E7E7Eu), or_c = vconst(0x04000400u);
  const float kscale = a.key_scale * a.scaling * LOG2E;
  const float vscale = a.value_scale * P_SCALE;
  {
    float s[8], nv[8];
    f32x4 st0 = {0.f, 0.f, 0.f, 0.f}, st1 = {0.f, 0.f, 0.f, 0.f};
    uint2 rlo[RESID ? 16 : 1], rhi[RESID ? 16 : 1];
    if constexpr (!RESID) {
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const uint32_t w0 = cur.k0[st >> 1], w1 = cur.k1[st >> 1];
        const uint32_t x0 = (st & 1) ? w0 : (w0 << 8), x1 = (st & 1) ? w1 : (w1 << 8);
        st0 = mfma_f16(codes_to_f16(x0, lut_hi, lut_lo, or_c), qf[st], st0);
        st1 = mfma_f16(codes_to_f16(x1, lut_hi, lut_lo, or_c), qf[st], st1);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = st0[i] * (half_of(cur.kn0, i) * kscale);
        s[4 + i] = st1[i] * (half_of(cur.kn1, i) * kscale);
        nv[i] = half_of(cur.vn0, i) * vscale;
        nv[4 + i] = half_of(cur.vn1, i) * vscale;
      }
    } else {
      // every load of the block first (K rows, V columns), then the MFMAs: left to itself the
      // scheduler interleaves load, wait and MFMA one tile at a time
      const uint16_t* rk = a.residual_key + ((b * a.kv_heads + h) * Rc + tb) * TD;
      const uint16_t* rv = a.residual_value_t + (b * a.kv_heads + h) * TD * Rc + tb;
      u32x4 ka[8], kb[8];
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        ka[st] = *(const u32x4*)(rk + r * TD + st * 32 + kq * 8);
        kb[st] = *(const u32x4*)(rk + (16 + r) * TD + st * 32 + kq * 8);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t dim = r * 16 + j;
        rlo[j] = *(const uint2*)(rv + dim * Rc + 4 * kq);
        rhi[j] = *(const uint2*)(rv + dim * Rc + 16 + 4 * kq);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const u32x4 qf = s_qf[st][lane];
        st0 = mfma_bf16(ka[st], qf, st0);
        st1 = mfma_bf16(kb[st], qf, st1);
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
    if (tb + TBT > tend) {
      // tokens past the end: their memory may hold anything (select, never multiply)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t t = tb + (i >> 2) * 16 + 4 * kq + (i & 3);
        if (t >= tend) {
          s[i] = -INFINITY;
          nv[i] = 0.f;
        }
      }
    }
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (__any(mx > m_run + LAZY)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] *= alpha;
      m_run = m_new;
    }
    u32x4 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p0 = __builtin_amdgcn_exp2f(s[i] - m_run), p1 = __builtin_amdgcn_exp2f(s[4 + i] - m_run);
      l_run += p0 + p1;
      pf[i] = RESID ? pack_bf16x2(p0 * nv[i], p1 * nv[4 + i]) : pkrtz(p0 * nv[i], p1 * nv[4 + i]);
    }
    if constexpr (!RESID) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t w = (j >> 3) ? cur.v1[(j >> 1) & 3] : cur.v0[(j >> 1) & 3];
        const uint32_t xv = __builtin_amdgcn_perm(w, w, (j & 1) ? 0x030C020Cu : 0x010C000Cu);
        acc[j] = mfma_f16(codes_to_f16(xv, lut_hi, lut_lo, or_c), pf, acc[j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint2 lo = rlo[j], hi = rhi[j];
        u32x4 av;
        av.x = __builtin_amdgcn_perm(hi.x, lo.x, 0x05040100u);
        av.y = __builtin_amdgcn_perm(hi.x, lo.x, 0x07060302u);
        av.z = __builtin_amdgcn_perm(hi.y, lo.y, 0x05040100u);
        av.w = __builtin_amdgcn_perm(hi.y, lo.y, 0x07060302u);
        acc[j] = mfma_bf16(av, pf, acc[j]);
      }
    }
  }
}

// The blocks of one item taken by one wave: blocks wave, wave + 8, ... (the first one of a
// packed item already loaded into A).  Packed blocks ping-pong between two register buffers in
// a loop over pairs with no exit in between (an exit inside the pair would give the
// accumulators two register homes and a copy per pair); the prefetch is unconditional (clamped
// to the last block) so that no wait for it is forced before the current block is consumed.
template <bool RESID>
__device__ __forceinline__ void run_blocks(const anna_mi_tq_decode_args& a, const u32x4 (*s_qf)[64], int64_t b, int64_t h,
                                           int64_t tb0, int64_t tend, int64_t nblk, int wave, int lane, BlockRaw& A,
                                           f32x4 (&acc)[16], float& m_run, float& l_run) {
  const int r = lane & 15, kq = lane >> 4;
  if constexpr (RESID) {
    for (int64_t blk = wave; blk < nblk; blk += SWAVES)
      block_step<true>(a, s_qf, nullptr, b, h, tb0 + blk * TBT, tend, lane, A, acc, m_run, l_run);
  } else {
    u32x4 qf[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) qf[st] = s_qf[st][lane];
    const int64_t cnt = wave < nblk ? (nblk - 1 - wave) / SWAVES + 1 : 0;
    auto slot = [&](int64_t i) {
      const int64_t c = wave + (int64_t)SWAVES * i;
      return tb0 + (c < nblk ? c : nblk - 1) * TBT;
    };
    BlockRaw B;
    int64_t i = 0;
    for (; i + 1 < cnt; i += 2) {
      load_block(a, h, slot(i + 1), r, kq, B);
      block_step<false>(a, s_qf, qf, b, h, slot(i), tend, lane, A, acc, m_run, l_run);
      load_block(a, h, slot(i + 2), r, kq, A);
      block_step<false>(a, s_qf, qf, b, h, slot(i + 1), tend, lane, B, acc, m_run, l_run);
    }
    if (i < cnt) block_step<false>(a, s_qf, qf, b, h, slot(i), tend, lane, A, acc, m_run, l_run);
  }
}

__global__ __launch_bounds__(64 * SWAVES) __attribute__((amdgpu_waves_per_eu(2, 8)))
void tq_decode_split_kernel(const anna_mi_tq_decode_args a) {
  // B operand of S^T = Khat Q'^T per dim-step and lane (fp16 q' or bf16 q)
  __shared__ u32x4 s_qf[8][64];
  __shared__ float s_m[SWAVES][16], s_l[SWAVES][16];
  // cross-wave sums: [wave][tile j][kq * 8 + head % 8]
  __shared__ f32x4 s_red[SWAVES][16][32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t item = blockIdx.x;
  const int32_t* it = a.items + item * 4;
  const int64_t b = it[0], h = it[1];
  const bool resid = it[2] < 0;
  const int64_t tb0 = resid ? 0 : it[2];
  const int64_t tend = it[3];  // end slot (packed) or window length (residual)
  const int G = (int)(a.q_heads / a.kv_heads);
  const int64_t Rc = a.residual_capacity;
  const int64_t nblk = (tend - tb0 + TBT - 1) / TBT;
  const uint16_t* qg = a.query + (b * a.q_heads + h * G) * TD;
  const int64_t bh = b * a.kv_heads + h;

  BlockRaw cur;
  if (!resid)  // in flight during the prologue (clamped: a wave without blocks reloads the last)
    load_block(a, h, tb0 + (wave < nblk ? wave : nblk - 1) * TBT, r, kq, cur);
  if (!resid) {
    s_qf[wave][lane] = *(const u32x4*)(a.query_frag + bh * 4096 + (wave * 64 + lane) * 8);
  } else {
    const u32x4 v = *(const u32x4*)(qg + (r < G ? r : 0) * TD + wave * 32 + kq * 8);
    s_qf[wave][lane] = r < G ? v : u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  f32x4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  if (resid)
    run_blocks<true>(a, s_qf, b, h, tb0, tend, nblk, wave, lane, cur, acc, m_run, l_run);
  else
    run_blocks<false>(a, s_qf, b, h, tb0, tend, nblk, wave, lane, cur, acc, m_run, l_run);

  // ---- reduce the waves
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (kq == 0) {
    s_m[wave][r] = m_run;
    s_l[wave][r] = l_run;
  }
  __syncthreads();
  {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < SWAVES; ++w) M = fmaxf(M, s_m[w][r]);
    const float f = l_run > 0.f ? __builtin_amdgcn_exp2f(m_run - M) * (1.0f / P_SCALE) : 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] *= f;
  }
  // partial_values[item] as f32x4 [head block hb/8][tile j][kq * 8 + head % 8]; element i of
  // entry (j, kq) is dim (4 kq + i) * 16 + j (the accumulator layout of O'^T)
  f32x4* pvi = (f32x4*)(a.partial_values + item * 16 * TD);
  for (int hb = 0; hb < G; hb += 8) {
    if (r >= hb && r < hb + 8) {
#pragma unroll
      for (int j = 0; j < 16; ++j) s_red[wave][j][kq * 8 + r - hb] = acc[j];
    }
    __syncthreads();
    const int t = threadIdx.x, j = t >> 5, e = t & 31;
    if (hb + (e & 7) < G) {
      f32x4 sum = s_red[0][j][e];
#pragma unroll
      for (int w = 1; w < SWAVES; ++w) sum += s_red[w][j][e];
      pvi[(hb / 8) * 512 + t] = sum;
    }
    __syncthreads();
  }
  if (threadIdx.x < (unsigned)G) {
    const int n = threadIdx.x;
    float Mx = -INFINITY, L = 0.f;
    for (int w = 0; w < SWAVES; ++w) Mx = fmaxf(Mx, s_m[w][n]);
    for (int w = 0; w < SWAVES; ++w)
      if (s_l[w][n] > 0.f) L += s_l[w][n] * __builtin_amdgcn_exp2f(s_m[w][n] - Mx);
    a.partial_stats[(item * 16 + n) * 2] = Mx;
    a.partial_stats[(item * 16 + n) * 2 + 1] = L;
  }
}

// ------------------------------------------------------------------ combine

// grid (B * Hkv, 8 tiles of 32 output dims), 256 threads: combines the items of one
// (b, kv-head) with log-sum-exp weights over all 256 rotated dims, applies R^T for the tile's
// 32 output dims (MFMA), adds the residual window's part and writes bf16.  Each of the 8 tile
// workgroups of a (b, kv-head) merges all dims itself: 8x the (L2-resident) partial reads, but
// 8x the compute units pulling them, which is what bounds this kernel.
constexpr int CMB_THREADS = 256, CMB_OT = 32;  // threads, output dims per workgroup
__global__ __launch_bounds__(CMB_THREADS) void tq_decode_combine_kernel(const anna_mi_tq_decode_args a) {
  constexpr int RP = TD + 8;  // padded fp16 rows of the rotated sum
  __shared__ uint16_t s_rot[16 * RP];
  __shared__ float s_res[16][CMB_OT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t bh = blockIdx.x, b = bh / a.kv_heads, h = bh % a.kv_heads;
  const int d0 = blockIdx.y * CMB_OT;
  const int G = (int)(a.q_heads / a.kv_heads);
  // R^T rows of the wave's output tile (waves 0 and 1): they depend on nothing, so they go first
  u32x4 bfr[8];
  if (wave < CMB_OT / 16) {
#pragma unroll
    for (int st = 0; st < 8; ++st)
      bfr[st] = *(const u32x4*)(a.rotation_t_f16 + (int64_t)(d0 + wave * 16 + r) * TD + st * 32 + kq * 8);
  }
  const int4 info = *(const int4*)(a.bh_items + bh * 4);  // first item, packed items, residual item
  const int i0 = info.x, npk = info.y, ires = info.z;
  const bool has_res = ires >= 0;
  constexpr int64_t IS = 16 * TD / 4;  // item stride of partial_values in f32x4
  // Entries (tile j, e) and (j + 8, e) of head n = hb + e % 8 in every item (512 entries per
  // head block; both of this thread's entries share n and so the stats): the thread combines the
  // items itself with an online log-sum-exp over batches of 16, every load of a batch issued
  // together (one round trip per 16 items).
  for (int hb = 0; hb < G; hb += 8) {
    const int t = tid, j = t >> 5, e = t & 31;
    const int n = hb + (e & 7), ekq = e >> 3;
    if (n >= G) continue;
    const f32x4* src = (const f32x4*)a.partial_values + (hb / 8) * 512 + t;
    const float* stn = a.partial_stats + n * 2;
    f32x4 vr0 = {0.f, 0.f, 0.f, 0.f}, vr1 = vr0;
    float2 mlr = {-INFINITY, 0.f};
    if (has_res) {
      vr0 = src[(int64_t)ires * IS];
      vr1 = src[(int64_t)ires * IS + CMB_THREADS];
      mlr = *(const float2*)(stn + (int64_t)ires * 32);
    }
    f32x4 sr0 = {0.f, 0.f, 0.f, 0.f}, sr1 = sr0;
    float M = -INFINITY, L = 0.f;
    for (int k0 = 0; k0 < npk; k0 += 16) {
      f32x4 v0[16], v1[16];
      float2 ml[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int64_t idx = i0 + (k0 + k < npk ? k0 + k : 0);
        v0[k] = src[idx * IS];
        v1[k] = src[idx * IS + CMB_THREADS];
        ml[k] = *(const float2*)(stn + idx * 32);
      }
      // all 48 loads of the batch go out before the first wait (left alone, the scheduler
      // issues the value loads only after the statistics have arrived)
      __builtin_amdgcn_sched_barrier(0);
      float mb = M;
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (k0 + k < npk && ml[k].y > 0.f) mb = fmaxf(mb, ml[k].x);
      if (mb == -INFINITY) continue;
      const float f = __builtin_amdgcn_exp2f(M - mb);  // 0 while M is -inf
      sr0 *= f;
      sr1 *= f;
      L *= f;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const float w = (k0 + k < npk && ml[k].y > 0.f) ? __builtin_amdgcn_exp2f(ml[k].x - mb) : 0.f;
        sr0 += v0[k] * w;
        sr1 += v1[k] * w;
        L += ml[k].y * w;
      }
      M = mb;
    }
    const float Mt = fmaxf(M, mlr.y > 0.f ? mlr.x : -INFINITY);
    const float fp = L > 0.f ? __builtin_amdgcn_exp2f(M - Mt) : 0.f;
    const float fr = mlr.y > 0.f ? __builtin_amdgcn_exp2f(mlr.x - Mt) : 0.f;
    const float inv = 1.0f / (L * fp + mlr.y * fr);
    sr0 *= fp * inv;
    sr1 *= fp * inv;
    vr0 *= fr * inv;
    vr1 *= fr * inv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int dim = (4 * ekq + i) * 16 + j + 8 * hf;
        s_rot[n * RP + dim] = f32_to_f16_bits(hf ? sr1[i] : sr0[i]);
        if (dim >= d0 && dim < d0 + CMB_OT) s_res[n][dim - d0] = hf ? vr1[i] : vr0[i];
      }
    }
  }
  __syncthreads();
  // out = rot R + res: wave w < 2 takes output dims [d0 + 16 w, d0 + 16 w + 16); A = rot (16 heads
  // x 32), B[k][d] = R[k][d] = R^T[d][k]; C lane: dim col r, heads 4 kq + i
  if (wave < CMB_OT / 16) {
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const u32x4 af = *(const u32x4*)(s_rot + r * RP + st * 32 + kq * 8);
      c = mfma_f16(af, bfr[st], c);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 4 * kq + i, dl = wave * 16 + r;
      if (n < G) a.out[(b * a.q_heads + h * G + n) * TD + d0 + dl] = f32_to_bf16_bits(c[i] + s_res[n][dl]);
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

// Blocks of 32 tokens per item for `slots` concurrent workgroups: the smallest count for which
// the items of every (b, kv-head) fit (an item of nb blocks puts at most ceil(nb / 4) of them on
// one SIMD, so no rounding to whole passes of the 8 waves).
static int64_t auto_blocks_per_item(int64_t batch, int64_t kv_heads, const int64_t* qlens, const int64_t* rlens) {
  constexpr int64_t SLOTS = 256;  // MI355X compute units: one 512-thread workgroup each
  int64_t total = 0, resid = 0;
  for (int64_t b = 0; b < batch; ++b) {
    total += (qlens[b] + TBT - 1) / TBT;
    resid += rlens[b] > 0;
  }
  total *= kv_heads;
  resid *= kv_heads;
  const int64_t slots = SLOTS - resid > kv_heads * batch ? SLOTS - resid : kv_heads * batch;
  int64_t bpi = (total + slots - 1) / slots;
  if (bpi < 1) bpi = 1;
  for (;; ++bpi) {
    int64_t n = 0;
    for (int64_t b = 0; b < batch; ++b) n += ((qlens[b] + TBT - 1) / TBT + bpi - 1) / bpi;
    if (n * kv_heads <= slots) return bpi;
  }
}

extern "C" int anna_mi_tq_decode_plan(int64_t batch, int64_t kv_heads, const int64_t* quantized_lens,
                                      const int64_t* residual_lens, const int64_t* seq_offsets,
                                      int64_t tokens_per_item, int32_t* items, int64_t items_capacity,
                                      int32_t* bh_items, int64_t* num_items) {
  ANNA_CHECK(items && bh_items && num_items && quantized_lens && residual_lens && seq_offsets,
             "anna_mi_tq_decode_plan: null pointer");
  ANNA_CHECK(tokens_per_item >= 0 && tokens_per_item % TBT == 0,
             "tokens_per_item must be 0 (automatic) or a positive multiple of 32");
  for (int64_t b = 0; b < batch; ++b) {
    ANNA_CHECK(quantized_lens[b] >= 0 && residual_lens[b] >= 0, "anna_mi_tq_decode_plan: negative length");
    ANNA_CHECK(quantized_lens[b] + residual_lens[b] > 0, "anna_mi_tq_decode_plan: a sequence has no tokens");
    ANNA_CHECK(seq_offsets[b] % TBT == 0, "anna_mi_tq_decode_plan: sequence offsets must be multiples of 32");
    ANNA_CHECK(seq_offsets[b] + quantized_lens[b] < ((int64_t)1 << 31), "anna_mi_tq_decode_plan: pool slot exceeds int32");
  }
  const int64_t bpi = tokens_per_item > 0 ? tokens_per_item / TBT
                                          : auto_blocks_per_item(batch, kv_heads, quantized_lens, residual_lens);
  int64_t n = 0;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t h = 0; h < kv_heads; ++h) {
      int32_t* info = bh_items + (b * kv_heads + h) * 4;
      info[0] = (int32_t)n, info[2] = -1, info[3] = 0;
      const int64_t q = quantized_lens[b], nb = (q + TBT - 1) / TBT;
      const int64_t k = (nb + bpi - 1) / bpi;  // items, with the blocks spread evenly over them
      for (int64_t i = 0; i < k; ++i) {
        ANNA_CHECK(n < items_capacity, "anna_mi_tq_decode_plan: items capacity too small");
        const int64_t b0 = nb * i / k, b1 = nb * (i + 1) / k;
        const int64_t t1 = b1 * TBT < q ? b1 * TBT : q;
        int32_t* it = items + n * 4;
        it[0] = (int32_t)b, it[1] = (int32_t)h;
        it[2] = (int32_t)(seq_offsets[b] + b0 * TBT), it[3] = (int32_t)(seq_offsets[b] + t1);
        ++n;
      }
      info[1] = (int32_t)k;
      if (residual_lens[b] > 0) {
        ANNA_CHECK(n < items_capacity, "anna_mi_tq_decode_plan: items capacity too small");
        info[2] = (int32_t)n;
        int32_t* it = items + n * 4;
        it[0] = (int32_t)b, it[1] = (int32_t)h, it[2] = -1, it[3] = (int32_t)residual_lens[b];
        ++n;
      }
    }
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
  ANNA_CHECK(a.query && a.out && a.query_frag && a.partial_stats && a.partial_values && a.items && a.bh_items,
             "anna_mi_tq_decode: null pointer");
  ANNA_CHECK(a.rotation_f16 && a.rotation_t_f16 && a.key_codes && a.key_norms && a.value_codes && a.value_norms,
             "anna_mi_tq_decode: null cache pointer");
  if (a.num_items <= 0) return ANNA_MI_OK;
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(tq_rotate_query_kernel, dim3((unsigned)(a.batch * a.kv_heads), 16), dim3(64), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_rotate_query_kernel");
  hipLaunchKernelGGL(tq_decode_split_kernel, dim3((unsigned)a.num_items), dim3(64 * SWAVES), 0, st, a);
  ANNA_LAUNCH_CHECK("tq_decode_split_kernel");
  hipLaunchKernelGGL(tq_decode_combine_kernel, dim3((unsigned)(a.batch * a.kv_heads), TD / CMB_OT), dim3(CMB_THREADS), 0,
                     st, a);
  ANNA_LAUNCH_CHECK("tq_decode_combine_kernel");
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
