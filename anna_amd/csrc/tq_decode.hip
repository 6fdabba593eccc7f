// Batched varlen GQA decode over a 2-bit TurboQuant-MSE KV cache (head_dim 256), MFMA, a split
// and a merge launch per step; and the append of one token per sequence.
//
// Cache layout (per KV head, a pool of `pool_tokens` token slots; sequence b owns the slots
// from seq_offsets[b], a multiple of 32):
//   key_codes   uint8 [Hkv][pool][64]       token-major, dim i at bits 2(i%4) of byte i/4
//   key_norms   fp16  [Hkv][pool]
//   value_codes uint8 [Hkv][pool/32][2048]  32-token blocks, byte ((t%16)/4)*512 + dim*2 + t/16,
//                                           token t at bits 2(t%4) (see tq_block_values_kernel)
//   value_norms fp16  [Hkv][pool]
//   residual_key     bf16 [B][Hkv][R][256]  ring of the newest tokens, token-major
//   residual_value_t bf16 [B][Hkv][256][R]  the same ring, dim-major
// Token j of sequence b sits in ring slot j % R while it is among the newest R; the older ones
// are the quantized prefix, pool slots seq_offsets[b] .. + length - R.  Codes are TQ-MSE with
// the randomized Hadamard rotation R = H diag(s) / 16 (tq_hadamard.hpp).
//
// tq_decode_kernel, one 512-thread workgroup per work item:
//   * plan (every workgroup, from seq_lengths): B*Hkv window items, then per sequence
//     ceil(blocks / bpi) items per KV head over its quantized prefix, bpi chosen so that all
//     items fit the grid.  No host round trip: the grid is fixed, spare workgroups exit.
//   * a packed item rotates its G query heads itself, q' = R q (FWHT in registers, one wave
//     per head), into the B-operand fragments of the score product; 8 waves take 32-token blocks
//     (the next block prefetched).  Scores are formed transposed, S^T = Khat Q'^T, by
//     v_mfma_f32_16x16x32_f16 on codes turned into fp16 centroids by a 256-entry LDS table (a
//     code byte -> its four centroids, one 8-byte read per four codes); S^T's accumulator
//     layout is the B operand of O'^T = Vhat^T P^T, so the probabilities never leave registers.  Online
//     softmax in base 2 with lazy rescaling (the running max moves only by > 2^4).  The window
//     item does the same on the dense bf16 ring with the unrotated q.
//   * each item writes (max, denominator) and its values divided by the denominator (fp16) to
//     the workspace;
//     the window item of (b, kv head) also writes where that pair's packed items are.
// tq_merge_kernel, one wave per (b, kv head, q head): merges the items with log-sum-exp weights,
// rotates the packed part back (R^T o' = s * FWHT(o') / 16), adds the window part, applies the
// sigmoid gate and writes bf16.  (A last-arriving-item merge inside the split kernel measured
// slower: its coherent partial stores, ticket and merge loads were a chain of round trips after
// the split, 27.2 against 24.2 us at config 4.)
//
// tq_append_kernel, one workgroup per sequence: quantizes the token leaving the ring into the
// pool (bit-exact with anna_mi_tq_hadamard_quantize), writes the new token into its ring slot
// and increments the sequence length.
#include <vector>

#include "common.hpp"
#include "tq_hadamard.hpp"

namespace anna {
namespace {

typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

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

// The fp16 2-bit centroids {-b, -a, +a, +b} (high bytes 0xC3, 0xBC, 0x3C, 0x43, common low byte
// 0x7E: -3.74609375, -1.123046875, 1.123046875, 3.74609375) and the decode table built from
// them: entry c of the 256 holds the centroids of the four codes of byte c (code i at bits 2i)
// as four fp16, lowest code first.
constexpr uint32_t TQ2_F16[4] = {0xC37Eu, 0xBC7Eu, 0x3C7Eu, 0x437Eu};
__device__ __forceinline__ uint2 tq2_lut_entry(uint32_t c) {
  return make_uint2(TQ2_F16[c & 3u] | (TQ2_F16[(c >> 2) & 3u] << 16),
                    TQ2_F16[(c >> 4) & 3u] | (TQ2_F16[(c >> 6) & 3u] << 16));
}

// Two code bytes (bits 8 s .. 8 s + 15 of w) -> the 8 fp16 centroids of their codes, in code
// order: one table read per byte.  (Turning codes into fp16 by byte permutes took 11 VALU
// instructions per 8 codes, two thirds of a block's VALU work; a table read is 1 VALU for the
// address and one LDS read.)
__device__ __forceinline__ u32x4 codes_lut(const uint2* lut, uint32_t w, int s) {
  const uint2 lo = lut[(w >> (8 * s)) & 0xFFu], hi = lut[(w >> (8 * s + 8)) & 0xFFu];
  return u32x4{lo.x, lo.y, hi.x, hi.y};
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}

// The token leaving sequence b's ring (its length n >= R, so ring slot n % R holds token n - R):
// vector is_v (K or V) of KV head h quantized by one wave into pool slot `slot` -- key codes
// token-major, value codes into their 2 bits of the 32-token blocked layout -- with its fp16
// norm (bit-exact with anna_mi_tq_hadamard_quantize).
// rec (or nullptr): also the code byte of the lane's 4 dims at rec[64 is_v + lane] and the norm
// at rec + 128 + 2 is_v.
__device__ __forceinline__ void evict_token(const anna_mi_tq_append_args& a, int64_t b, int64_t h, int n, int64_t slot,
                                            bool is_v, int lane, uint8_t* rec = nullptr) {
  const int64_t H = a.kv_heads, R = a.residual_capacity, T = a.pool_tokens, rpos = n % R;
  float x[4];
  if (!is_v) {
    const uint2 raw = *(const uint2*)(a.residual_key + ((b * H + h) * R + rpos) * TD + 4 * lane);
    x[0] = bf16_bits_to_f32((uint16_t)(raw.x & 0xFFFFu));
    x[1] = bf16_bits_to_f32((uint16_t)(raw.x >> 16));
    x[2] = bf16_bits_to_f32((uint16_t)(raw.y & 0xFFFFu));
    x[3] = bf16_bits_to_f32((uint16_t)(raw.y >> 16));
  } else {
    const uint16_t* col = a.residual_value_t + (b * H + h) * TD * R + rpos;
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = bf16_bits_to_f32(col[(4 * lane + e) * R]);
  }
  uint32_t code[4];
  const float nrm = hadamard_codes_wave<4>(x, a.signs, a.thresholds, 3, 1.0f / 16.0f, code);
  const uint16_t nb16 = f32_to_f16_bits(nrm);
  const uint8_t byte = (uint8_t)(code[0] | (code[1] << 2) | (code[2] << 4) | (code[3] << 6));
  if (rec) {
    rec[64 * is_v + lane] = byte;
    if (lane == 0) ((uint16_t*)(rec + 128))[is_v] = nb16;
  }
  if (!is_v) {
    a.key_codes[(h * T + slot) * 64 + lane] = byte;
    if (lane == 0) a.key_norms[h * T + slot] = nb16;
  } else {
    const int64_t t = slot % TBT;
    uint8_t* blk = a.value_codes + (h * (T / TBT) + slot / TBT) * 2048 + ((t % 16) / 4) * 512 + (t / 16);
    const int sh = 2 * (int)(t % 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint8_t* p = blk + (4 * lane + e) * 2;
      *p = (uint8_t)(sh == 0 ? code[e] : (*p | (code[e] << sh)));
    }
    if (lane == 0) a.value_norms[h * T + slot] = nb16;
  }
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

// One 32-token block of one wave (slot / window position tb): scores, online softmax, and
// the value product into acc.  RESID: the dense residual window (bf16 MFMAs, loads issued
// here); otherwise the 2-bit codes already loaded into cur.
// qf: the packed path's B fragments of the score product, held in registers for the whole item
// (the residual path reads s_qf and passes nullptr)
// lut: the code-byte table in LDS.  Token order of the value product's k dimension (lane (r, kq),
// element e): token 16 (e / 4) + 4 kq + e % 4, for the packed codes and the window alike.
template <bool RESID>
__device__ __forceinline__ void block_step(const anna_mi_tq_decode_args& a, const u32x4 (*s_qf)[64], const u32x4* qf,
                                           const uint2* lut, int64_t b, int64_t h, int64_t tb, int64_t tend,
                                           int64_t skip, int lane, const BlockRaw& cur, f32x4 (&acc)[16],
                                           float& m_run, float& l_run) {
  const int r = lane & 15, kq = lane >> 4;
  const int64_t Rc = a.residual_capacity;
  const float kscale = a.key_scale * a.scaling * LOG2E;
  const float vscale = a.value_scale * P_SCALE;
  {
    float s[8], nv[8];
    f32x4 st0 = {0.f, 0.f, 0.f, 0.f}, st1 = {0.f, 0.f, 0.f, 0.f};
    uint2 rlo[RESID ? 16 : 1], rhi[RESID ? 16 : 1];
    if constexpr (!RESID) {
      // step st: code bytes 2 (st % 2), + 1 of word st / 2 (dims 64 kq + 16 (st / 2) + 8 (st % 2) ..
      // + 7 of tokens r and 16 + r)
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        st0 = mfma_f16(codes_lut(lut, cur.k0[st >> 1], 2 * (st & 1)), qf[st], st0);
        st1 = mfma_f16(codes_lut(lut, cur.k1[st >> 1], 2 * (st & 1)), qf[st], st1);
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
    if (RESID && skip >= tb && skip < tb + TBT) {
      // the window slot whose token has just left the ring (the fused append + decode)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t t = tb + (i >> 2) * 16 + 4 * kq + (i & 3);
        if (t == skip) {
          s[i] = -INFINITY;
          nv[i] = 0.f;
        }
      }
    }
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i]);
    mx = fmaxf(mx, lane_xor16(mx));
    mx = fmaxf(mx, lane_xor32(mx));
    if (__any(mx > m_run + LAZY)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] *= alpha;
      m_run = m_new;
    }
    // s[i] is token 4 kq + i (i < 4) or 16 + 4 kq + i - 4: element i of the value product's B
    u32x4 pf;
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
      float p0 = __builtin_amdgcn_exp2f(s[2 * i2] - m_run), p1 = __builtin_amdgcn_exp2f(s[2 * i2 + 1] - m_run);
      if (RESID) {  // a window block can be all masked (the skipped slot alone), m_run still -inf
        p0 = s[2 * i2] == -INFINITY ? 0.f : p0;
        p1 = s[2 * i2 + 1] == -INFINITY ? 0.f : p1;
      }
      l_run += p0 + p1;
      pf[i2] = RESID ? pack_bf16x2(p0 * nv[2 * i2], p1 * nv[2 * i2 + 1]) : pkrtz(p0 * nv[2 * i2], p1 * nv[2 * i2 + 1]);
    }
    if constexpr (!RESID) {
      // tile j: the two code bytes of dim 16 r + j (tokens 4 kq .. + 3, then 16 + 4 kq .. + 3)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t w = (j >> 3) ? cur.v1[(j >> 1) & 3] : cur.v0[(j >> 1) & 3];
        acc[j] = mfma_f16(codes_lut(lut, w, 2 * (j & 1)), pf, acc[j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] = mfma_bf16(u32x4{rlo[j].x, rlo[j].y, rhi[j].x, rhi[j].y}, pf, acc[j]);
    }
  }
}

// The blocks of one item taken by one wave: blocks wave, wave + 8, ... (the first one of a
// packed item already loaded into A).  Packed blocks ping-pong between two register buffers in
// a loop over pairs with no exit in between (an exit inside the pair would give the
// accumulators two register homes and a copy per pair); the prefetch is unconditional (clamped
// to the last block) so that no wait for it is forced before the current block is consumed.
template <bool RESID>
__device__ __forceinline__ void run_blocks(const anna_mi_tq_decode_args& a, const u32x4 (*s_qf)[64], const uint2* lut,
                                           int64_t b, int64_t h,
                                           int64_t tb0, int64_t tend, int64_t skip, int64_t nblk, int wave, int lane,
                                           BlockRaw& A, f32x4 (&acc)[16], float& m_run, float& l_run) {
  const int r = lane & 15, kq = lane >> 4;
  if constexpr (RESID) {
    for (int64_t blk = wave; blk < nblk; blk += SWAVES)
      block_step<true>(a, s_qf, nullptr, lut, b, h, tb0 + blk * TBT, tend, skip, lane, A, acc, m_run, l_run);
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
      block_step<false>(a, s_qf, qf, lut, b, h, slot(i), tend, -1, lane, A, acc, m_run, l_run);
      load_block(a, h, slot(i + 2), r, kq, A);
      block_step<false>(a, s_qf, qf, lut, b, h, slot(i + 1), tend, -1, lane, B, acc, m_run, l_run);
    }
    if (i < cnt) block_step<false>(a, s_qf, qf, lut, b, h, slot(i), tend, -1, lane, A, acc, m_run, l_run);
  }
}


constexpr int MAX_SEQS = 1024;  // sequences per call (the plan keeps their block counts in LDS)

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

struct ItemInfo {
  int kind;    // 0 packed, 1 window, 2 zero output (empty sequence), -1 none
  int b, h;
  int tb0, tend;      // packed: pool slots [tb0, tend); window: [0, window length)
  int kb;             // packed items of each (b, kv head) of this sequence
  int first_packed;   // workgroup index of item 0 of (b, h = 0)
};

// Work item of this workgroup (computed by wave 0, broadcast through LDS).
__device__ void plan_item(const anna_mi_tq_decode_args& a, int lane, int* s_nb, int* s_len, int* s_off,
                          ItemInfo* out) {
  const int B = (int)a.batch, H = (int)a.kv_heads, R = (int)a.residual_capacity;
  const int w = (int)blockIdx.x, nwg = (int)a.num_workgroups;
  int T = 0;
  for (int c = 0; c < B; c += 64) {
    const int b = c + lane;
    int nb = 0;
    if (b < B) {
      const int len = a.seq_lengths[b], off = a.seq_offsets[b];  // the plan's only global loads
      s_len[b] = len;
      s_off[b] = off;
      int q = len > R ? len - R : 0;
      const int room = (int)a.pool_tokens - off;  // never read past the pool
      q = q < room ? q : (room > 0 ? room : 0);
      nb = (q + TBT - 1) / TBT;
      s_nb[b] = len > 0 ? nb : -1;  // -1: empty sequence
    }
    T += wave_sum_int(nb);
  }
  T *= H;
  // blocks per item: the caller's, if its items fit the grid (lengths within the capacities the
  // grid was sized for), else the smallest count that fits (always possible: the grid holds at
  // least 2 B Hkv + 1 workgroups, and sum_b ceil(nb_b / bpi) <= T / (Hkv bpi) + B)
  int bpi = (int)a.blocks_per_item;
  if (bpi > 0) {
    int items = 0;
    for (int c = 0; c < B; c += 64) {
      const int b = c + lane;
      const int nb = b < B ? s_nb[b] : 0;
      items += wave_sum_int(nb > 0 ? (nb + bpi - 1) / bpi : 0);
    }
    if (items * H > nwg - B * H) bpi = 0;
  }
  if (bpi <= 0) {
    int avail = nwg - 2 * B * H;
    avail = avail < 1 ? 1 : avail;
    bpi = (T + avail - 1) / avail;
    bpi = bpi < 1 ? 1 : bpi;
  }
  // target: the sequence of a window workgroup, or the item index p of a packed one
  const bool window = w < B * H;
  const int p = w - B * H;
  int base = 0, found_b = window ? w / H : -1, found_excl = 0, found_kb = 0;
  for (int c = 0; c < B; c += 64) {
    const int b = c + lane;
    const int nb = b < B ? s_nb[b] : 0;
    const int kb = nb > 0 ? (nb + bpi - 1) / bpi : 0;
    const int incl = wave_incl_scan(kb * H, lane);
    const int excl = incl - kb * H;
    if (window) {
      if (b == found_b) {
        found_excl = base + excl;
        found_kb = kb;
      }
    } else {
      const bool hit = b < B && kb > 0 && p >= base + excl && p < base + incl;
      const unsigned long long m = __ballot(hit);
      if (m && found_b < 0) {
        const int src = __ffsll((long long)m) - 1;
        found_b = __shfl(b, src, 64);
        found_excl = __shfl(base + excl, src, 64);
        found_kb = __shfl(kb, src, 64);
      }
    }
    base += __shfl(incl, 63, 64);
  }
  if (window) {
    // the lane that held found_b published it; take it from there
    const int src = found_b % 64;
    found_excl = __shfl(found_excl, src, 64);
    found_kb = __shfl(found_kb, src, 64);
  }
  if (lane != 0) return;
  ItemInfo it{};
  it.kind = -1;
  if (found_b >= 0) {
    const int b = found_b;
    const int len = s_len[b];
    it.b = b;
    it.kb = found_kb;
    it.first_packed = B * H + found_excl;
    if (window) {
      it.h = w % H;
      it.kind = len > 0 ? 1 : 2;
      it.tb0 = 0;
      it.tend = len < R ? len : R;
    } else {
      const int q = p - found_excl;
      it.h = q / found_kb;
      const int i = q % found_kb;
      const int nb = s_nb[b];
      const int blk0 = (int)((int64_t)nb * i / found_kb), blk1 = (int)((int64_t)nb * (i + 1) / found_kb);
      const int off = s_off[b];
      int qlen = len - R;
      qlen = qlen < (int)a.pool_tokens - off ? qlen : (int)a.pool_tokens - off;
      it.kind = 0;
      it.tb0 = off + blk0 * TBT;
      it.tend = off + (blk1 * TBT < qlen ? blk1 * TBT : qlen);
    }
  }
  *out = it;
}

constexpr int MRG_BATCH = 16;  // items whose partials the merge loads together

// The fused step's record of the token leaving (b, h)'s ring, in the unused upper half of the
// window item's partial slot (the window items are workgroups 0 .. B Hkv - 1): key code bytes
// [64], value code bytes [64] (lane l: dims 4 l .. 4 l + 3, 2 bits each), the two fp16 norms,
// and whether the token was stored (int32 at byte 132).  The merge reads it at an address that
// does not depend on the item table.
__device__ __forceinline__ uint8_t* evict_record(const anna_mi_tq_decode_args& a, int64_t bh) {
  return (uint8_t*)(a.partial_values + bh * 16 * TD) + 12288;
}

// FUSED: the step's append as well (ap describes the same cache).  The plan and the packed items
// see the lengths before the append; the window workgroup of (b, h) quantizes the token leaving
// its ring into the pool slot just past the packed items' range and leaves that ring slot out
// of its own attention; the merge launch adds the leaving token (from its fresh codes) and the
// new one, then writes the new token into the ring and the new length.  Item table entries are
// 4 per (b, h): first packed item, item count, length before the append, whether the leaving
// token was stored.
template <bool FUSED>
__global__ __launch_bounds__(64 * SWAVES) __attribute__((amdgpu_waves_per_eu(2, 8)))
void tq_decode_kernel(const anna_mi_tq_decode_args a, const anna_mi_tq_append_args ap) {
  // one 64 KB buffer, used in turn for the rotated query (fp32 [16][256]), the cross-wave sums
  // ([wave][tile j][kq * 8 + head % 8] f32x4) and the merge's two [16][256] fp32 results
  __shared__ __attribute__((aligned(16))) float s_big[SWAVES * 16 * 32 * 4];
  __shared__ u32x4 s_qf[8][64];  // B operand of S^T = Khat Q'^T per dim-step and lane
  __shared__ float s_m[SWAVES][16], s_l[SWAVES][16];
  __shared__ int s_nb[MAX_SEQS], s_len[MAX_SEQS], s_off[MAX_SEQS];
  __shared__ ItemInfo s_it;
  __shared__ uint2 s_lut[256];  // code byte -> its four fp16 centroids
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  if (wave == 0) plan_item(a, lane, s_nb, s_len, s_off, &s_it);
  if (threadIdx.x >= 256) s_lut[threadIdx.x - 256] = tq2_lut_entry(threadIdx.x - 256);
  __syncthreads();
  const ItemInfo it = s_it;
  if (it.kind < 0) return;
  const int G = (int)(a.q_heads / a.kv_heads);
  const int64_t b = it.b, h = it.h, bh = b * a.kv_heads + h;
  int64_t skip = -1;  // window slot left out (the fused append's leaving token)
  if constexpr (FUSED) {
    if (it.kind != 0) {
      const int n = s_len[b];
      const int64_t R = a.residual_capacity;
      const bool room = n >= R && n - R < ap.seq_capacity[b];
      if (n >= R) {
        skip = n % R;
        if (!room && threadIdx.x == 0 && ap.overflow) *ap.overflow = 1;
      }
      if (threadIdx.x == 0) {
        *(int*)(evict_record(a, bh) + 132) = room ? 1 : 0;
        a.item_table[4 * bh] = it.first_packed + (int)h * it.kb;
        a.item_table[4 * bh + 1] = it.kb;
        a.item_table[4 * bh + 2] = n;
        a.item_table[4 * bh + 3] = room ? 1 : 0;
      }
    }
  } else {
    if (it.kind != 0 && threadIdx.x == 0) {
      // the window item of (b, h) tells the merge where its packed items are (-1: empty sequence)
      a.item_table[2 * bh] = it.kind == 2 ? -1 : it.first_packed + (int)h * it.kb;
      a.item_table[2 * bh + 1] = it.kb;
    }
    if (it.kind == 2) {  // empty sequence: zeros
      for (int i = threadIdx.x; i < G * TD; i += blockDim.x) a.out[(b * a.q_heads + h * G) * TD + i] = 0;
      return;
    }
  }
  // (fused: an empty sequence's window item runs with no slots and writes empty stats)
  const bool resid = it.kind != 0;
  const int64_t tb0 = it.tb0, tend = it.tend;
  const int64_t nblk = (tend - tb0 + TBT - 1) / TBT;
  const uint16_t* qg = a.query + (b * a.q_heads + h * G) * TD;
  const float inv = 1.0f / 16.0f;  // fp32(1/sqrt(256)), exact

  BlockRaw cur;
  // the query rows and signs first: issued behind the block loads they would wait for the
  // whole first wave of block data
  uint2 qraw[2] = {make_uint2(0u, 0u), make_uint2(0u, 0u)};
  float4 sg4 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (!resid) {
    sg4 = *(const float4*)(a.signs + 4 * lane);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int n = wave + SWAVES * k;
      if (n < G) qraw[k] = *(const uint2*)(qg + n * TD + 4 * lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    load_block(a, h, tb0 + (wave < nblk ? wave : nblk - 1) * TBT, r, kq, cur);
    __builtin_amdgcn_sched_barrier(0);
    // q' = R q: wave w rotates heads w and w + 8 (lane: dims 4 lane .. 4 lane + 3)
    float* s_q = s_big;  // [16][TD]
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int n = wave + SWAVES * k;
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (n < G) {
        const uint2 raw = qraw[k];
        v[0] = bf16_bits_to_f32((uint16_t)(raw.x & 0xFFFFu)) * sg4.x;
        v[1] = bf16_bits_to_f32((uint16_t)(raw.x >> 16)) * sg4.y;
        v[2] = bf16_bits_to_f32((uint16_t)(raw.y & 0xFFFFu)) * sg4.z;
        v[3] = bf16_bits_to_f32((uint16_t)(raw.y >> 16)) * sg4.w;
        fwht_wave<4>(v);
      }
      *(float4*)(s_q + n * TD + 4 * lane) = make_float4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    }
    __syncthreads();
    // fragment of step st = wave: element e holds dim 64 kq + 16 (st >> 1) + 8 (st & 1) + e
    const int dim0 = 64 * kq + 16 * (wave >> 1) + 8 * (wave & 1);
    const float* qr = s_q + r * TD + dim0;
    u32x4 f;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) f[e2] = pack_f16x2(qr[2 * e2], qr[2 * e2 + 1]);
    s_qf[wave][lane] = f;
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
    run_blocks<true>(a, s_qf, s_lut, b, h, tb0, tend, skip, nblk, wave, lane, cur, acc, m_run, l_run);
  else
    run_blocks<false>(a, s_qf, s_lut, b, h, tb0, tend, -1, nblk, wave, lane, cur, acc, m_run, l_run);

  if constexpr (FUSED) {
    // the window workgroup quantizes the token leaving the ring into the pool slot just past its
    // sequence's packed items (which do not read it), after its own attention loop
    if (resid && skip >= 0 && wave < 2) {
      const int n = s_len[b];
      const int64_t R = a.residual_capacity;
      if (n - R < ap.seq_capacity[b])
        evict_token(ap, b, h, n, s_off[b] + (n - R), wave == 1, lane, evict_record(a, bh));
    }
  }
  // ---- reduce the waves, write this item's partials (workgroup index = item slot)
  const int64_t item = blockIdx.x;
  l_run += lane_xor16(l_run);
  l_run += lane_xor32(l_run);
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
  // partial_values[item] as 4 x fp16 entries [head block hb/8][tile j][kq * 8 + head % 8];
  // element i of entry (j, kq) is dim (4 kq + i) * 16 + j (the accumulator layout of O'^T).
  // The values are divided by the item's denominator: a convex combination of dequantized
  // values, whose magnitude the fp16 value norms bound (the window's tokens too: each enters the
  // pool with an fp16 norm), so fp16 holds them (2^-11 relative, below the bf16 output's
  // rounding) at half the bytes the merge reads.
  f32x4* s_red = (f32x4*)s_big;  // [SWAVES][16][32]
  u32x2v* pvi = (u32x2v*)(a.partial_values + item * 16 * TD);
  for (int hb = 0; hb < G; hb += 8) {
    if (r >= hb && r < hb + 8) {
#pragma unroll
      for (int j = 0; j < 16; ++j) s_red[(wave * 16 + j) * 32 + kq * 8 + r - hb] = acc[j];
    }
    __syncthreads();
    const int t = threadIdx.x, j = t >> 5, e = t & 31;
    if (hb + (e & 7) < G) {
      const int n = hb + (e & 7);
      float Mx = -INFINITY, L = 0.f;
#pragma unroll
      for (int w = 0; w < SWAVES; ++w) Mx = fmaxf(Mx, s_m[w][n]);
#pragma unroll
      for (int w = 0; w < SWAVES; ++w)
        if (s_l[w][n] > 0.f) L += s_l[w][n] * __builtin_amdgcn_exp2f(s_m[w][n] - Mx);
      const float inv = L > 0.f ? 1.0f / L : 0.f;
      f32x4 sum = s_red[j * 32 + e];
#pragma unroll
      for (int w = 1; w < SWAVES; ++w) sum += s_red[(w * 16 + j) * 32 + e];
      const u32x2v o = {pack_f16x2(sum[0] * inv, sum[1] * inv), pack_f16x2(sum[2] * inv, sum[3] * inv)};
      __builtin_nontemporal_store(o, pvi + (hb / 8) * 512 + t);  // streamed: read once, by the merge
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

// grid (B * Hkv * G), one wave per (b, h, query head n): the merge of (b, h)'s items -- the window
// item bh and the packed items item_table[2 bh] .. + item_table[2 bh + 1] - 1 -- for head n, with
// log-sum-exp weights; the packed part is rotated back (R^T o' = s * FWHT(o') / 16), the window
// part added, the sigmoid gate applied.  Lane (j, kq) owns entry (tile j, kq) of the head in the
// partials' layout, dims (4 kq + i) * 16 + j; an LDS transpose puts dims 4 l .. 4 l + 3 in lane l
// for the FWHT.  One wave per head spreads the partial reads over many CUs (one workgroup per
// (b, h) had read all of a sequence's partials through one CU).
template <bool FUSED>
__global__ __launch_bounds__(64) void tq_merge_kernel(const anna_mi_tq_decode_args a, const anna_mi_tq_append_args ap) {
  __shared__ __attribute__((aligned(16))) float s_o[TD], s_w[TD];
  const int lane = threadIdx.x;
  const int G = (int)(a.q_heads / a.kv_heads);
  const int64_t bh = blockIdx.x / G, b = bh / a.kv_heads, h = bh % a.kv_heads;
  const int n = (int)(blockIdx.x % G);
  const int64_t orow = (b * a.q_heads + h * G + n) * TD + 4 * lane;
  // fused: the query row and the new token (independent of the item table), loaded first
  uint2 qraw = make_uint2(0u, 0u), nkraw = make_uint2(0u, 0u), nvraw = make_uint2(0u, 0u);
  if constexpr (FUSED) {
    qraw = *(const uint2*)(a.query + orow);
    nkraw = *(const uint2*)(ap.new_key + bh * TD + 4 * lane);
    nvraw = *(const uint2*)(ap.new_value + bh * TD + 4 * lane);
  }
  constexpr int TS = FUSED ? 4 : 2;  // item table entries per (b, h)
  const int first_item = a.item_table[TS * bh], kb = a.item_table[TS * bh + 1];
  if (!FUSED && first_item < 0) return;  // empty sequence: its window workgroup wrote the zeros
  const int j = lane & 15, kq = lane >> 4;
  constexpr int64_t IS = 16 * TD / 2;  // item stride of partial_values in 4 x fp16 entries
  const int64_t ent = (n / 8) * 512 + j * 32 + kq * 8 + (n % 8);
  const u32x2v* pv = (const u32x2v*)a.partial_values;
  auto f16x4 = [](u32x2v w) {
    return f32x4{f16_bits_to_f32((uint16_t)(w[0] & 0xFFFFu)), f16_bits_to_f32((uint16_t)(w[0] >> 16)),
                 f16_bits_to_f32((uint16_t)(w[1] & 0xFFFFu)), f16_bits_to_f32((uint16_t)(w[1] >> 16))};
  };
  // everything the output needs besides the partials, loaded first
  const float4 sg = *(const float4*)(a.signs + 4 * lane);
  uint2 graw = make_uint2(0u, 0u);
  if (a.gate) graw = *(const uint2*)(a.gate + orow);
  const float2 mlr = *(const float2*)(a.partial_stats + (bh * 16 + n) * 2);
  const u32x2v vr = pv[bh * IS + ent];
  // fused: the codes of the token that left the ring, in its pool slot (written by the split
  // launch): lane l's dims 4 l .. 4 l + 3
  int len0 = 0, stored = 0;
  uint32_t kcode = 0, vcode[4] = {0u, 0u, 0u, 0u}, norms = 0;
  if constexpr (FUSED) {
    const uint8_t* rec = evict_record(a, bh);
    stored = *(const int*)(rec + 132);
    kcode = rec[lane];
    const uint32_t vb = rec[64 + lane];
#pragma unroll
    for (int e = 0; e < 4; ++e) vcode[e] = vb >> (2 * e);
    norms = *(const uint32_t*)(rec + 128);
    len0 = a.item_table[4 * bh + 2];
  }
  const uint16_t knorm = (uint16_t)(norms & 0xFFFFu), vnorm = (uint16_t)(norms >> 16);
  // online log-sum-exp over the packed items, MRG_BATCH at a time with every load issued first
  float M = mlr.y > 0.f ? mlr.x : -INFINITY, L = 0.f;
  f32x4 sp = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < kb; k0 += MRG_BATCH) {
    u32x2v v[MRG_BATCH];
    float2 ml[MRG_BATCH];
#pragma unroll
    for (int k = 0; k < MRG_BATCH; ++k) {
      const int64_t slot = first_item + (k0 + k < kb ? k0 + k : 0);
      v[k] = pv[slot * IS + ent];
      ml[k] = *(const float2*)(a.partial_stats + (slot * 16 + n) * 2);
    }
    __builtin_amdgcn_sched_barrier(0);
    float mb = M;
#pragma unroll
    for (int k = 0; k < MRG_BATCH; ++k)
      if (k0 + k < kb && ml[k].y > 0.f) mb = fmaxf(mb, ml[k].x);
    const float f = mb == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - mb);  // 0 while M is -inf
    sp *= f;
    L *= f;
#pragma unroll
    for (int k = 0; k < MRG_BATCH; ++k) {
      const float wgt = (k0 + k < kb && ml[k].y > 0.f) ? __builtin_amdgcn_exp2f(ml[k].x - mb) : 0.f;
      sp += f16x4(v[k]) * (wgt * ml[k].y);  // the partials are normalized by their denominators
      L += ml[k].y * wgt;
    }
    M = mb;
  }
  // fused: the two tokens of the append, one score each (log2 units): the new one against the
  // query as the window scores it, the leaving one from its codes against the rotated query as
  // the packed items score it; both enter the log-sum-exp with denominator 1
  float we = 0.f, wn = 0.f, vev[4] = {0.f, 0.f, 0.f, 0.f}, vnew[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (FUSED) {
    const float q[4] = {bf16_bits_to_f32((uint16_t)(qraw.x & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(qraw.x >> 16)),
                        bf16_bits_to_f32((uint16_t)(qraw.y & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(qraw.y >> 16))};
    const float kn[4] = {bf16_bits_to_f32((uint16_t)(nkraw.x & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(nkraw.x >> 16)),
                         bf16_bits_to_f32((uint16_t)(nkraw.y & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(nkraw.y >> 16))};
    vnew[0] = bf16_bits_to_f32((uint16_t)(nvraw.x & 0xFFFFu));
    vnew[1] = bf16_bits_to_f32((uint16_t)(nvraw.x >> 16));
    vnew[2] = bf16_bits_to_f32((uint16_t)(nvraw.y & 0xFFFFu));
    vnew[3] = bf16_bits_to_f32((uint16_t)(nvraw.y >> 16));
    // q' = R q (lane: dims 4 lane .. 4 lane + 3), as the packed items rotate it
    float qr[4] = {q[0] * sg.x, q[1] * sg.y, q[2] * sg.z, q[3] * sg.w};
    fwht_wave<4>(qr);
    // the 2-bit centroids, as the score product's fp16 table holds them
    constexpr float C2[4] = {-3.74609375f, -TQ2_A16, TQ2_A16, 3.74609375f};
    float dn = 0.f, de = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dn = __builtin_fmaf(q[e], kn[e], dn);
      de = __builtin_fmaf(qr[e] * (1.0f / 16.0f), C2[(kcode >> (2 * e)) & 3u], de);
      vev[e] = C2[vcode[e] & 3u];
    }
    dn = wave_sum(dn);
    de = wave_sum(de);
    const float sn = dn * (a.scaling * LOG2E);
    const float se = de * (f16_bits_to_f32(knorm) * a.key_scale * a.scaling * LOG2E);
    const float M2 = fmaxf(fmaxf(M, sn), stored ? se : -INFINITY);
    const float f = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - M2);
    sp *= f;
    L *= f;
    M = M2;
    wn = __builtin_amdgcn_exp2f(sn - M);
    we = stored ? __builtin_amdgcn_exp2f(se - M) : 0.f;
    L += wn + we;
    const float vs = stored ? f16_bits_to_f32(vnorm) * a.value_scale : 0.f;  // the record is stale otherwise
#pragma unroll
    for (int e = 0; e < 4; ++e) vev[e] *= vs;
  }
  const float wr_w = mlr.y > 0.f ? __builtin_amdgcn_exp2f(mlr.x - M) : 0.f;
  L += mlr.y * wr_w;
  const float invL = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int dim = (4 * kq + i) * 16 + j;
    s_o[dim] = sp[i] * invL;
    s_w[dim] = f16x4(vr)[i] * (wr_w * mlr.y) * invL;
  }
  __syncthreads();
  // out = R^T o' + window part = s * FWHT(o') / 16 + w, times sigmoid(gate)
  float v[4];
  const float4 o4 = *(const float4*)(s_o + 4 * lane);
  v[0] = o4.x, v[1] = o4.y, v[2] = o4.z, v[3] = o4.w;
  if constexpr (FUSED) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += vev[e] * (we * invL);
  }
  fwht_wave<4>(v);
  const float4 w4 = *(const float4*)(s_w + 4 * lane);
  const float sgv[4] = {sg.x, sg.y, sg.z, sg.w};
  float wv[4] = {w4.x, w4.y, w4.z, w4.w};
  if constexpr (FUSED) {
#pragma unroll
    for (int e = 0; e < 4; ++e) wv[e] += vnew[e] * (wn * invL);
  }
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = v[e] * sgv[e] * (1.0f / 16.0f) + wv[e];
  if (a.gate) {
    const float gv[4] = {bf16_bits_to_f32((uint16_t)(graw.x & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(graw.x >> 16)),
                         bf16_bits_to_f32((uint16_t)(graw.y & 0xFFFFu)), bf16_bits_to_f32((uint16_t)(graw.y >> 16))};
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = o[e] / (1.0f + __expf(-gv[e]));
  }
  *(uint2*)(a.out + orow) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
  if constexpr (FUSED) {
    // the new token takes the ring slot the leaving one had; the length grows (no wave of this
    // launch reads the ring or the lengths)
    if (n == 0) {
      const int64_t R = a.residual_capacity, rpos = len0 % R;
      *(uint2*)(ap.residual_key + (bh * R + rpos) * TD + 4 * lane) = nkraw;
      uint16_t* col = ap.residual_value_t + bh * TD * R + rpos;
      col[(4 * lane + 0) * R] = (uint16_t)(nvraw.x & 0xFFFFu);
      col[(4 * lane + 1) * R] = (uint16_t)(nvraw.x >> 16);
      col[(4 * lane + 2) * R] = (uint16_t)(nvraw.y & 0xFFFFu);
      col[(4 * lane + 3) * R] = (uint16_t)(nvraw.y >> 16);
      if (h == 0 && lane == 0) ap.seq_lengths[b] = len0 + 1;
    }
  }
}

// ------------------------------------------------------------------ append

// One workgroup (4 waves) per sequence.  Wave w quantizes vector w of {K, V} x kv heads that
// leaves the ring (when length >= R), all waves then write the new token into the ring slot,
// thread 0 increments the length.
__global__ __launch_bounds__(256) void tq_append_kernel(const anna_mi_tq_append_args a) {
  const int wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b = blockIdx.x, H = a.kv_heads, R = a.residual_capacity;
  const int n = a.seq_lengths[b];
  const int64_t rpos = n % R;
  if (n >= R) {
    const int64_t q = n - R;
    const bool room = q < a.seq_capacity[b];
    if (!room) {
      if (threadIdx.x == 0 && a.overflow) *a.overflow = 1;
    } else {
      for (int64_t vi = wave; vi < 2 * H; vi += 4)
        evict_token(a, b, vi >> 1, n, a.seq_offsets[b] + q, vi & 1, threadIdx.x & 63);
    }
  }
  __syncthreads();  // the leaving token is read before its slot is overwritten
  for (int64_t i = threadIdx.x; i < H * TD; i += blockDim.x) {
    const int64_t h = i / TD, d = i % TD;
    a.residual_key[((b * H + h) * R + rpos) * TD + d] = a.new_key[(b * H + h) * TD + d];
    a.residual_value_t[((b * H + h) * TD + d) * R + rpos] = a.new_value[(b * H + h) * TD + d];
  }
  if (threadIdx.x == 0) a.seq_lengths[b] = n + 1;
}


// ------------------------------------------------------------------ pack (prefill)

// K and V of `tokens` tokens of every KV head into the pool (one launch): wave w of the grid
// takes 4 consecutive tokens t0 .. t0 + 3 of one (head, K or V) (the four tokens of one byte of
// the blocked value layout), quantizes them with the Hadamard quantizer (bit-exact with
// anna_mi_tq_hadamard_quantize) and writes key codes token-major, value codes in the 32-token
// blocked layout, and the fp16 norms.
template <int QPW>  // quads of 4 tokens per wave: their vectors go through the transform together
__global__ __launch_bounds__(256) void tq_pack_kv_kernel(const anna_mi_tq_pack_args a) {
  constexpr int NV = 4 * QPW;
  const int lane = threadIdx.x & 63;
  const int64_t groups = (a.tokens + NV - 1) / NV;
  // the wave index through readfirstlane: everything derived from it (token, head, addresses) is
  // then wave-uniform and computed on the scalar unit, not per lane (the kernel is VALU-bound)
  const int64_t wid = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wid >= 2 * a.kv_heads * groups) return;  // whole wave
  const int64_t g = wid % groups, hv = wid / groups, h = hv >> 1;
  const bool is_v = hv & 1;
  const int64_t t0 = g * NV;
  const uint16_t* src = (is_v ? a.values : a.keys) + h * a.stride_head;
  float xv[NV][4];
  uint2 raw[NV];
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const int64_t t = t0 + n < a.tokens ? t0 + n : a.tokens - 1;  // tail: repeats the last token
    raw[n] = *(const uint2*)(src + t * a.stride_token + 4 * lane);
  }
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    xv[n][0] = bf16_bits_to_f32((uint16_t)(raw[n].x & 0xFFFFu));
    xv[n][1] = bf16_bits_to_f32((uint16_t)(raw[n].x >> 16));
    xv[n][2] = bf16_bits_to_f32((uint16_t)(raw[n].y & 0xFFFFu));
    xv[n][3] = bf16_bits_to_f32((uint16_t)(raw[n].y >> 16));
  }
  uint32_t code[NV][4];
  float nrm[NV];
  hadamard_codes_wave_n<NV, 4>(xv, a.signs, a.thresholds, 3, 1.0f / 16.0f, code, nrm);
  const int64_t T = a.pool_tokens, slot0 = a.slot_offset + t0;
  const int nvalid = a.tokens - t0 < NV ? (int)(a.tokens - t0) : NV;
  float nrm_lane = 0.f;  // lanes 0 .. NV - 1 store the norms
#pragma unroll
  for (int n = 0; n < NV; ++n) nrm_lane = lane == n ? nrm[n] : nrm_lane;
  if (!is_v) {
#pragma unroll
    for (int n = 0; n < NV; ++n)
      if (n < nvalid)
        a.key_codes[(h * T + slot0 + n) * 64 + lane] =
            (uint8_t)(code[n][0] | (code[n][1] << 2) | (code[n][2] << 4) | (code[n][3] << 6));
    if (lane < nvalid) a.key_norms[h * T + slot0 + lane] = f32_to_f16_bits(nrm_lane);
  } else {
    // slot0 % 4 == 0: quad q fills bits 0..7 of one byte per dim
#pragma unroll
    for (int q = 0; q < QPW; ++q) {
      if (4 * q >= nvalid) break;
      const int64_t sq = slot0 + 4 * q, t = sq % TBT;
      uint8_t* blk = a.value_codes + (h * (T / TBT) + sq / TBT) * 2048 + ((t % 16) / 4) * 512 + (t / 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t byte = 0;
#pragma unroll
        for (int n = 0; n < 4; ++n)
          if (4 * q + n < nvalid) byte |= code[4 * q + n][e] << (2 * n);
        blk[(4 * lane + e) * 2] = (uint8_t)byte;
      }
    }
    if (lane < nvalid) a.value_norms[h * T + slot0 + lane] = f32_to_f16_bits(nrm_lane);
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
extern "C" int64_t anna_mi_sizeof_tq_append_args(void) { return (int64_t)sizeof(anna_mi_tq_append_args); }

extern "C" int64_t anna_mi_tq_decode_workgroups(int64_t batch, int64_t kv_heads, const int64_t* pool_capacity,
                                                int64_t blocks_per_item) {
  if (batch <= 0 || kv_heads <= 0) return 0;
  const int64_t bh = batch * kv_heads;
  // one 512-thread item per MI355X compute unit at a time (232 VGPRs: two waves per SIMD), so
  // up to 256 workgroups run in one round; 224 (longer items, fewer partials for the merge)
  // measured best at config 4 (21.8 us per call against 22.8 with 256; 208: 21.8, 192: 23.0,
  // 240: 22.7); >= 2 bh + 1 so that any lengths fit (see plan_item)
  constexpr int64_t SLOTS = 224;
  const int64_t automatic = SLOTS > 2 * bh ? SLOTS : 2 * bh + 1;
  if (blocks_per_item <= 0) return automatic;
  int64_t n = 0;
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t nb = (pool_capacity[b] + TBT - 1) / TBT;
    n += (nb + blocks_per_item - 1) / blocks_per_item;
  }
  return bh + n * kv_heads > automatic ? bh + n * kv_heads : automatic;
}

namespace {
int check_decode_args(const anna_mi_tq_decode_args& a) {
  ANNA_CHECK(a.head_dim == TD, "anna_mi_tq_decode: head_dim must be 256");
  ANNA_CHECK(a.key_bits == 2 && a.value_bits == 2, "anna_mi_tq_decode: 2-bit codes only (use anna_mi_gqa_decode_splitkv)");
  ANNA_CHECK(a.batch > 0 && a.batch <= MAX_SEQS, "anna_mi_tq_decode: batch must be in [1, %d]", MAX_SEQS);
  ANNA_CHECK(a.kv_heads > 0 && a.q_heads % a.kv_heads == 0 && a.q_heads / a.kv_heads <= 16,
             "anna_mi_tq_decode: need q_heads = G * kv_heads with G <= 16");
  ANNA_CHECK(a.pool_tokens % TBT == 0 && a.residual_capacity % TBT == 0 && a.residual_capacity > 0,
             "pool and residual capacity must be positive multiples of 32");
  ANNA_CHECK(a.pool_tokens < ((int64_t)1 << 31), "anna_mi_tq_decode: pool slots exceed int32");
  ANNA_CHECK(a.num_workgroups > 2 * a.batch * a.kv_heads && a.num_workgroups < ((int64_t)1 << 31),
             "anna_mi_tq_decode: num_workgroups must come from anna_mi_tq_decode_workgroups");
  ANNA_CHECK(a.query && a.out && a.partial_stats && a.partial_values && a.item_table && a.seq_offsets && a.seq_lengths &&
                 a.signs,
             "anna_mi_tq_decode: null pointer");
  ANNA_CHECK(a.key_codes && a.key_norms && a.value_codes && a.value_norms && a.residual_key && a.residual_value_t,
             "anna_mi_tq_decode: null cache pointer");
  return ANNA_MI_OK;
}

int check_append_args(const anna_mi_tq_append_args& a) {
  ANNA_CHECK(a.head_dim == TD, "anna_mi_tq_append: head_dim must be 256");
  ANNA_CHECK(a.batch > 0 && a.kv_heads > 0, "anna_mi_tq_append: empty batch or heads");
  ANNA_CHECK(a.pool_tokens % TBT == 0 && a.residual_capacity % TBT == 0 && a.residual_capacity > 0,
             "pool and residual capacity must be positive multiples of 32");
  ANNA_CHECK(a.new_key && a.new_value && a.key_codes && a.key_norms && a.value_codes && a.value_norms &&
                 a.residual_key && a.residual_value_t && a.seq_offsets && a.seq_capacity && a.seq_lengths && a.signs &&
                 a.thresholds,
             "anna_mi_tq_append: null pointer");
  return ANNA_MI_OK;
}
}  // namespace

extern "C" int anna_mi_tq_decode(const anna_mi_tq_decode_args* ap, void* stream) {
  ANNA_CHECK(ap != nullptr, "anna_mi_tq_decode: null args");
  const anna_mi_tq_decode_args& a = *ap;
  if (const int rc = check_decode_args(a)) return rc;
  const anna_mi_tq_append_args none{};
  hipLaunchKernelGGL(tq_decode_kernel<false>, dim3((unsigned)a.num_workgroups), dim3(64 * SWAVES), 0, as_stream(stream),
                     a, none);
  ANNA_LAUNCH_CHECK("tq_decode_kernel");
  hipLaunchKernelGGL(tq_merge_kernel<false>, dim3((unsigned)(a.q_heads * a.batch)), dim3(64), 0, as_stream(stream), a,
                     none);
  ANNA_LAUNCH_CHECK("tq_merge_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_append_decode(const anna_mi_tq_decode_args* dp, const anna_mi_tq_append_args* app,
                                        void* stream) {
  ANNA_CHECK(dp != nullptr && app != nullptr, "anna_mi_tq_append_decode: null args");
  const anna_mi_tq_decode_args& a = *dp;
  const anna_mi_tq_append_args& p = *app;
  if (const int rc = check_decode_args(a)) return rc;
  if (const int rc = check_append_args(p)) return rc;
  ANNA_CHECK(p.batch == a.batch && p.kv_heads == a.kv_heads && p.head_dim == a.head_dim &&
                 p.pool_tokens == a.pool_tokens && p.residual_capacity == a.residual_capacity,
             "anna_mi_tq_append_decode: the append and decode arguments describe different caches");
  ANNA_CHECK(p.key_codes == a.key_codes && p.key_norms == a.key_norms && p.value_codes == a.value_codes &&
                 p.value_norms == a.value_norms && p.residual_key == a.residual_key &&
                 p.residual_value_t == a.residual_value_t && p.seq_offsets == a.seq_offsets &&
                 p.seq_lengths == a.seq_lengths && p.signs == a.signs,
             "anna_mi_tq_append_decode: the append and decode arguments describe different caches");
  hipLaunchKernelGGL(tq_decode_kernel<true>, dim3((unsigned)a.num_workgroups), dim3(64 * SWAVES), 0, as_stream(stream),
                     a, p);
  ANNA_LAUNCH_CHECK("tq_decode_kernel (fused append)");
  hipLaunchKernelGGL(tq_merge_kernel<true>, dim3((unsigned)(a.q_heads * a.batch)), dim3(64), 0, as_stream(stream), a, p);
  ANNA_LAUNCH_CHECK("tq_merge_kernel (fused append)");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_append(const anna_mi_tq_append_args* ap, void* stream) {
  ANNA_CHECK(ap != nullptr, "anna_mi_tq_append: null args");
  const anna_mi_tq_append_args& a = *ap;
  if (const int rc = check_append_args(a)) return rc;
  hipLaunchKernelGGL(tq_append_kernel, dim3((unsigned)a.batch), dim3(256), 0, as_stream(stream), a);
  ANNA_LAUNCH_CHECK("tq_append_kernel");
  return ANNA_MI_OK;
}

extern "C" int64_t anna_mi_sizeof_tq_pack_args(void) { return (int64_t)sizeof(anna_mi_tq_pack_args); }

extern "C" int anna_mi_tq_pack_kv(const anna_mi_tq_pack_args* ap, void* stream) {
  ANNA_CHECK(ap != nullptr, "anna_mi_tq_pack_kv: null args");
  const anna_mi_tq_pack_args& a = *ap;
  ANNA_CHECK(a.head_dim == TD, "anna_mi_tq_pack_kv: head_dim must be 256");
  ANNA_CHECK(a.keys && a.values && a.key_codes && a.key_norms && a.value_codes && a.value_norms && a.signs &&
                 a.thresholds,
             "anna_mi_tq_pack_kv: null pointer");
  ANNA_CHECK(a.kv_heads > 0 && a.tokens >= 0, "anna_mi_tq_pack_kv: bad sizes");
  ANNA_CHECK(a.slot_offset % TBT == 0 && a.pool_tokens % TBT == 0 && a.slot_offset + a.tokens <= a.pool_tokens,
             "anna_mi_tq_pack_kv: slots must start at a multiple of 32 and fit the pool");
  ANNA_CHECK(a.stride_token >= TD && a.stride_token % 4 == 0 && a.stride_head % 4 == 0 &&
                 (uintptr_t)a.keys % 8 == 0 && (uintptr_t)a.values % 8 == 0,
             "anna_mi_tq_pack_kv: rows must be 8-byte aligned with a stride of at least 256");
  if (a.tokens == 0) return ANNA_MI_OK;
  // one quad per wave: the kernel is VALU-bound (about 600 VALU instructions per wave at 8
  // waves per SIMD), and two quads per wave measured slower (fewer waves to hide the exchanges)
  constexpr int QPW = 1;
  const int64_t waves = 2 * a.kv_heads * ((a.tokens + 4 * QPW - 1) / (4 * QPW));
  hipLaunchKernelGGL(tq_pack_kv_kernel<QPW>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, as_stream(stream), a);
  ANNA_LAUNCH_CHECK("tq_pack_kv_kernel");
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
