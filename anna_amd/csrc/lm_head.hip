// Tiled int4 GEMV (the LM-head weight layout) and the fused LM-head top-k on gfx950.
//
// Layout (reference quantization.py:491-538, sycl:3272-3343): qweight int32 [N/T][Kp/8][T]
// (T = 1, 2, 4, 8; T = 1 is the plain [N][Kp/8] layout), row n = T * tile + t, word w of row n
// at [tile][w][t]; scale / zero point of (group g, row n) at g * ss_g + n * ss_n, which covers
// [G][N] (ss_g = N, ss_n = 1; also the tiled [G][N/T][T]) and the LM-head top-k layout [N][G]
// (ss_g = 1, ss_n = G).  w = (q - z) * s.
//
//   int4_gemv_tiled_kernel  one wave per tile: lane l walks words l, l + 64, ... of the tile;
//                           each word is one T x 4-byte coalesced load (8 k of T rows) used
//                           against 8 activations of up to MR rows; fp32 accumulation
//                           (s * (sum x q - z sum x) per word), wave reduction at the end.
//   int4_gemv_tiled_lds_kernel  (1..4 rows) the same with x and the tile scales and zero points
//                           staged in LDS: one memory load per weight word.
//   topk_rows_kernel        k <= 8, per row, 1024 threads: pass 1 takes each thread's maximum and
//                           merges the maxima into a top-k list; its k-th entry bounds the row's
//                           k-th best from below.  Pass 2 keeps only the logits at or above that
//                           bound in sorted register lists, merged pairwise through LDS by a
//                           bitonic merge (value descending, ties to the lower index).
//   topk_rows_lds_kernel    k > 8: the same bound, the sorted lists in LDS.
//   topk_chunk_wave_kernel, topk_merge_waves_kernel   k <= 8, few long rows (the fused LM head):
//                           one wave per 1024 logits keeps register lists whose heads a
//                           tournament across the lanes pops in order; one wave per row merges
//                           the chunk lists the same way.
#include <type_traits>

#include "common.hpp"
#include "int4_frag.hpp"

namespace anna {
namespace {

constexpr int TG_MR = 4;  // activation rows per weight pass

template <int T>
struct TileWords {
  uint32_t v[T];
};

template <int T>
__device__ __forceinline__ TileWords<T> load_tile_words(const uint32_t* p) {
  // the weights are read once per call: non-temporal loads
  TileWords<T> r;
  if constexpr (T == 8) {
    const u32x4 a = __builtin_nontemporal_load((const u32x4*)p), b = __builtin_nontemporal_load((const u32x4*)(p + 4));
    r.v[0] = a.x, r.v[1] = a.y, r.v[2] = a.z, r.v[3] = a.w, r.v[4] = b.x, r.v[5] = b.y, r.v[6] = b.z, r.v[7] = b.w;
  } else if constexpr (T == 4) {
    const u32x4 a = __builtin_nontemporal_load((const u32x4*)p);
    r.v[0] = a.x, r.v[1] = a.y, r.v[2] = a.z, r.v[3] = a.w;
  } else if constexpr (T == 2) {
    typedef uint32_t u32x2t __attribute__((ext_vector_type(2)));
    const u32x2t a = __builtin_nontemporal_load((const u32x2t*)p);
    r.v[0] = a[0], r.v[1] = a[1];
  } else {
    r.v[0] = __builtin_nontemporal_load(p);
  }
  return r;
}

// OUT_F32: y is fp32 (logits); otherwise y is in the activation dtype.
template <int XDT, int SDT, int T, bool OUT_F32>
__global__ __launch_bounds__(256) void int4_gemv_tiled_kernel(
    const typename Elem<XDT>::T* __restrict__ x, int64_t M, int64_t K, int64_t xs, const uint32_t* __restrict__ qw,
    int64_t tiles, int64_t pc, const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz,
    int64_t ss_g, int64_t ss_n, int64_t gsz, int64_t N, void* __restrict__ y, int64_t ys) {
  const int lane = threadIdx.x & 63;
  const int64_t tile = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (tile >= tiles) return;
  const int64_t words = (K + 7) / 8;
  const bool vec_x = (K % 8) == 0 && (xs % 8) == 0;
  const uint32_t* tw = qw + tile * pc * T;
  for (int64_t m0 = 0; m0 < M; m0 += TG_MR) {
    float acc[TG_MR][T];
#pragma unroll
    for (int m = 0; m < TG_MR; ++m)
#pragma unroll
      for (int t = 0; t < T; ++t) acc[m][t] = 0.f;
    bool fast = false;
    if constexpr (XDT != ANNA_MI_F32) {
      if (vec_x) {
        // Words w and w + 64 of the lane alternate between two register sets: the loads of the
        // next word (weights, raw scales and zero points, x) are issued before the current one
        // is used, pinned there by a scheduling barrier (converted right at their loads, each
        // word cost a full round trip)
        using ST = typename Elem<SDT>::T;
        struct Word {
          TileWords<T> q;
          ST s[T];
          int8_t z[T];
          u32x4 x[TG_MR];
        };
        auto load = [&](int64_t w, Word& D) {
          D.q = load_tile_words<T>(tw + w * T);
          const int64_t g = (w * 8) / gsz;
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const int64_t n = tile * T + t;
            const int64_t nc = n < N ? n : 0;
            D.s[t] = qs[g * ss_g + nc * ss_n];
            D.z[t] = qz[g * ss_g + nc * ss_n];
          }
#pragma unroll
          for (int m = 0; m < TG_MR; ++m) {
            const int64_t mr = m0 + m < M ? m0 + m : m0;
            D.x[m] = *(const u32x4*)((const uint16_t*)x + mr * xs + w * 8);
          }
        };
        // Nibble pairs become 16-bit "off + q" values with one AND-OR (exact), dot2 accumulates them
        // in fp32 against x reordered to the same pairs, and the zero point comes off once per
        // word and row: s * (sum x (off + q) - (off + z) sum x).
        constexpr float OFF = XDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
        constexpr uint32_t ONES = XDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
        auto compute = [&](const Word& D) {
#pragma unroll
          for (int m = 0; m < TG_MR; ++m) {
            if (m0 + m >= M) continue;
            const u32x4 xi = interleave_x(D.x[m]);
            float sx = dot2_acc<XDT>(xi.x, ONES, 0.f);
            sx = dot2_acc<XDT>(xi.y, ONES, sx);
            sx = dot2_acc<XDT>(xi.z, ONES, sx);
            sx = dot2_acc<XDT>(xi.w, ONES, sx);
#pragma unroll
            for (int t = 0; t < T; ++t) {
              const u32x4 f = nibbles_to_frag<XDT>(D.q.v[t]);
              float d = dot2_acc<XDT>(xi.x, f.x, 0.f);
              d = dot2_acc<XDT>(xi.y, f.y, d);
              d = dot2_acc<XDT>(xi.z, f.z, d);
              d = dot2_acc<XDT>(xi.w, f.w, d);
              acc[m][t] = fmaf(Elem<SDT>::to_f32(D.s[t]), d - (OFF + (float)D.z[t]) * sx, acc[m][t]);
            }
          }
        };
        Word A, B;
        int64_t w = lane;
        if (w < words) load(w, A);
        for (; w < words; w += 128) {
          if (w + 64 < words) load(w + 64, B);
          __builtin_amdgcn_sched_barrier(0);
          compute(A);
          if (w + 64 >= words) break;
          if (w + 128 < words) load(w + 128, A);
          __builtin_amdgcn_sched_barrier(0);
          compute(B);
        }
        fast = true;
      }
    }
    for (int64_t w = lane; !fast && w < words; w += 64) {
      const TileWords<T> q = load_tile_words<T>(tw + w * T);
      const int64_t k0 = w * 8;
      const int64_t g = k0 / gsz;
      float s[T], z[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int64_t n = tile * T + t;
        const int64_t nc = n < N ? n : 0;
        s[t] = Elem<SDT>::load(qs, g * ss_g + nc * ss_n);
        z[t] = (float)qz[g * ss_g + nc * ss_n];
      }
#pragma unroll
      for (int m = 0; m < TG_MR; ++m) {
        if (m0 + m >= M) continue;
        float xv[8];
        const int64_t row = (m0 + m) * xs;
        bool done = false;
        if constexpr (XDT != ANNA_MI_F32) {
          if (vec_x) {
            const u32x4 v = *(const u32x4*)((const uint16_t*)x + row + k0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              xv[2 * e] = Elem<XDT>::to_f32((uint16_t)(v[e] & 0xFFFFu));
              xv[2 * e + 1] = Elem<XDT>::to_f32((uint16_t)(v[e] >> 16));
            }
            done = true;
          }
        }
        if (!done) {
#pragma unroll
          for (int e = 0; e < 8; ++e) xv[e] = k0 + e < K ? Elem<XDT>::load(x, row + k0 + e) : 0.f;
        }
        float sx = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sx += xv[e];
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(xv[e], (float)((q.v[t] >> (4 * e)) & 0xFu), d);
          acc[m][t] = fmaf(s[t], d - z[t] * sx, acc[m][t]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < TG_MR; ++m) {
      if (m0 + m >= M) continue;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float v = wave_sum_rows(acc[m][t]);
        const int64_t n = tile * T + t;
        if (lane == 0 && n < N) {
          if constexpr (OUT_F32) ((float*)y)[(m0 + m) * ys + n] = v;
          else ((typename Elem<XDT>::T*)y)[(m0 + m) * ys + n] = Elem<XDT>::cvt(v);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ top-k

constexpr int TK_MAX = 32;         // top_k handled per call (larger k: error)
constexpr int TK_LDS = 64 * 1024;  // bytes of the per-thread lists (value + index, KT each)
constexpr int TK_BATCH = 16;       // values one thread loads before it looks at any

__device__ __forceinline__ bool tk_better(float va, int32_t ia, float vb, int32_t ib) {
  return va > vb || (va == vb && ia < ib);
}

// compare-exchange: (a) ends up the better of the two
__device__ __forceinline__ void tk_ce(float& va, int32_t& ia, float& vb, int32_t& ib) {
  if (tk_better(vb, ib, va, ia)) {
    const float tv = va;
    const int32_t ti = ia;
    va = vb, ia = ib, vb = tv, ib = ti;
  }
}

// Threads per row for register lists of KT entries: the most (a power of two, <= 1024) whose
// lists fit TK_LDS.
inline int tk_threads(int kt) { return TK_LDS / (kt * 8) < 1024 ? TK_LDS / (kt * 8) : 1024; }

// k <= 8 (KT = 8).  grid (rows), tk_threads(KT) threads, dynamic LDS nt * KT * 8 bytes.  The values are fp32
// [rows][ld]; out values in ODT.  Order: descending, ties to the lower index (a strict total
// order, so the networks below give exactly the sorted top-k).
//   bound  a first pass finds each thread's best; the k-th best of those bounds the answer;
//   scan   each thread keeps the KT best of its strided share that pass the bound, sorted in
//          registers (a new entry replaces the last and bubbles up: static indices, no LDS),
//          loading TK_BATCH values before it compares any;
//   merge  pairwise tree over the threads' lists through LDS: a thread reads its partner's list
//          (independent loads), keeps the better of A[i] and B[KT-1-i] (the top half of the
//          bitonic A ++ reverse(B)) and sorts that half with a bitonic network, in registers.
// The earlier form (lists in LDS, a two-pointer merge) spent its time in chains of dependent
// LDS reads: 24 us at V = 31, 240 us at V = 151936.
// (Few long rows take the wave-level chunk kernels below instead.)  Elements [blockIdx.x S,
// blockIdx.x S + S) of the row, clipped to V (S = V: the whole row).
template <int ODT, int KT>
__global__ __launch_bounds__(1024) void topk_rows_kernel(float* __restrict__ logits, int64_t V, int64_t ld, int k,
                                                         typename Elem<ODT>::T* __restrict__ out_v,
                                                         int64_t* __restrict__ out_i, int64_t S) {
  extern __shared__ float tk_lists[];  // values [nt][KT], then indices [nt][KT]
  const int nt = blockDim.x, tid = threadIdx.x;
  const int64_t row = blockIdx.y;
  float* const lg = logits + row * ld;
  const int64_t lo = (int64_t)blockIdx.x * S, hi = lo + S < V ? lo + S : V;
  float* lv = tk_lists;
  int32_t* li = (int32_t*)(tk_lists + nt * KT);
  float rv[KT];
  int32_t ri[KT];
  auto clear = [&]() {
#pragma unroll
    for (int j = 0; j < KT; ++j) rv[j] = -INFINITY, ri[j] = INT32_MAX;
  };
  // the threads' register lists -> thread 0's list (in LDS too) holds the best KT of them all
  auto merge_tree = [&]() {
#pragma unroll
    for (int j = 0; j < KT; ++j) lv[tid * KT + j] = rv[j], li[tid * KT + j] = ri[j];
    __syncthreads();
    for (int half = nt / 2; half >= 1; half >>= 1) {
      if (tid < half) {
        float bv[KT];
        int32_t bi[KT];
#pragma unroll
        for (int j = 0; j < KT; ++j) bv[j] = lv[(tid + half) * KT + j], bi[j] = li[(tid + half) * KT + j];
#pragma unroll
        for (int j = 0; j < KT; ++j) {
          if (tk_better(bv[KT - 1 - j], bi[KT - 1 - j], rv[j], ri[j])) rv[j] = bv[KT - 1 - j], ri[j] = bi[KT - 1 - j];
        }
#pragma unroll
        for (int s = KT / 2; s >= 1; s >>= 1)
#pragma unroll
          for (int j = 0; j < KT; ++j)
            if ((j & s) == 0) tk_ce(rv[j], ri[j], rv[j + s], ri[j + s]);
#pragma unroll
        for (int j = 0; j < KT; ++j) lv[tid * KT + j] = rv[j], li[tid * KT + j] = ri[j];
      }
      __syncthreads();
    }
  };
  // pass 1: the k-th best of the threads' maxima bounds the row's k-th best from below (k
  // distinct elements are at least as good), so pass 2 skips everything worse than it and its
  // lists rarely change (a wave whose lanes insert often walks the insertion for all of them)
  float mxv = -INFINITY;
  int32_t mxi = INT32_MAX;
  for (int64_t n0 = lo + tid; n0 < hi; n0 += (int64_t)TK_BATCH * nt) {
    float v[TK_BATCH];
#pragma unroll
    for (int b = 0; b < TK_BATCH; ++b) {
      const int64_t n = n0 + (int64_t)b * nt;
      v[b] = lg[n < hi ? n : lo];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < TK_BATCH; ++b) {
      const int64_t n = n0 + (int64_t)b * nt;
      if (n < hi && tk_better(v[b], (int32_t)n, mxv, mxi)) mxv = v[b], mxi = (int32_t)n;
    }
  }
  clear();
  rv[0] = mxv, ri[0] = mxi;
  merge_tree();
  const float tau_v = lv[k - 1];
  const int32_t tau_i = li[k - 1];
  __syncthreads();  // everyone has read the bound before the lists are rewritten
  // pass 2: each thread keeps the KT best of its share that are not worse than the bound,
  // sorted in registers (a new entry replaces the last and bubbles up)
  clear();
  for (int64_t n0 = lo + tid; n0 < hi; n0 += (int64_t)TK_BATCH * nt) {
    float v[TK_BATCH];
#pragma unroll
    for (int b = 0; b < TK_BATCH; ++b) {
      const int64_t n = n0 + (int64_t)b * nt;
      v[b] = lg[n < hi ? n : lo];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < TK_BATCH; ++b) {
      const int64_t n = n0 + (int64_t)b * nt;
      if (n >= hi || tk_better(tau_v, tau_i, v[b], (int32_t)n) || !tk_better(v[b], (int32_t)n, rv[KT - 1], ri[KT - 1]))
        continue;
      rv[KT - 1] = v[b], ri[KT - 1] = (int32_t)n;
#pragma unroll
      for (int j = KT - 1; j >= 1; --j) tk_ce(rv[j - 1], ri[j - 1], rv[j], ri[j]);
    }
  }
  merge_tree();
  if (tid < k) {  // the merged list is thread 0's
    out_v[row * k + tid] = Elem<ODT>::cvt(lv[tid]);
    out_i[row * k + tid] = li[tid];
  }
}

// Wave-level top-8 for few long rows.  Every lane keeps a sorted list (best first) of the
// elements it reads; then eight rounds of a tournament over the lanes' list heads (a six-step
// xor-shuffle arg-best, every lane ending with the winner) emit the wave's best 8 in order, the
// lane that held each winner popping its head.  Order: larger value first, then smaller index
// (tk_better); indices are unique, so the winner's lane is the one whose head carries its index.
// (Butterfly merges of whole 8-lists between lanes cost about twice as long.)
__device__ __forceinline__ void tk8_insert(float (&rv)[8], int32_t (&ri)[8], float v, int32_t i) {
  if (!tk_better(v, i, rv[7], ri[7])) return;
  rv[7] = v, ri[7] = i;
#pragma unroll
  for (int j = 7; j >= 1; --j) tk_ce(rv[j - 1], ri[j - 1], rv[j], ri[j]);
}

// Value of a lane's DPP partner (a symmetric pairing inside 16-lane rows: quad permutes, the
// half-row and the row mirror); one VALU move, no trip through the LDS pipe.
template <int CTRL>
__device__ __forceinline__ int32_t tk_dpp(int32_t v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

// Arg-best over the wave, every lane ending with the winner: four DPP pairings inside each
// 16-lane row (xor 1, xor 2, then i <-> 7 - i and i <-> 15 - i, which pair the quads and the
// halves), then the two row swaps.  (Six xor shuffles chained twelve LDS-pipe round trips per
// winner.)
__device__ __forceinline__ void tk_wave_best(float& bv, int32_t& bi) {
  auto take = [&](float pv, int32_t pi) {
    if (tk_better(pv, pi, bv, bi)) bv = pv, bi = pi;
  };
  take(__int_as_float(tk_dpp<0xB1>(__float_as_int(bv))), tk_dpp<0xB1>(bi));    // quad_perm [1, 0, 3, 2]
  take(__int_as_float(tk_dpp<0x4E>(__float_as_int(bv))), tk_dpp<0x4E>(bi));    // quad_perm [2, 3, 0, 1]
  take(__int_as_float(tk_dpp<0x141>(__float_as_int(bv))), tk_dpp<0x141>(bi));  // row_half_mirror
  take(__int_as_float(tk_dpp<0x140>(__float_as_int(bv))), tk_dpp<0x140>(bi));  // row_mirror
  take(lane_xor16(bv), lane_xor16(bi));
  take(lane_xor32(bv), lane_xor32(bi));
}

__device__ __forceinline__ void tk8_wave_tournament(float (&rv)[8], int32_t (&ri)[8], float (&ov)[8], int32_t (&oi)[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    float bv = rv[0];
    int32_t bi = ri[0];
    tk_wave_best(bv, bi);
    ov[r] = bv, oi[r] = bi;
    if (ri[0] == bi) {
#pragma unroll
      for (int j = 0; j < 7; ++j) rv[j] = rv[j + 1], ri[j] = ri[j + 1];
      rv[7] = -INFINITY, ri[7] = INT32_MAX;
    }
  }
}

// grid (C, rows), one wave per chunk: chunk c is [c S, c S + S), the last one [(C - 1) S, V)
// (at least 16 elements: the host folds a shorter tail into it).  The chunk's best 8 are written
// over its first 16 floats (values, then the indices' bits; the wave has read the chunk by then)
// for topk_merge_waves_kernel.
constexpr int TKW_PER = 16;  // elements per lane and batch of loads
__global__ __launch_bounds__(64) void topk_chunk_wave_kernel(float* __restrict__ logits, int64_t V, int64_t ld,
                                                             int64_t S) {
  const int lane = threadIdx.x;
  float* const lg = logits + (int64_t)blockIdx.y * ld;
  const int64_t lo = (int64_t)blockIdx.x * S, hi = blockIdx.x + 1 == gridDim.x ? V : lo + S;
  float rv[8];
  int32_t ri[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) rv[j] = -INFINITY, ri[j] = INT32_MAX;
  for (int64_t n0 = lo + lane; n0 < hi; n0 += 64 * TKW_PER) {
    float v[TKW_PER];
#pragma unroll
    for (int j = 0; j < TKW_PER; ++j) {
      const int64_t n = n0 + 64 * j;
      v[j] = lg[n < hi ? n : lo];
    }
#pragma unroll
    for (int j = 0; j < TKW_PER; ++j) {
      const int64_t n = n0 + 64 * j;
      if (n < hi) tk8_insert(rv, ri, v[j], (int32_t)n);
    }
  }
  float ov[8];
  int32_t oi[8];
  tk8_wave_tournament(rv, ri, ov, oi);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (lane == j) {
      lg[lo + j] = ov[j];
      lg[lo + 8 + j] = __int_as_float(oi[j]);
    }
}

// grid (rows), TKM_WAVES waves per row: the C chunk lists of topk_chunk_wave_kernel merged the same
// way, in two levels -- wave w takes the w-th share of the C * 8 candidates (a few per lane) to its
// best 8, and wave 0 merges those lists (one candidate per lane) -- instead of one wave inserting
// every candidate (~19 per lane at C = 148: 10.9 us).  The union of the shares' best 8 holds the
// row's best 8, and the order (tk_better, unique indices) is the same at both levels.
constexpr int TKM_WAVES = 8;
template <int ODT>
__global__ __launch_bounds__(64 * TKM_WAVES) void topk_merge_waves_kernel(const float* __restrict__ logits, int64_t ld, int64_t C,
                                                                          int64_t S, int k, typename Elem<ODT>::T* __restrict__ out_v,
                                                                          int64_t* __restrict__ out_i) {
  __shared__ float s_v[TKM_WAVES * 8];
  __shared__ int32_t s_i[TKM_WAVES * 8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const float* lg = logits + row * ld;
  float rv[8];
  int32_t ri[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) rv[j] = -INFINITY, ri[j] = INT32_MAX;
  // this wave's share of the candidates; every load of a batch is issued before any is compared
  const int64_t n = C * 8, per = (n + TKM_WAVES - 1) / TKM_WAVES;
  const int64_t e_lo = wave * per, e_hi = e_lo + per < n ? e_lo + per : n;
  constexpr int NB = 4;
  for (int64_t e0 = e_lo; e0 < e_hi; e0 += 64 * NB) {
    float cv[NB];
    int32_t ci[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int64_t e0u = e0 + lane + 64 * u, e = e0u < e_hi ? e0u : e_lo;
      const int64_t c = e / 8, j = e % 8;
      cv[u] = lg[c * S + j];
      ci[u] = __float_as_int(lg[c * S + 8 + j]);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u)
      if (e0 + lane + 64 * u < e_hi) tk8_insert(rv, ri, cv[u], ci[u]);
  }
  float ov[8];
  int32_t oi[8];
  tk8_wave_tournament(rv, ri, ov, oi);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (lane == j) s_v[wave * 8 + j] = ov[j], s_i[wave * 8 + j] = oi[j];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int j = 0; j < 8; ++j) rv[j] = -INFINITY, ri[j] = INT32_MAX;
  if (lane < TKM_WAVES * 8) rv[0] = s_v[lane], ri[0] = s_i[lane];
  tk8_wave_tournament(rv, ri, ov, oi);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (lane == j && j < k) {
      out_v[row * k + j] = Elem<ODT>::cvt(ov[j]);
      out_i[row * k + j] = oi[j];
    }
}


// k > 8: the lists stay in LDS (a register list of 16 or 32 entries and its partner spill), with
// the same bound, batched loads and a register copy of the list's last entry; merged pairwise
// with a two-pointer merge into registers (loops over the compile-time TK_MAX keep them there).
template <int ODT>
__global__ __launch_bounds__(1024) void topk_rows_lds_kernel(const float* __restrict__ logits, int64_t V, int64_t ld,
                                                             int k, typename Elem<ODT>::T* __restrict__ out_v,
                                                             int64_t* __restrict__ out_i) {
  extern __shared__ float tk_lists[];  // values [nt][k], then indices [nt][k]
  const int nt = blockDim.x, tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* lg = logits + row * ld;
  float* lv = tk_lists + tid * k;
  int32_t* li = (int32_t*)(tk_lists + nt * k) + tid * k;
  auto clear = [&]() {
    for (int j = 0; j < k; ++j) lv[j] = -INFINITY, li[j] = INT32_MAX;
  };
  // thread 0's list becomes the best k of all lists
  auto merge_tree = [&]() {
    __syncthreads();
    for (int half = nt / 2; half >= 1; half >>= 1) {
      if (tid < half) {
        float mv[TK_MAX];
        int32_t mi[TK_MAX];
        const float* bv = tk_lists + (tid + half) * k;
        const int32_t* bi = (const int32_t*)(tk_lists + nt * k) + (tid + half) * k;
        int a = 0, b = 0;
#pragma unroll
        for (int j = 0; j < TK_MAX; ++j) {
          if (j < k) {
            if (tk_better(lv[a], li[a], bv[b], bi[b])) mv[j] = lv[a], mi[j] = li[a], ++a;
            else mv[j] = bv[b], mi[j] = bi[b], ++b;
          }
        }
#pragma unroll
        for (int j = 0; j < TK_MAX; ++j)
          if (j < k) lv[j] = mv[j], li[j] = mi[j];
      }
      __syncthreads();
    }
  };
  // pass 1: the bound (the k-th best of the threads' maxima), as in topk_rows_kernel
  float mxv = -INFINITY;
  int32_t mxi = INT32_MAX;
  for (int64_t n0 = tid; n0 < V; n0 += (int64_t)TK_BATCH * nt) {
    float v[TK_BATCH];
#pragma unroll
    for (int b = 0; b < TK_BATCH; ++b) {
      const int64_t n = n0 + (int64_t)b * nt;
      v[b] = lg[n < V ? n : 0];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < TK_BATCH; ++b) {
      const int64_t n = n0 + (int64_t)b * nt;
      if (n < V && tk_better(v[b], (int32_t)n, mxv, mxi)) mxv = v[b], mxi = (int32_t)n;
    }
  }
  clear();
  lv[0] = mxv, li[0] = mxi;
  merge_tree();
  const float tau_v = tk_lists[k - 1];
  const int32_t tau_i = ((const int32_t*)(tk_lists + nt * k))[k - 1];
  __syncthreads();
  // pass 2: the elements not worse than the bound, into the thread's sorted LDS list
  clear();
  float last_v = -INFINITY;
  int32_t last_i = INT32_MAX;
  for (int64_t n0 = tid; n0 < V; n0 += (int64_t)TK_BATCH * nt) {
    float v[TK_BATCH];
#pragma unroll
    for (int b = 0; b < TK_BATCH; ++b) {
      const int64_t n = n0 + (int64_t)b * nt;
      v[b] = lg[n < V ? n : 0];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < TK_BATCH; ++b) {
      const int64_t n = n0 + (int64_t)b * nt;
      if (n >= V || tk_better(tau_v, tau_i, v[b], (int32_t)n) || !tk_better(v[b], (int32_t)n, last_v, last_i)) continue;
      int j = k - 1;
      while (j > 0 && tk_better(v[b], (int32_t)n, lv[j - 1], li[j - 1])) {
        lv[j] = lv[j - 1], li[j] = li[j - 1];
        --j;
      }
      lv[j] = v[b], li[j] = (int32_t)n;
      last_v = lv[k - 1], last_i = li[k - 1];
    }
  }
  merge_tree();
  if (tid < k) {  // the merged list is thread 0's
    out_v[row * k + tid] = Elem<ODT>::cvt(tk_lists[tid]);
    out_i[row * k + tid] = ((const int32_t*)(tk_lists + nt * k))[tid];
  }
}

// LDS-staged form of the tiled GEMV (16-bit activations, K % 8 == 0, x row stride % 8 == 0, M <= TG_MR,
// everything below fitting in LDS): the workgroup stages x once, as interleaved words with their
// sums, and each wave stages its tile's scales (converted to fp32) and zero points, so that the
// word loop issues one memory load per word (the weights) instead of one per weight word, x
// word, scale and zero point (10 for T = 4).  Same arithmetic, in the same order, as the fast
// path of int4_gemv_tiled_kernel, so the two agree bit for bit.  NW: the lane's words (words
// lane, lane + 64, ..., at most NW of them, K <= 512 NW), all requested before the staging barrier.
// Dynamic LDS: x words u32x4 [M][words], x sums float [M][words], scales float [4 waves][G][T],
// zero points uint8 [4 waves][G][ZB].
template <int XDT, int SDT, int T, int NW, bool OUT_F32>
__global__ __launch_bounds__(256) void int4_gemv_tiled_lds_kernel(
    const typename Elem<XDT>::T* __restrict__ x, int64_t M, int64_t K, int64_t xs, const uint32_t* __restrict__ qw,
    int64_t tiles, int64_t pc, const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz,
    int64_t ss_g, int64_t ss_n, int64_t gsz, int64_t N, void* __restrict__ y, int64_t ys) {
  extern __shared__ __attribute__((aligned(16))) uint8_t tl_smem[];
  constexpr int ZB = T <= 4 ? 4 : 8;
  constexpr float OFF = XDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
  constexpr uint32_t ONES = XDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const int lane = threadIdx.x & 63, wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  const bool active = tile < tiles;
  const int64_t words = K / 8, G = (K + gsz - 1) / gsz;
  const int64_t MW = (M * words + 3) & ~(int64_t)3;  // keeps the scale rows 16-byte aligned
  u32x4* s_x = (u32x4*)tl_smem;
  float* s_sx = (float*)(s_x + MW);
  float* s_sc = s_sx + MW + (int64_t)wave * G * T;
  uint8_t* s_z = (uint8_t*)(s_sx + MW + 4 * G * T) + (int64_t)wave * G * ZB;
  const uint32_t* tw = qw + tile * pc * T;
  // x words first (everything waits for them), then the tile's scales and zero points, then every
  // weight word of the lane (clamped to the last word: no load is conditional, so no wait is
  // widened at a join)
  constexpr int XPT = 4;  // x words per thread (the host picks this kernel for M * words <= 1024)
  u32x4 xw[XPT];
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    const int64_t i = threadIdx.x + 256 * j;
    const int64_t m = i / words, w = i % words;
    xw[j] = i < M * words ? *(const u32x4*)((const uint16_t*)x + m * xs + w * 8) : u32x4{0u, 0u, 0u, 0u};
  }
  if (active) {
    for (int64_t e = lane; e < G * T; e += 64) {
      const int64_t g = e / T, t = e % T;
      const int64_t n = tile * T + t;
      const int64_t nc = n < N ? n : 0;
      s_sc[e] = Elem<SDT>::load(qs, g * ss_g + nc * ss_n);
      s_z[g * ZB + t] = (uint8_t)qz[g * ss_g + nc * ss_n];
    }
  }
  TileWords<T> R[NW];
  if (active) {
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const int64_t w = lane + 64 * j;
      R[j] = load_tile_words<T>(tw + (w < words ? w : words - 1) * T);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    const int64_t i = threadIdx.x + 256 * j;
    if (i < M * words) {
      const u32x4 xi = interleave_x(xw[j]);
      s_x[i] = xi;
      float sx = dot2_acc<XDT>(xi.x, ONES, 0.f);
      sx = dot2_acc<XDT>(xi.y, ONES, sx);
      sx = dot2_acc<XDT>(xi.z, ONES, sx);
      s_sx[i] = dot2_acc<XDT>(xi.w, ONES, sx);
    }
  }
  __syncthreads();
  if (!active) return;
  float acc[TG_MR][T];
#pragma unroll
  for (int m = 0; m < TG_MR; ++m)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[m][t] = 0.f;
  auto compute = [&](int64_t w, const TileWords<T>& q) {
    const int64_t g = (w * 8) / gsz;
    float sc[T];
    uint8_t zb[ZB];
    if constexpr (T == 4) {
      const float4 v = *(const float4*)(s_sc + g * T);
      sc[0] = v.x, sc[1] = v.y, sc[2] = v.z, sc[3] = v.w;
    } else {
#pragma unroll
      for (int t = 0; t < T; ++t) sc[t] = s_sc[g * T + t];
    }
    if constexpr (ZB == 4) {
      const uint32_t zz = *(const uint32_t*)(s_z + g * ZB);
#pragma unroll
      for (int t = 0; t < 4; ++t) zb[t] = (uint8_t)(zz >> (8 * t));
    } else {
      const uint2 zz = *(const uint2*)(s_z + g * ZB);
#pragma unroll
      for (int t = 0; t < 8; ++t) zb[t] = (uint8_t)(((t < 4) ? zz.x : zz.y) >> (8 * (t & 3)));
    }
#pragma unroll
    for (int m = 0; m < TG_MR; ++m) {
      if (m >= M) continue;
      const u32x4 xi = s_x[m * words + w];
      const float sx = s_sx[m * words + w];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const u32x4 f = nibbles_to_frag<XDT>(q.v[t]);
        float d = dot2_acc<XDT>(xi.x, f.x, 0.f);
        d = dot2_acc<XDT>(xi.y, f.y, d);
        d = dot2_acc<XDT>(xi.z, f.z, d);
        d = dot2_acc<XDT>(xi.w, f.w, d);
        acc[m][t] = fmaf(sc[t], d - (OFF + (float)(int8_t)zb[t]) * sx, acc[m][t]);
      }
    }
  };
#pragma unroll
  for (int j = 0; j < NW; ++j)
    if (lane + 64 * j < words) compute(lane + 64 * j, R[j]);
#pragma unroll
  for (int m = 0; m < TG_MR; ++m) {
    if (m >= M) continue;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float v = wave_sum_rows(acc[m][t]);
      const int64_t n = tile * T + t;
      if (lane == 0 && n < N) {
        if constexpr (OUT_F32) ((float*)y)[m * ys + n] = v;
        else ((typename Elem<XDT>::T*)y)[m * ys + n] = Elem<XDT>::cvt(v);
      }
    }
  }
}

// ANNA_MI_TILED_PLAIN=1 keeps the tiled GEMV off its LDS-staged form (for comparisons and tests)
static const int g_tiled_plain = [] {
  const char* v = getenv("ANNA_MI_TILED_PLAIN");
  return v ? atoi(v) : 0;
}();

template <int XDT, int SDT, bool OUT_F32>
int launch_tiled(const void* x, int64_t M, int64_t K, int64_t xs, const uint32_t* qw, int64_t tiles, int64_t pc,
                 int64_t T, const void* qs, const int8_t* qz, int64_t ssg, int64_t ssn, int64_t gsz, int64_t N, void* y,
                 int64_t ys, hipStream_t st) {
  using XT = typename Elem<XDT>::T;
  using ST = typename Elem<SDT>::T;
  const dim3 grid((unsigned)((tiles + 3) / 4));
#define ANNA_TILED_LAUNCH(TT)                                                                                  \
  hipLaunchKernelGGL((int4_gemv_tiled_kernel<XDT, SDT, TT, OUT_F32>), grid, dim3(256), 0, st, (const XT*)x, M, K, \
                     xs, qw, tiles, pc, (const ST*)qs, qz, ssg, ssn, gsz, N, y, ys)
  // the LDS-staged form when x, its sums and four tiles' scales and zero points fit in 64 KB
  const int64_t words = K / 8, G = (K + gsz - 1) / gsz;
  const int64_t lds = ((M * words + 3) & ~(int64_t)3) * 20 + 4 * G * T * 4 + 4 * G * (T <= 4 ? 4 : 8);
  if (XDT != ANNA_MI_F32 && K % 8 == 0 && xs % 8 == 0 && M >= 1 && M <= TG_MR && M * words <= 1024 &&
      words <= 512 && lds <= 65536 && (uintptr_t)x % 16 == 0 && (uintptr_t)qw % 16 == 0 && !g_tiled_plain) {
#define ANNA_TILED_LDS_LAUNCH(TT) \
  if (words <= 256) \
    hipLaunchKernelGGL((int4_gemv_tiled_lds_kernel<XDT, SDT, TT, 4, OUT_F32>), grid, dim3(256), (size_t)lds, st, \
                       (const XT*)x, M, K, xs, qw, tiles, pc, (const ST*)qs, qz, ssg, ssn, gsz, N, y, ys); \
  else \
    hipLaunchKernelGGL((int4_gemv_tiled_lds_kernel<XDT, SDT, TT, 8, OUT_F32>), grid, dim3(256), (size_t)lds, st, \
                       (const XT*)x, M, K, xs, qw, tiles, pc, (const ST*)qs, qz, ssg, ssn, gsz, N, y, ys)
    switch (T) {
      case 1: ANNA_TILED_LDS_LAUNCH(1); break;
      case 2: ANNA_TILED_LDS_LAUNCH(2); break;
      case 4: ANNA_TILED_LDS_LAUNCH(4); break;
      case 8: ANNA_TILED_LDS_LAUNCH(8); break;
      default: set_error("output tile must be 1, 2, 4 or 8 (got %lld)", (long long)T); return ANNA_MI_EINVAL;
    }
#undef ANNA_TILED_LDS_LAUNCH
    ANNA_LAUNCH_CHECK("int4_gemv_tiled_lds_kernel");
    return ANNA_MI_OK;
  }
  switch (T) {
    case 1: ANNA_TILED_LAUNCH(1); break;
    case 2: ANNA_TILED_LAUNCH(2); break;
    case 4: ANNA_TILED_LAUNCH(4); break;
    case 8: ANNA_TILED_LAUNCH(8); break;
    default: set_error("output tile must be 1, 2, 4 or 8 (got %lld)", (long long)T); return ANNA_MI_EINVAL;
  }
#undef ANNA_TILED_LAUNCH
  ANNA_LAUNCH_CHECK("int4_gemv_tiled_kernel");
  return ANNA_MI_OK;
}

int check_tiled(const void* x, int64_t M, int64_t K, int64_t xs, const uint32_t* qw, int64_t tiles, int64_t pc,
                int64_t T, const void* qs, const int8_t* qz, int64_t G, int64_t gsz, int64_t N) {
  ANNA_CHECK(x && qw && qs && qz, "int4 tiled GEMV: null pointer");
  ANNA_CHECK(M >= 0 && K > 0 && xs >= K, "int4 tiled GEMV: bad activation shape");
  ANNA_CHECK(tiles > 0 && pc * 8 >= K, "qweight packed columns are smaller than in_features");
  ANNA_CHECK(tiles * T >= N && N > 0, "qweight output tiles are smaller than out_features");
  ANNA_CHECK(gsz > 0 && gsz % 8 == 0 && G * gsz >= K, "qscale group count is smaller than in_features");
  return ANNA_MI_OK;
}

}  // namespace
}  // namespace anna

using namespace anna;

extern "C" int anna_mi_int4_gemv_tiled(const void* x, int x_dtype, int64_t M, int64_t K, int64_t x_row_stride,
                                       const int32_t* qweight, int64_t tiles, int64_t packed_cols, int64_t tile,
                                       const void* qscale, int scale_dtype, const int8_t* qzeros, int64_t group_count,
                                       int64_t scale_stride_group, int64_t scale_stride_row, int64_t group_size,
                                       int64_t N, void* y, int y_is_f32, int64_t y_row_stride, void* stream) {
  const int rc = check_tiled(x, M, K, x_row_stride, (const uint32_t*)qweight, tiles, packed_cols, tile, qscale, qzeros,
                             group_count, group_size, N);
  if (rc != ANNA_MI_OK) return rc;
  ANNA_CHECK(y != nullptr && y_row_stride >= N, "anna_mi_int4_gemv_tiled: bad output");
  if (M == 0) return ANNA_MI_OK;
  ANNA_DISPATCH_DTYPE(x_dtype, XDT, {
    ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
      return y_is_f32 ? launch_tiled<XDT, SDT, true>(x, M, K, x_row_stride, (const uint32_t*)qweight, tiles,
                                                     packed_cols, tile, qscale, qzeros, scale_stride_group,
                                                     scale_stride_row, group_size, N, y, y_row_stride, as_stream(stream))
                      : launch_tiled<XDT, SDT, false>(x, M, K, x_row_stride, (const uint32_t*)qweight, tiles,
                                                      packed_cols, tile, qscale, qzeros, scale_stride_group,
                                                      scale_stride_row, group_size, N, y, y_row_stride,
                                                      as_stream(stream));
    });
  });
  return ANNA_MI_OK;
}

namespace anna {
namespace {
// scratch_ok: values may be overwritten (the LM head's own logits), which lets few long rows
// split over several workgroups
int topk_rows(const float* values, int64_t rows, int64_t V, int64_t ld, int64_t top_k, void* out_values, int out_dtype,
              int64_t* out_indices, void* stream, bool scratch_ok) {
  ANNA_CHECK(values && out_values && out_indices, "anna_mi_topk_rows: null pointer");
  ANNA_CHECK(top_k >= 1 && top_k <= TK_MAX && top_k <= V, "top_k must be in [1, min(vocab_size, 32)]");
  ANNA_CHECK(rows >= 0 && ld >= V && V < INT32_MAX, "anna_mi_topk_rows: bad shape");
  if (rows == 0) return ANNA_MI_OK;
  ANNA_DISPATCH_DTYPE(out_dtype, ODT, {
    if (top_k <= 8) {
      // few long rows: each row is split over C workgroups whose lists a second launch merges
      // (one workgroup per row of V = 151936 took ~50 us, a chain of dependent passes; workgroup
      // chunks merged by LDS trees ~26 us): one wave per 1024 elements, then one wave per row
      if (scratch_ok && rows <= 16 && V >= 8192) {
        const int64_t S = 64 * TKW_PER;
        int64_t C = (V + S - 1) / S;
        if (V - (C - 1) * S < 16) --C;  // the last chunk takes the short tail
        hipLaunchKernelGGL(topk_chunk_wave_kernel, dim3((unsigned)C, (unsigned)rows), dim3(64), 0, as_stream(stream),
                           const_cast<float*>(values), V, ld, S);
        hipLaunchKernelGGL((topk_merge_waves_kernel<ODT>), dim3((unsigned)rows), dim3(64 * TKM_WAVES), 0, as_stream(stream),
                           values, ld, C, S, (int)top_k, (typename Elem<ODT>::T*)out_values, out_indices);
      } else {
        const int nt = tk_threads(8);
        hipLaunchKernelGGL((topk_rows_kernel<ODT, 8>), dim3(1u, (unsigned)rows), dim3((unsigned)nt), (size_t)nt * 8 * 8,
                           as_stream(stream), const_cast<float*>(values), V, ld, (int)top_k,
                           (typename Elem<ODT>::T*)out_values, out_indices, V);
      }
    } else {
      int nt = 1024;
      while (nt > 64 && (int64_t)nt * top_k * 8 > TK_LDS) nt >>= 1;
      hipLaunchKernelGGL((topk_rows_lds_kernel<ODT>), dim3((unsigned)rows), dim3((unsigned)nt), (size_t)nt * top_k * 8,
                         as_stream(stream), values, V, ld, (int)top_k, (typename Elem<ODT>::T*)out_values, out_indices);
    }
  });
  ANNA_LAUNCH_CHECK("topk_rows_kernel");
  return ANNA_MI_OK;
}
}  // namespace
}  // namespace anna

extern "C" int anna_mi_topk_rows(const float* values, int64_t rows, int64_t V, int64_t ld, int64_t top_k,
                                 void* out_values, int out_dtype, int64_t* out_indices, void* stream) {
  return topk_rows(values, rows, V, ld, top_k, out_values, out_dtype, out_indices, stream, false);
}

extern "C" int anna_mi_lm_head_int4_topk(const void* x, int x_dtype, int64_t rows, int64_t K, int64_t x_row_stride,
                                         const int32_t* qweight, int64_t tiles, int64_t packed_cols, int64_t tile,
                                         const void* qscale, int scale_dtype, const int8_t* qzeros, int64_t group_count,
                                         int64_t scale_stride_group, int64_t scale_stride_row, int64_t group_size,
                                         int64_t vocab, int64_t top_k, float* logits, void* values, int64_t* indices,
                                         void* stream) {
  ANNA_CHECK(logits && values && indices, "anna_mi_lm_head_int4_topk: null pointer");
  int rc = anna_mi_int4_gemv_tiled(x, x_dtype, rows, K, x_row_stride, qweight, tiles, packed_cols, tile, qscale,
                                   scale_dtype, qzeros, group_count, scale_stride_group, scale_stride_row, group_size,
                                   vocab, logits, 1, vocab, stream);
  if (rc != ANNA_MI_OK) return rc;
  return topk_rows(logits, rows, vocab, vocab, top_k, values, x_dtype, indices, stream, true);
}
