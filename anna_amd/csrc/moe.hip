// Mixture-of-experts routing and grouped int4 expert MLP on gfx950.
//
//   moe_router_kernel     one wave per token: fp32 softmax over the experts, top-k by repeated
//                         wave arg-max (ties go to the lower expert index, the order of the
//                         reference's insertion sort), optional renormalisation, usage counts.
//   moe_route_small_kernel  routes <= 1024: router, dispatch order and the MLP's expert list
//                         in one workgroup (same outputs and order as the kernels below).
//   moe_order_kernel      one workgroup per expert: expert offsets (prefix sum of usage) and
//                         the compact route order sorted by (expert, token, k) -- the order
//                         of the reference's CPU path -- by a ballot prefix scan over the
//                         routes in token-major order; optionally the list of experts with
//                         routes that the grouped MLP walks.  Deterministic (no atomics).
//   moe_gather_kernel     compact_hidden[p] = hidden[sorted_token_idx[p]].
//   moe_int4_mlp_kernel   grouped W4A16 expert MLP.  grid (64-row output tiles, active
//                         experts); each workgroup takes the routes of its expert 16 at a
//                         time (staged in LDS as the MFMA A operand) against 4 waves x 16 rows
//                         of int4 weights turned into bf16/f16 "off + q" fragments in registers
//                         (v_mfma_f32_16x16x32).  Pass 1 (gate, up): act = silu(x Wg^T) * (x Wu^T)
//                         in fp32; pass 2 (down): out = (act Wd^T) * routing weight.  Experts
//                         without routes exit at once, so every expert of the bank can be passed
//                         as active without a host synchronisation.
//   moe_scatter_*         out[t] = sum of the compact rows of token t (fp32 atomics, the
//                         reference op); moe_combine_kernel does the same as a deterministic
//                         gather through the route positions written by the dispatch.
#include <algorithm>

#include "common.hpp"
#include "int4_frag.hpp"

namespace anna {
namespace {

// ------------------------------------------------------------------ router

// LDS scratch route_token needs per wave, in floats
__host__ __device__ constexpr int route_scratch(int64_t E) { return (int)((E + 3) / 4 * 4) + 128; }

// Softmax over the E logits of token t and its top_k (ties to the lower expert index), by one
// wave; lane l holds experts l, l + 64, ...  Lane j < top_k returns route j's weight (normalized
// over the top_k when asked) and expert.  The top_k is found by rank, not by k rounds of a
// cross-lane argmax: the probabilities go to the wave's LDS scratch sp (route_scratch(E)
// floats), every lane counts for each of its experts how many experts beat it (a larger
// probability, or an equal one at a lower index), and an expert of rank j < top_k is route j.
// MAXV: experts per lane, E <= 64 MAXV (instantiated for E <= 64, 128, 256 and 1024).
template <int LDT, int MAXV>
__device__ __forceinline__ void route_token(const typename Elem<LDT>::T* __restrict__ logits, int64_t t, int64_t E,
                                            int64_t ls, int64_t top_k, int normalize, int lane, float* sp,
                                            float& w_out, int64_t& e_out) {
  float v[MAXV];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int64_t e = lane + 64 * i;
    v[i] = e < E ? Elem<LDT>::load(logits, t * ls + e) : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
  mx = wave_max(mx);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int64_t e = lane + 64 * i;
    v[i] = e < E ? expf(v[i] - mx) : 0.f;
    s += v[i];
  }
  const float inv = 1.0f / wave_sum(s);
  const int E4 = (int)((E + 3) / 4 * 4);
  float* stp = sp + E4;                 // route j's probability
  int* ste = (int*)(sp + E4 + 64);      // route j's expert
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int e = lane + 64 * i;
    if (e < E) sp[e] = v[i] * inv;
    else if (e < E4) sp[e] = -2.0f;     // padding: beats nothing, ties nothing
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int e = lane; e < E; e += 64) {
    const float p = sp[e];
    int rank = 0;
    for (int j = 0; j < E4; j += 4) {
      const float4 q = *(const float4*)(sp + j);
      rank += (q.x > p || (q.x == p && j < e)) + (q.y > p || (q.y == p && j + 1 < e)) +
              (q.z > p || (q.z == p && j + 2 < e)) + (q.w > p || (q.w == p && j + 3 < e));
    }
    if (rank < top_k) {
      stp[rank] = p;
      ste[rank] = e;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float top_sum = 0.f;  // in route order (descending), as the k rounds of argmax summed them
  for (int64_t j = 0; j < top_k; ++j) top_sum += stp[j];
  const float scale = normalize && top_sum > 0.f ? 1.0f / top_sum : 1.0f;
  w_out = lane < top_k ? stp[lane] * scale : 0.f;
  e_out = lane < top_k ? ste[lane] : 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();  // sp is reused by the wave's next token
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Experts per lane for E experts (the route_token instantiations).
inline int route_maxv(int64_t E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : 16; }
#define ANNA_DISPATCH_MAXV(E, NAME, ...)                                  \
  switch (route_maxv(E)) {                                                \
    case 1: { constexpr int NAME = 1; __VA_ARGS__; break; }               \
    case 2: { constexpr int NAME = 2; __VA_ARGS__; break; }               \
    case 4: { constexpr int NAME = 4; __VA_ARGS__; break; }               \
    default: { constexpr int NAME = 16; __VA_ARGS__; break; }             \
  }

// One wave per token.
template <int LDT, int MAXV>
__global__ __launch_bounds__(256) void moe_router_kernel(const typename Elem<LDT>::T* __restrict__ logits,
                                                         int64_t T, int64_t E, int64_t ls, int64_t top_k, int normalize,
                                                         float* __restrict__ weights, int64_t* __restrict__ selected,
                                                         int32_t* __restrict__ usage) {
  extern __shared__ float r_scratch[];  // 4 x route_scratch(E)
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float w;
  int64_t e;
  route_token<LDT, MAXV>(logits, t, E, ls, top_k, normalize, lane, r_scratch + (threadIdx.x >> 6) * route_scratch(E), w, e);
  if (lane < top_k) {
    weights[t * top_k + lane] = w;
    selected[t * top_k + lane] = e;
    atomicAdd(usage + e, 1);
  }
}

// Exclusive prefix sum of v over the 1024 threads of a workgroup (s: 16 ints of LDS); *total
// receives the sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* s, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(inc, off, 64);
    if (lane >= off) inc += o;
  }
  if (lane == 63) s[wave] = inc;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    before += w < wave ? s[w] : 0;
    all += s[w];
  }
  __syncthreads();  // s may be reused by the caller
  *total = all;
  return before + inc - v;
}

// Router + dispatch order + the MLP's item list in one workgroup, for small batches (routes =
// tokens x top_k <= 1024, E <= 1024): the outputs of moe_router_kernel (usage included, no
// separate clearing) and of moe_order_kernel (offsets, sorted token / route, route_pos), in the
// same deterministic (expert, token, k) order, plus items as moe_compact_items_kernel writes
// them for the experts with routes (bank slot slots[e]).  Four launches become one; each of
// them costs a few microseconds here whatever its work.
template <int LDT, int MAXV>
__global__ __launch_bounds__(1024) void moe_route_small_kernel(
    const typename Elem<LDT>::T* __restrict__ logits, int64_t T, int64_t E, int64_t ls, int64_t top_k, int normalize,
    float* __restrict__ weights, int64_t* __restrict__ selected, int32_t* __restrict__ usage,
    int64_t* __restrict__ offsets, int64_t* __restrict__ sorted_token, int64_t* __restrict__ sorted_route,
    int64_t* __restrict__ route_pos, const int64_t* __restrict__ slots, int32_t* __restrict__ items) {
  __shared__ int s_cnt[1024], s_sel[1024], s_off[1024], s_scan[16];
  extern __shared__ float r_scratch[];  // 16 x route_scratch(E)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t R = T * top_k;
  // this thread's expert's bank slot, read now so that its latency hides behind the routing
  const int64_t my_slot = threadIdx.x < E ? slots[threadIdx.x] : 0;
  s_cnt[threadIdx.x] = 0;
  __syncthreads();
  for (int64_t t = wave; t < T; t += 16) {
    float w;
    int64_t e;
    route_token<LDT, MAXV>(logits, t, E, ls, top_k, normalize, lane, r_scratch + wave * route_scratch(E), w, e);
    if (lane < top_k) {
      weights[t * top_k + lane] = w;
      selected[t * top_k + lane] = e;
      s_sel[t * top_k + lane] = (int)e;
      atomicAdd(&s_cnt[e], 1);
    }
  }
  __syncthreads();
  const int e = threadIdx.x;
  const int cnt = e < E ? s_cnt[e] : 0;
  int total;
  const int start = block_exclusive_scan(cnt, s_scan, &total);
  int nact;
  const int j = block_exclusive_scan(cnt > 0 ? 1 : 0, s_scan, &nact);
  if (e < E) {
    usage[e] = cnt;
    offsets[e] = start;
    s_off[e] = start;
    if (cnt > 0) *(int4*)(items + 4 + 4 * j) = make_int4((int)my_slot, start, start + cnt, 0);
  }
  if (e == 0) {
    offsets[E] = total;
    items[0] = nact;
  }
  __syncthreads();
  // route r: position = first slot of its expert + the routes before it with the same expert
  const int r = threadIdx.x;
  if (r < R) {
    const int er = s_sel[r];
    int rank = 0;
    for (int q = 0; q < r; ++q) rank += s_sel[q] == er;
    const int64_t pos = s_off[er] + rank;
    sorted_token[pos] = r / top_k;
    sorted_route[pos] = r;
    if (route_pos) route_pos[r] = pos;
  }
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// ------------------------------------------------------------------ dispatch

// With items (and slots) set, also the grouped MLP's list of experts with routes, as
// moe_compact_items_kernel writes it: workgroup e counts the experts before it that have routes
// (workgroup 0 counts all of them), so no separate launch builds the list.
template <typename U>
__global__ __launch_bounds__(256) void moe_order_kernel(const int64_t* __restrict__ selected, int64_t routes,
                                                        int64_t top_k, const U* __restrict__ usage, int64_t E,
                                                        int64_t* __restrict__ offsets, int64_t* __restrict__ sorted_token,
                                                        int64_t* __restrict__ sorted_route, int64_t* __restrict__ route_pos,
                                                        const int64_t* __restrict__ slots, int32_t* __restrict__ items) {
  __shared__ int64_t s_part[4];
  __shared__ int s_act[4], s_all[4];
  __shared__ int s_cnt[4];
  const int64_t e = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t part = 0;
  int act = 0, all = 0;  // experts with routes before e / in all (the latter for workgroup 0)
  const int64_t lim = items && e == 0 ? E : e;
  for (int64_t i = threadIdx.x; i < lim; i += blockDim.x) {
    const int64_t u = (int64_t)usage[i];
    if (i < e) {
      part += u;
      act += u > 0;
    }
    all += u > 0;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    part += __shfl_xor(part, off, 64);
    act += __shfl_xor(act, off, 64);
    all += __shfl_xor(all, off, 64);
  }
  if (lane == 0) {
    s_part[wave] = part;
    s_act[wave] = act;
    s_all[wave] = all;
  }
  __syncthreads();
  const int64_t base = s_part[0] + s_part[1] + s_part[2] + s_part[3];
  const int64_t cnt = (int64_t)usage[e];
  if (threadIdx.x == 0) {
    offsets[e + 1] = base + cnt;
    if (e == 0) offsets[0] = 0;
    if (items) {
      if (e == 0) items[0] = s_all[0] + s_all[1] + s_all[2] + s_all[3];
      if (cnt > 0)
        *(int4*)(items + 4 + 4 * (s_act[0] + s_act[1] + s_act[2] + s_act[3])) =
            make_int4((int)slots[e], (int)base, (int)(base + cnt), 0);
    }
  }
  if (cnt == 0) return;
  int64_t running = 0;
  for (int64_t c = 0; c < routes; c += blockDim.x) {
    const int64_t route = c + threadIdx.x;
    const bool match = route < routes && selected[route] == e;
    const uint64_t bal = __ballot(match);
    const int below = __popcll(bal & ((1ull << lane) - 1ull));
    __syncthreads();  // s_cnt of the previous chunk has been read
    if (lane == 0) s_cnt[wave] = __popcll(bal);
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += s_cnt[w];
    if (match) {
      const int64_t pos = base + running + before + below;
      sorted_token[pos] = route / top_k;
      sorted_route[pos] = route;
      if (route_pos) route_pos[route] = pos;
    }
    running += s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
  }
}

// grid (routes), 64 threads x 16 B: compact row p = hidden row of its token; the compact
// routing weight = routing_weights[route] (dtype WDT) rounded to the hidden dtype.
template <int HDT, int WDT>
__global__ __launch_bounds__(64) void moe_gather_kernel(const typename Elem<HDT>::T* __restrict__ hidden, int64_t H,
                                                        int64_t hs, const typename Elem<WDT>::T* __restrict__ rw,
                                                        const int64_t* __restrict__ sorted_route, int64_t top_k,
                                                        typename Elem<HDT>::T* __restrict__ compact,
                                                        typename Elem<HDT>::T* __restrict__ compact_w) {
  using T = typename Elem<HDT>::T;
  constexpr int VEC = 16 / sizeof(T);
  const int64_t p = blockIdx.x;
  const int64_t route = sorted_route[p];
  const int64_t t = route / top_k;
  const T* src = hidden + t * hs;
  T* dst = compact + p * H;
  if ((H % VEC) == 0 && (hs % VEC) == 0) {
    for (int64_t c = threadIdx.x; c < H / VEC; c += blockDim.x) ((u32x4*)dst)[c] = ((const u32x4*)src)[c];
  } else {
    for (int64_t c = threadIdx.x; c < H; c += blockDim.x) dst[c] = src[c];
  }
  if (threadIdx.x == 0) compact_w[p] = HDT == WDT ? (T)rw[route] : Elem<HDT>::cvt(Elem<WDT>::load(rw, route));
}

// ------------------------------------------------------------------ scatter / combine

template <int HDT>
__global__ void moe_scatter_add_kernel(const typename Elem<HDT>::T* __restrict__ compact, int64_t H,
                                       const int64_t* __restrict__ sorted_token, float* __restrict__ acc) {
  const int64_t p = blockIdx.x;
  const int64_t t = sorted_token[p];
  for (int64_t c = (int64_t)blockIdx.y * blockDim.x + threadIdx.x; c < H; c += (int64_t)gridDim.y * blockDim.x)
    atomicAdd(acc + t * H + c, Elem<HDT>::load(compact, p * H + c));
}

template <int HDT>
__global__ void moe_cast_kernel(const float* __restrict__ acc, int64_t n, typename Elem<HDT>::T* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = Elem<HDT>::cvt(acc[i]);
}

__global__ void fill_f32_kernel(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// out[t] = sum_j compact[route_pos[t * top_k + j]], j ascending, fp32.
template <int HDT>
__global__ void moe_combine_kernel(const typename Elem<HDT>::T* __restrict__ compact, int64_t H,
                                   const int64_t* __restrict__ route_pos, int64_t top_k,
                                   typename Elem<HDT>::T* __restrict__ out) {
  const int64_t t = blockIdx.x;
  for (int64_t c = (int64_t)blockIdx.y * blockDim.x + threadIdx.x; c < H; c += (int64_t)gridDim.y * blockDim.x) {
    float s = 0.f;
    for (int64_t j = 0; j < top_k; ++j) s += Elem<HDT>::load(compact, route_pos[t * top_k + j] * H + c);
    out[t * H + c] = Elem<HDT>::cvt(s);
  }
}

// ------------------------------------------------------------------ grouped int4 MLP

constexpr int MOE_ROWS = 64;  // output rows per workgroup (4 waves x 16)
constexpr int MOE_PB = 4;     // 128-k blocks per pass (x is staged 512 k at a time)
constexpr int MOE_XP = MOE_PB * 128 + 8;  // LDS row pitch of the staged x slice (16-bit elements)
constexpr int MOE_MAXC = 4;   // 16-route chunks per sweep over the weights (64 routes)
// Whole-x staging (gate/up with one 16-route chunk): the x rows of all of K (<= MOE_XF_KMAX) go
// to LDS once, by buffer loads with an LDS destination, in the same round trip as the first
// pass's weights; the passes then wait only for their (prefetched) weights.
constexpr int MOE_XF_KMAX = 2048;
typedef __attribute__((address_space(3))) void* moe_lds_ptr;

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// One pass's worth of one wave's weights: PB blocks x NM matrices, with the scale and the zero
// point of each group kept raw (as loaded) until the pass that uses them: a conversion next to
// the load would make the prefetch wait for its data.
template <int SDT, int NM, int GPB>
struct MoePass {
  u32x4 w[MOE_PB][NM];
  typename Elem<SDT>::T s[MOE_PB][GPB][NM];
  int8_t z[MOE_PB][GPB][NM];
};

// One sweep of a workgroup over its 64 output rows x all K for NC chunks of 16 routes.
// Per pass: load this pass's x slice and store it to LDS, issue the next pass's weight loads
// (after the x loads: vector loads complete in order, so waiting for x never waits for
// them), then run the MFMAs of every chunk on the weights already in registers.
template <int HDT, int SDT, bool GU, int GPB, int NC, bool XF = false>
__device__ __forceinline__ void moe_sweep(const anna_mi_moe_mlp_args& a, uint16_t* xs, int64_t c0, int64_t nrows,
                                          int64_t slot, int64_t N, int64_t K, int64_t n, bool n_ok,
                                          const uint32_t* const* wrow, const void* const* sc, const int8_t* const* zp) {
  constexpr int MDT = (GU && HDT == ANNA_MI_F16) ? ANNA_MI_F16 : ANNA_MI_BF16;
  constexpr int SRC = GU ? HDT : ANNA_MI_F32;  // dtype of the activations read
  constexpr float OFF = MDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
  constexpr uint32_t ONES = MDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr int NM = GU ? 2 : 1;
  constexpr int XPT = NC * 16 * (MOE_PB * 16) / 256;  // 16 B x chunks per thread per pass
  using ST = typename Elem<SDT>::T;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t nblk = K / 128;
  const int64_t npass = (nblk + MOE_PB - 1) / MOE_PB;
  const void* xsrc = GU ? a.compact_hidden : (const void*)a.activation;
  const u32x4 ones = {ONES, ONES, ONES, ONES};

  auto load_pass = [&](int64_t p, MoePass<SDT, NM, GPB>& P) {
#pragma unroll
    for (int j = 0; j < MOE_PB; ++j) {
      int64_t b = p * MOE_PB + j;
      b = b < nblk ? b : nblk - 1;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        P.w[j][m] = __builtin_nontemporal_load((const u32x4*)(wrow[m] + b * 16));
#pragma unroll
        for (int q = 0; q < GPB; ++q) {
          const int64_t gi = (b * GPB + q) * N;
          P.s[j][q][m] = ((const ST*)sc[m])[gi];
          P.z[j][q][m] = zp[m][gi];
        }
      }
    }
  };

  f32x4 out[NC][NM];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int m = 0; m < NM; ++m) out[c][m] = f32x4{0.f, 0.f, 0.f, 0.f};

  MoePass<SDT, NM, GPB> cur, nxt;
  load_pass(0, cur);
  // down: the routing weights of the lane's output routes, loaded now and kept raw (loaded
  // at the stores, each would be a round trip of its own behind the previous store)
  using HT = typename Elem<HDT>::T;
  HT wraw[GU ? 1 : NC][4];
  if constexpr (!GU) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = c * 16 + 4 * kq + i;
        wraw[c][i] = ((const HT*)a.compact_weights)[c0 + (m < nrows ? m : 0)];
      }
  }
  // x row pitch in LDS (16-bit elements): a 512-k slice per pass, or all of K (XF)
  const int64_t xp = XF ? K + 8 : MOE_XP;
  if constexpr (XF) {
    static_assert(NC == 1 && GU, "whole-x staging is for the gate/up pass with one chunk");
    // wave w copies rows 4w .. 4w + 3, 512 k (1 KB) per load; rows past the expert's routes
    // fall outside the descriptor and read as zero
    const int wave = threadIdx.x >> 6;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(xsrc), 0, (int)(((c0 + nrows) * K) * 2), 0x00020000);
    const int64_t nq = K / 512;
    for (int rr = 0; rr < 4; ++rr) {
      const int row = 4 * wave + rr;
      for (int64_t q = 0; q < nq; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (moe_lds_ptr)(xs + row * xp + q * 512), 16, (uint32_t)(lane * 16),
                                                 (int)(((c0 + row) * K + q * 512) * 2), 0, 0);
    }
    // both the weights of pass 0 and x are needed now: wait for everything, then publish x
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  for (int64_t p = 0; p < npass; ++p) {
    // x slice [NC*16 rows][512 k] of this pass (rows past the expert's routes read as zero)
    if constexpr (!XF) {
    // every load of the slice first, then the conversions (converting each chunk as it
    // arrives would wait for it before the next chunk's load is issued)
    typedef u32x4 Raw[SRC == ANNA_MI_F32 ? 2 : 1];
    Raw raw[XPT];
    bool okv[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int e = threadIdx.x + 256 * i;  // chunk index: row e / 64, 8-k column e % 64
      const int row = e >> 6, col = (e & 63) * 8;
      const int64_t k = p * MOE_PB * 128 + col;
      okv[i] = row < nrows && k < K;
      const int64_t idx = (c0 + (okv[i] ? row : 0)) * K + (okv[i] ? k : 0);
      if constexpr (SRC == ANNA_MI_F32) {
        raw[i][0] = *(const u32x4*)((const float*)xsrc + idx);
        raw[i][1] = *(const u32x4*)((const float*)xsrc + idx + 4);
      } else {
        raw[i][0] = *(const u32x4*)((const uint16_t*)xsrc + idx);
      }
    }
    u32x4 xv[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      if constexpr (SRC == ANNA_MI_F32) {
        const float4 lo = __builtin_bit_cast(float4, raw[i][0]), hi = __builtin_bit_cast(float4, raw[i][1]);
        xv[i].x = (uint32_t)f32_to_bf16_bits(lo.x) | ((uint32_t)f32_to_bf16_bits(lo.y) << 16);
        xv[i].y = (uint32_t)f32_to_bf16_bits(lo.z) | ((uint32_t)f32_to_bf16_bits(lo.w) << 16);
        xv[i].z = (uint32_t)f32_to_bf16_bits(hi.x) | ((uint32_t)f32_to_bf16_bits(hi.y) << 16);
        xv[i].w = (uint32_t)f32_to_bf16_bits(hi.z) | ((uint32_t)f32_to_bf16_bits(hi.w) << 16);
      } else {
        xv[i] = raw[i][0];
      }
      if (!okv[i]) xv[i] = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();  // every wave is done with the previous slice
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int e = threadIdx.x + 256 * i;
      *(u32x4*)(xs + (e >> 6) * MOE_XP + (e & 63) * 8) = xv[i];
    }
    __syncthreads();
    }
    if (p + 1 < npass) load_pass(p + 1, nxt);  // in flight during this pass's MFMAs
#pragma unroll
    for (int j = 0; j < MOE_PB; ++j) {
      if (p * MOE_PB + j >= nblk) continue;
      if constexpr (GPB == 1) {
        // One group per block: its 4 steps accumulate in the MFMA (one accumulator per route
        // chunk and matrix), and the group's scale and zero point apply once per block:
        //   sum_k x (q - z) s = s * (sum_k x (off + q) - (off + z) sum_k x).
        f32x4 acc[NC][NM], sx[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          sx[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int m = 0; m < NM; ++m) acc[c][m] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          u32x4 wf[NM];
#pragma unroll
          for (int m = 0; m < NM; ++m) wf[m] = nibbles_to_frag<MDT>(cur.w[j][m][s]);
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const u32x4 xa = interleave_x(*(const u32x4*)(xs + (c * 16 + r) * xp + (XF ? p * (MOE_PB * 128) : 0) + j * 128 + kq * 32 + s * 8));
            sx[c] = mfma16<MDT>(xa, ones, sx[c]);
#pragma unroll
            for (int m = 0; m < NM; ++m) acc[c][m] = mfma16<MDT>(xa, wf[m], acc[c][m]);
          }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              out[c][m][i] = fmaf(Elem<SDT>::to_f32(cur.s[j][0][m]), acc[c][m][i] - (OFF + (float)cur.z[j][0][m]) * sx[c][i],
                                  out[c][m][i]);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          // lanes kq hold k = 128 b + 32 kq + 8 s + e: a step spans the whole block, so each of
          // its GPB groups gets its own MFMA with the other groups' lanes zeroed, scaled per step
          u32x4 wf[NM];
#pragma unroll
          for (int m = 0; m < NM; ++m) wf[m] = nibbles_to_frag<MDT>(cur.w[j][m][s]);
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const u32x4 xa = interleave_x(*(const u32x4*)(xs + (c * 16 + r) * xp + (XF ? p * (MOE_PB * 128) : 0) + j * 128 + kq * 32 + s * 8));
#pragma unroll
            for (int q = 0; q < GPB; ++q) {
              const u32x4 xm = kq / (4 / GPB) == q ? xa : u32x4{0u, 0u, 0u, 0u};
              const f32x4 sxq = mfma16<MDT>(xm, ones, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
              for (int m = 0; m < NM; ++m) {
                const f32x4 accq = mfma16<MDT>(xm, wf[m], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int i = 0; i < 4; ++i)
                  out[c][m][i] = fmaf(Elem<SDT>::to_f32(cur.s[j][q][m]), accq[i] - (OFF + (float)cur.z[j][q][m]) * sxq[i],
                                      out[c][m][i]);
              }
            }
          }
        }
      }
    }
    cur = nxt;
  }
  // C layout: lane holds routes c0 + 16 c + 4 kq + i of output row n
  if (n_ok) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = c * 16 + 4 * kq + i;
        if (m >= nrows) continue;
        const int64_t route = c0 + m;
        if constexpr (GU) {
          a.activation[route * N + n] = silu(out[c][0][i]) * out[c][1][i];
        } else {
          ((HT*)a.compact_outputs)[route * N + n] = Elem<HDT>::cvt(out[c][0][i] * Elem<HDT>::to_f32(wraw[c][i]));
        }
      }
  }
}

// GU: pass 1 (gate and up, K = hidden, N = intermediate, act fp32 out); otherwise pass 2
// (down, K = intermediate, N = hidden, compact outputs in HDT).  GPB: int4 groups per 128-k
// block (group size 128 / GPB; larger groups count as 1).  grid (N / 64, active experts).
// One work item: output rows [64 tile, 64 tile + 64) of bank slot `slot` for the compact routes
// [start, end) of one expert.
template <int HDT, int SDT, bool GU, int GPB, int NCMAX, bool XF>
__device__ __forceinline__ void moe_mlp_item(const anna_mi_moe_mlp_args& a, uint16_t* xs, int64_t tile, int64_t slot,
                                             int64_t start, int64_t end) {
  constexpr int NM = GU ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int64_t N = GU ? a.intermediate_dim : a.hidden_dim;
  const int64_t K = GU ? a.hidden_dim : a.intermediate_dim;
  const int64_t pc = GU ? a.hidden_packed_cols : a.intermediate_packed_cols;
  const int64_t G = GU ? a.hidden_groups : a.intermediate_groups;
  const int64_t n = tile * MOE_ROWS + wave * 16 + r;
  const bool n_ok = n < N;
  const int64_t nc = n_ok ? n : 0;
  const uint32_t* wrow[NM];
  const void* sc[NM];
  const int8_t* zp[NM];
  using ST = typename Elem<SDT>::T;
  if constexpr (GU) {
    wrow[0] = (const uint32_t*)a.gate_qweight + (slot * N + nc) * pc + kq * 4;
    wrow[1] = (const uint32_t*)a.up_qweight + (slot * N + nc) * pc + kq * 4;
    sc[0] = (const ST*)a.gate_qscale + slot * G * N + nc;
    sc[1] = (const ST*)a.up_qscale + slot * G * N + nc;
    zp[0] = a.gate_qzeros + slot * G * N + nc;
    zp[1] = a.up_qzeros + slot * G * N + nc;
  } else {
    wrow[0] = (const uint32_t*)a.down_qweight + (slot * N + nc) * pc + kq * 4;
    sc[0] = (const ST*)a.down_qscale + slot * G * N + nc;
    zp[0] = a.down_qzeros + slot * G * N + nc;
  }
  const int64_t sweep = (int64_t)a.sweep_chunks * 16;  // routes per sweep (the LDS holds their x slice)
  for (int64_t c0 = start; c0 < end; c0 += sweep) {
    const int64_t nrows = end - c0 < sweep ? end - c0 : sweep;
    if constexpr (XF)
      moe_sweep<HDT, SDT, GU, GPB, 1, true>(a, xs, c0, nrows, slot, N, K, n, n_ok, wrow, sc, zp);
    else if (NCMAX == 1 || nrows <= 16)
      moe_sweep<HDT, SDT, GU, GPB, 1>(a, xs, c0, nrows, slot, N, K, n, n_ok, wrow, sc, zp);
    else if (NCMAX == 2 || nrows <= 32)
      moe_sweep<HDT, SDT, GU, GPB, (NCMAX >= 2 ? 2 : 1)>(a, xs, c0, nrows, slot, N, K, n, n_ok, wrow, sc, zp);
    else
      moe_sweep<HDT, SDT, GU, GPB, NCMAX>(a, xs, c0, nrows, slot, N, K, n, n_ok, wrow, sc, zp);
    __syncthreads();  // the next sweep overwrites xs
  }
}

// Two forms.  Without a.items: grid (tiles, active experts), one item per workgroup, empty
// experts exit.  With a.items (the experts that have routes, compacted by
// moe_compact_items_kernel): a persistent grid that walks the items (entry, tile) of the
// compacted list, so no workgroup is dispatched for an empty expert (dispatching thousands of
// workgroups that exit at once costs tens of microseconds here).
template <int HDT, int SDT, bool GU, int GPB, int NCMAX, bool XF = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GU ? 1 : 3))) void moe_int4_mlp_kernel(const anna_mi_moe_mlp_args a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [sweep_chunks * 16][MOE_XP]
  if (a.items == nullptr) {
    const int64_t ai = blockIdx.y;
    const int64_t e = a.active_experts[ai], slot = a.active_slots[ai];
    const int64_t start = a.expert_offsets[e], end = a.expert_offsets[e + 1];
    if (end <= start) return;
    moe_mlp_item<HDT, SDT, GU, GPB, NCMAX, XF>(a, xs, blockIdx.x, slot, start, end);
    return;
  }
  const int64_t N = GU ? a.intermediate_dim : a.hidden_dim;
  const int tiles = (int)((N + MOE_ROWS - 1) / MOE_ROWS);
  const int64_t nitems = (int64_t)a.items[0] * tiles;
  int64_t it = blockIdx.x;
  if (it >= nitems) return;
  int4 cur = *(const int4*)(a.items + 4 + 4 * (it / tiles));  // {slot, start, end, -}
  for (;;) {
    const int64_t nx = it + gridDim.x;
    const int4 nxt = *(const int4*)(a.items + 4 + 4 * ((nx < nitems ? nx : it) / tiles));  // in flight meanwhile
    moe_mlp_item<HDT, SDT, GU, GPB, NCMAX, XF>(a, xs, it % tiles, cur.x, cur.y, cur.z);
    if (nx >= nitems) break;
    it = nx;
    cur = nxt;
  }
}

// ------------------------------------------------------------------ grouped int4 MLP, wide form
//
// For 16-bit hidden states and group 128 (the BASELINE bank): one 8-wave workgroup per CU walks
// (expert, tile) items tile-major.  A gate/up item is 128 rows of the gate and the same rows of the
// up matrix (wave w: rows 16 w .. 16 w + 15 of both), a down item 256 rows (wave w: rows 32 w ..
// 32 w + 31, two 16-row fragments).  Every route of the expert goes through in one sweep of up to
// 48 routes (NC chunks of 16), so each weight is loaded and turned into an MFMA fragment once per
// sweep, not once per 16 routes.  K runs in passes of 256: the workgroup stages the pass's x rows
// into LDS once, already in the order of the weight fragments (interleave_x), double-buffered with
// one barrier per pass; each wave's weights (two fragments x two 128-k blocks per pass) come two
// passes ahead in registers.  gate/up writes act = silu(x Wg^T) * (x Wu^T) rounded to bf16 (the
// down product reads bf16 operands either way), down reads it.

constexpr int W_GU_ROWS = 128, W_DN_ROWS = 256;
constexpr int W_MAXR = 48;       // routes per sweep
constexpr int W_PK = 256;        // k per pass
constexpr int W_XP = W_PK + 8;   // LDS row pitch of a staged x slice (16-bit elements)
constexpr int W_STAGES = 3;      // weight stages in LDS per wave: two passes in flight during one
constexpr int W_XBYTES = 2 * W_MAXR * W_XP * 2;
constexpr int W_WBYTES = 8 * W_STAGES * 4 * 1024;  // [wave][stage][block][fragment] 1 KB
constexpr int W_LDS = W_XBYTES + W_WBYTES;

template <int SDT>
struct WideScales {
  typename Elem<SDT>::T s[2][2];  // [block][fragment]
  int8_t z[2][2];
};

template <int HDT, int SDT, bool GU, int NC>
__device__ __forceinline__ void wide_sweep(const anna_mi_moe_mlp_args& a, unsigned char* lds, int64_t slot,
                                           int64_t tile, int64_t c0, int64_t R) {
  constexpr int MDT = GU ? HDT : ANNA_MI_BF16;  // the x operand's format (the activation is bf16)
  constexpr float OFF = MDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
  constexpr uint32_t ONES = MDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
  // loads per pass group, in issue order: NC x chunks, 4 weight copies into LDS, 8 scales/zeros
  constexpr int GROUP = NC + 12;
  using ST = typename Elem<SDT>::T;
  uint16_t* xs = (uint16_t*)lds;
  const int lane = threadIdx.x & 63, wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, kq = lane >> 4;
  unsigned char* wl = lds + W_XBYTES + wave * (W_STAGES * 4096);
  const int64_t N = GU ? a.intermediate_dim : a.hidden_dim;
  const int64_t K = GU ? a.hidden_dim : a.intermediate_dim;
  const int64_t pc = GU ? a.hidden_packed_cols : a.intermediate_packed_cols;
  const uint16_t* x = GU ? (const uint16_t*)a.compact_hidden : (const uint16_t*)a.activation;
  // the wave's two 16-row fragments: gate and up rows n (gate/up), or rows n and n + 16 (down)
  int64_t nf[2];
  if constexpr (GU) {
    nf[0] = nf[1] = tile * W_GU_ROWS + wave * 16 + r;
  } else {
    nf[0] = tile * W_DN_ROWS + wave * 32 + r;
    nf[1] = nf[0] + 16;
  }
  __amdgpu_buffer_rsrc_t rw[2];
  uint32_t woff[2];
  const ST* sc[2];
  const int8_t* zp[2];
  const int64_t G = K / 128;
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int64_t n = nf[f] < N ? nf[f] : N - 1;  // rows past N load row N - 1 and are not stored
    const int32_t* qw = GU ? (f == 0 ? a.gate_qweight : a.up_qweight) : a.down_qweight;
    const void* qs = GU ? (f == 0 ? a.gate_qscale : a.up_qscale) : a.down_qscale;
    const int8_t* qz = GU ? (f == 0 ? a.gate_qzeros : a.up_qzeros) : a.down_qzeros;
    rw[f] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(qw), 0, 0x7FFFFFFF, 0x00020000);
    woff[f] = (uint32_t)(((slot * N + n) * pc + kq * 4) * 4);
    sc[f] = (const ST*)qs + slot * G * N + n;
    zp[f] = qz + slot * G * N + n;
  }
  const int64_t npass = K / W_PK;
  // pass q's weights: lane (r, kq) copies its 16 bytes of block 2q + j, fragment f into LDS
  // (stage st), where it reads them back itself; scales and zero points into registers
  auto load_pass = [&](int64_t q, int st, WideScales<SDT>& S) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int f = 0; f < 2; ++f)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw[f], (moe_lds_ptr)(wl + st * 4096 + (j * 2 + f) * 1024), 16,
                                                 woff[f] + (uint32_t)((2 * q + j) * 64), 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        S.s[j][f] = sc[f][(2 * q + j) * N];
        S.z[j][f] = zp[f][(2 * q + j) * N];
      }
  };
  // x chunk i of this thread: row (t + 512 i) / 32, 8-k column (t + 512 i) % 32
  auto load_x = [&](int64_t q, u32x4 (&xr)[NC]) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int e = (int)threadIdx.x + 512 * i, row = e >> 5, col = (e & 31) * 8;
      const bool ok = row < R;
      xr[i] = *(const u32x4*)(x + (c0 + (ok ? row : 0)) * K + q * W_PK + col);
      if (!ok) xr[i] = u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_x = [&](const u32x4 (&xr)[NC], uint16_t* buf) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int e = (int)threadIdx.x + 512 * i;
      *(u32x4*)(buf + (e >> 5) * W_XP + (e & 31) * 8) = interleave_x(xr[i]);
    }
  };
  const u32x4 ones = {ONES, ONES, ONES, ONES};
  f32x4 out[NC][2];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int f = 0; f < 2; ++f) out[c][f] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int st, const WideScales<SDT>& S, const uint16_t* xb) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 wq0 = *(const u32x4*)(wl + st * 4096 + (j * 2 + 0) * 1024 + lane * 16);
      const u32x4 wq1 = *(const u32x4*)(wl + st * 4096 + (j * 2 + 1) * 1024 + lane * 16);
      f32x4 acc[NC][2], sx[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        sx[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc[c][0] = acc[c][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4 w0 = nibbles_to_frag<MDT>(wq0[s]), w1 = nibbles_to_frag<MDT>(wq1[s]);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const u32x4 xa = *(const u32x4*)(xb + (c * 16 + r) * W_XP + j * 128 + kq * 32 + s * 8);
          sx[c] = mfma16<MDT>(xa, ones, sx[c]);
          acc[c][0] = mfma16<MDT>(xa, w0, acc[c][0]);
          acc[c][1] = mfma16<MDT>(xa, w1, acc[c][1]);
        }
        // the x fragments of later steps are not read (and held) ahead
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const float sf = Elem<SDT>::to_f32(S.s[j][f]), zf = OFF + (float)S.z[j][f];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) out[c][f][i] = fmaf(sf, fmaf(-zf, sx[c][i], acc[c][f][i]), out[c][f][i]);
      }
    }
  };
  // one pass: request the x rows and the weights two passes ahead (clamped to the last pass,
  // so that every pass issues the same GROUP loads and the counted wait below is exact), wait
  // for this pass's weights, compute, publish the next pass's x (loaded a pass ago)
  auto pass = [&](int64_t p, int st, const WideScales<SDT>& cur, WideScales<SDT>& ahead2, const u32x4 (&xnext)[NC],
                  u32x4 (&xahead2)[NC]) {
    const int64_t q = p + 2 < npass ? p + 2 : npass - 1;
    load_x(q, xahead2);
    load_pass(q, (st + 2) % W_STAGES, ahead2);
    // this pass's weight copies and scales were issued two groups ago
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * GROUP) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    compute(st, cur, xs + (p & 1) * (W_MAXR * W_XP));
    store_x(xnext, xs + ((p + 1) & 1) * (W_MAXR * W_XP));
    __syncthreads();
  };
  WideScales<SDT> A, B, C;
  u32x4 XA[NC], XB[NC], XC[NC];
  // prologue: the groups of passes 0 and 1, then x of pass 0 into LDS
  load_x(0, XA);
  load_pass(0, 0, A);
  load_x(npass > 1 ? 1 : 0, XB);
  load_pass(npass > 1 ? 1 : 0, 1, B);
  store_x(XA, xs);
  __syncthreads();
  for (int64_t p = 0; p < npass; p += 3) {
    pass(p, 0, A, C, XB, XC);
    if (p + 1 < npass) pass(p + 1, 1, B, A, XC, XA);
    if (p + 2 < npass) pass(p + 2, 2, C, B, XA, XB);
  }
  // the clamped copies of the last passes are still in flight into stages no wave reads; the
  // next sweep's first copies must not land while they do
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // C layout: lane (r, kq) element i is route c0 + 16 c + 4 kq + i of its output row
  using HT = typename Elem<HDT>::T;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = c * 16 + 4 * kq + i;
      if (m >= R) continue;
      const int64_t route = c0 + m;
      if constexpr (GU) {
        if (nf[0] < N) ((uint16_t*)a.activation)[route * N + nf[0]] = f32_to_bf16_bits(silu(out[c][0][i]) * out[c][1][i]);
      } else {
        const float wr = Elem<HDT>::to_f32(((const HT*)a.compact_weights)[route]);
#pragma unroll
        for (int f = 0; f < 2; ++f)
          if (nf[f] < N) ((HT*)a.compact_outputs)[route * N + nf[f]] = Elem<HDT>::cvt(out[c][f][i] * wr);
      }
    }
}

// Resident forms: the routes' x rows (all of K) stay in LDS for a whole item, so the waves
// stream their weights step after step (tile after tile, pass after pass) through their own
// 3-stage LDS rings with no barrier between the steps, and store a tile after its last pass.
//   down (intermediate <= 512): up to 48 routes per sweep; an item is W_DN_TPI consecutive
//     256-row tiles of one expert (wave w: rows 32 w .. 32 w + 31, two fragments); the routing
//     weights are staged next to x.
//   gate/up (hidden <= 2048, few routes per expert): up to 16 routes per sweep; an item is
//     W_GU_TPI consecutive 128-row tiles (wave w: rows 16 w .. of the gate and of the up matrix).
// x rows are K elements apart with 16-byte chunk c of row r stored at chunk c ^ (r & 7): the 16
// rows of an MFMA operand read then hit distinct banks without padding (padding would not let
// 16 x 2048 of x and the weight rings fit the 160 KB).
constexpr int W_DN_KMAX = 512, W_DN_TPI = 4;
constexpr int W_GU_KMAX = 2048, W_GU_TPI = 2, W_GU_RMAX = 16;
constexpr int W_RES_LDS = 16 * W_GU_KMAX * 2 + W_WBYTES;  // the larger of the two layouts
static_assert(W_MAXR * W_DN_KMAX * 2 + W_MAXR * 4 + W_WBYTES <= W_RES_LDS, "down layout fits");
static_assert(W_RES_LDS <= 160 * 1024, "LDS of one workgroup");

template <int HDT, int SDT, bool GU, int NC>
__device__ __forceinline__ void resident_item(const anna_mi_moe_mlp_args& a, unsigned char* lds, int64_t slot,
                                              int64_t tile0, int64_t ntile, int64_t c0, int64_t R) {
  constexpr int MDT = GU ? HDT : ANNA_MI_BF16;  // x operand format (the activation is bf16)
  constexpr float OFF = MDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
  constexpr uint32_t ONES = MDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr int GROUP = 12;          // loads per step: 4 weight copies into LDS, 8 scales/zeros
  constexpr int64_t ROWS = GU ? W_GU_ROWS : W_DN_ROWS;
  using ST = typename Elem<SDT>::T;
  using HT = typename Elem<HDT>::T;
  uint16_t* xs = (uint16_t*)lds;
  const int lane = threadIdx.x & 63, wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int64_t N = GU ? a.intermediate_dim : a.hidden_dim;
  const int64_t K = GU ? a.hidden_dim : a.intermediate_dim;
  const int64_t pc = GU ? a.hidden_packed_cols : a.intermediate_packed_cols, G = K / 128;
  unsigned char* wl = lds + (GU ? 16 * W_GU_KMAX * 2 : W_MAXR * W_DN_KMAX * 2 + W_MAXR * 4) + wave * (W_STAGES * 4096);
  float* s_wr = (float*)(xs + W_MAXR * K);  // down: routing weights after x
  const int64_t npass = K / W_PK, nstep = ntile * npass;
  const uint16_t* x = GU ? (const uint16_t*)a.compact_hidden : (const uint16_t*)a.activation;
  const __amdgpu_buffer_rsrc_t rw[2] = {
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(GU ? a.gate_qweight : a.down_qweight), 0, 0x7FFFFFFF,
                                        0x00020000),
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(GU ? a.up_qweight : a.down_qweight), 0, 0x7FFFFFFF,
                                        0x00020000)};
  const ST* scb[2] = {(const ST*)(GU ? a.gate_qscale : a.down_qscale) + slot * G * N,
                      (const ST*)(GU ? a.up_qscale : a.down_qscale) + slot * G * N};
  const int8_t* zpb[2] = {(GU ? a.gate_qzeros : a.down_qzeros) + slot * G * N,
                          (GU ? a.up_qzeros : a.down_qzeros) + slot * G * N};
  // step q = (tile t, pass p); the wave's fragment f rows: gate/up n = 128 (tile0 + t) + 16 wave + r
  // for both matrices, down n = 256 (tile0 + t) + 32 wave + r + 16 f.  Rows past N (a partial last
  // tile) load row N - 1 and are not stored.  Byte offsets and indices in 32 bits.
  const int64_t nrow0 = tile0 * ROWS + wave * (GU ? 16 : 32) + r;
  auto row_of = [&](int64_t t, int f) {
    const int64_t n = nrow0 + t * ROWS + (GU ? 0 : 16 * f);
    return (uint32_t)(n < N ? n : N - 1);
  };
  const uint32_t wbase = (uint32_t)((slot * N * pc + kq * 4) * 4), pcb = (uint32_t)(pc * 4);
  auto load_step = [&](int64_t q, int st, WideScales<SDT>& S) {
    const int64_t t = q / npass, p = q % npass;
    const uint32_t r0 = row_of(t, 0), r1 = row_of(t, 1);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int f = 0; f < 2; ++f)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw[f], (moe_lds_ptr)(wl + st * 4096 + (j * 2 + f) * 1024), 16,
                                                 wbase + (f ? r1 : r0) * pcb, (int)((2 * p + j) * 64), 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const uint32_t gi = (uint32_t)((2 * p + j) * N) + (f ? r1 : r0);
        S.s[j][f] = scb[f][gi];
        S.z[j][f] = zpb[f][gi];
      }
  };
  const u32x4 ones = {ONES, ONES, ONES, ONES};
  f32x4 out[NC][2];
  auto clear = [&]() {
#pragma unroll
    for (int c = 0; c < NC; ++c) out[c][0] = out[c][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  clear();
  auto compute = [&](int st, const WideScales<SDT>& S, int64_t p) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 wq0 = *(const u32x4*)(wl + st * 4096 + (j * 2 + 0) * 1024 + lane * 16);
      const u32x4 wq1 = *(const u32x4*)(wl + st * 4096 + (j * 2 + 1) * 1024 + lane * 16);
      f32x4 acc[NC][2], sx[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        sx[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc[c][0] = acc[c][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const u32x4 w0 = nibbles_to_frag<MDT>(wq0[s4]), w1 = nibbles_to_frag<MDT>(wq1[s4]);
        const int64_t ci = p * (W_PK / 8) + j * 16 + kq * 4 + s4;  // 16-byte chunk of the row
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const u32x4 xa = *(const u32x4*)(xs + (c * 16 + r) * K + ((ci ^ (r & 7)) * 8));
          sx[c] = mfma16<MDT>(xa, ones, sx[c]);
          acc[c][0] = mfma16<MDT>(xa, w0, acc[c][0]);
          acc[c][1] = mfma16<MDT>(xa, w1, acc[c][1]);
        }
        // the x fragments of later steps are not read (and held) ahead
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const float sf = Elem<SDT>::to_f32(S.s[j][f]), zf = OFF + (float)S.z[j][f];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) out[c][f][i] = fmaf(sf, fmaf(-zf, sx[c][i], acc[c][f][i]), out[c][f][i]);
      }
    }
  };
  // C layout: lane (r, kq) element i is route c0 + 16 c + 4 kq + i of its output row
  auto store_tile = [&](int64_t t) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = c * 16 + 4 * kq + i;
        if (m >= R) continue;
        if constexpr (GU) {
          const int64_t n = nrow0 + t * ROWS;
          if (n < N) ((uint16_t*)a.activation)[(c0 + m) * N + n] = f32_to_bf16_bits(silu(out[c][0][i]) * out[c][1][i]);
        } else {
          const float wr = s_wr[m];
#pragma unroll
          for (int f = 0; f < 2; ++f) {
            const int64_t n = nrow0 + t * ROWS + 16 * f;
            if (n < N) ((HT*)a.compact_outputs)[(c0 + m) * N + n] = Elem<HDT>::cvt(out[c][f][i] * wr);
          }
        }
      }
  };
  auto step = [&](int64_t q, int st, const WideScales<SDT>& cur, WideScales<SDT>& ahead2) {
    load_step(q + 2 < nstep ? q + 2 : nstep - 1, (st + 2) % W_STAGES, ahead2);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * GROUP) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    const int64_t p = q % npass;
    compute(st, cur, p);
    if (p == npass - 1) {
      store_tile(q / npass);
      clear();
    }
  };
  WideScales<SDT> A, B, C;
  // the first two steps' weights first, then x (whose stores wait for its loads, queued behind)
  load_step(0, 0, A);
  load_step(nstep > 1 ? 1 : 0, 1, B);
  {
    // x rows c0 .. c0 + R - 1, all of K, interleaved and chunk-swizzled: chunk e = t + 512 i is
    // row e / (K / 8), chunk e % (K / 8)
    const int cpr = (int)(K / 8);
    constexpr int KMAX = GU ? W_GU_KMAX : W_DN_KMAX;
#pragma unroll
    for (int i = 0; i < NC * 16 * (KMAX / 8) / 512; ++i) {
      const int e = (int)threadIdx.x + 512 * i, row = e / cpr, ch = e % cpr;
      if (row >= NC * 16) break;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row < R) v = *(const u32x4*)(x + (c0 + row) * K + ch * 8);
      *(u32x4*)(xs + row * K + ((ch ^ (row & 7)) * 8)) = interleave_x(v);
    }
    if constexpr (!GU) {
      if (threadIdx.x < (unsigned)R) s_wr[threadIdx.x] = Elem<HDT>::to_f32(((const HT*)a.compact_weights)[c0 + threadIdx.x]);
    }
  }
  __syncthreads();  // x staged
  for (int64_t q = 0; q < nstep; q += 3) {
    step(q, 0, A, C);
    if (q + 1 < nstep) step(q + 1, 1, B, A);
    if (q + 2 < nstep) step(q + 2, 2, C, B);
  }
  // the clamped copies of the last steps land in stages no wave reads; wait for them before the
  // LDS is reused, and for every wave before x is restaged
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

template <int HDT, int SDT, bool GU>
__global__ __launch_bounds__(512) void moe_int4_resident_kernel(const anna_mi_moe_mlp_args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char wide_lds[];  // W_RES_LDS bytes
  const int64_t N = GU ? a.intermediate_dim : a.hidden_dim;
  const int64_t rows = GU ? W_GU_ROWS : W_DN_ROWS;
  const int64_t rmax = GU ? W_GU_RMAX : W_MAXR;
  const int64_t tiles = (N + rows - 1) / rows;
  const bool listed = a.items != nullptr;
  const int64_t nact = listed ? a.items[0] : a.active_count;
  const int64_t tpi = GU ? W_GU_TPI : W_DN_TPI;
  const int64_t groups = (tiles + tpi - 1) / tpi;
  const int64_t nitems = nact * groups;
  // tile-group-major items, as in moe_int4_mlp_wide_kernel: an expert's groups share an XCD
  for (int64_t it = blockIdx.x; it < nitems; it += gridDim.x) {
    int4 e;  // {slot, start, end, -}
    if (listed) {
      e = *(const int4*)(a.items + 4 + 4 * (it % nact));
    } else {
      const int64_t ai = it % nact, ex = a.active_experts[ai];
      e = make_int4((int)a.active_slots[ai], (int)a.expert_offsets[ex], (int)a.expert_offsets[ex + 1], 0);
    }
    const int64_t t0 = (it / nact) * tpi;
    const int64_t nt = tiles - t0 < tpi ? tiles - t0 : tpi;
    for (int64_t c0 = e.y; c0 < e.z; c0 += rmax) {
      const int64_t R = e.z - c0 < rmax ? e.z - c0 : rmax;
      if constexpr (GU) {
        resident_item<HDT, SDT, true, 1>(a, wide_lds, e.x, t0, nt, c0, R);
      } else {
        if (R <= 16)
          resident_item<HDT, SDT, false, 1>(a, wide_lds, e.x, t0, nt, c0, R);
        else if (R <= 32)
          resident_item<HDT, SDT, false, 2>(a, wide_lds, e.x, t0, nt, c0, R);
        else
          resident_item<HDT, SDT, false, 3>(a, wide_lds, e.x, t0, nt, c0, R);
      }
    }
  }
}

template <int HDT, int SDT, bool GU>
__global__ __launch_bounds__(512) void moe_int4_mlp_wide_kernel(const anna_mi_moe_mlp_args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char wide_lds[];  // W_LDS bytes
  const int64_t N = GU ? a.intermediate_dim : a.hidden_dim;
  const int64_t tiles = (N + (GU ? W_GU_ROWS : W_DN_ROWS) - 1) / (GU ? W_GU_ROWS : W_DN_ROWS);
  // tile-major items (item it: tile it / nact of list entry it % nact), so that the tiles of
  // one expert, taken by workgroups it, it + nact, ..., land on one XCD (workgroup w runs on
  // XCD w % 8; the grid is a multiple of 8) and share its L2 copy of the expert's x rows
  // the list of experts with routes (a.items), or every active expert (empty ones skipped here)
  const bool listed = a.items != nullptr;
  const int64_t nact = listed ? a.items[0] : a.active_count;
  const int64_t nitems = nact * tiles;
  for (int64_t it = blockIdx.x; it < nitems; it += gridDim.x) {
    int4 e;  // {slot, start, end, -}
    if (listed) {
      e = *(const int4*)(a.items + 4 + 4 * (it % nact));
    } else {
      const int64_t ai = it % nact, ex = a.active_experts[ai];
      e = make_int4((int)a.active_slots[ai], (int)a.expert_offsets[ex], (int)a.expert_offsets[ex + 1], 0);
    }
    const int64_t tile = it / nact;
    for (int64_t c0 = e.y; c0 < e.z; c0 += W_MAXR) {
      const int64_t R = e.z - c0 < W_MAXR ? e.z - c0 : W_MAXR;
      if (R <= 16)
        wide_sweep<HDT, SDT, GU, 1>(a, wide_lds, e.x, tile, c0, R);
      else if (R <= 32)
        wide_sweep<HDT, SDT, GU, 2>(a, wide_lds, e.x, tile, c0, R);
      else
        wide_sweep<HDT, SDT, GU, 3>(a, wide_lds, e.x, tile, c0, R);
    }
  }
}

// items[0] = number of active experts with routes; items[4 + 4 j ..] = {bank slot, first
// compact route, end route, 0} of the j-th of them, in active-list order.  One workgroup.
__global__ __launch_bounds__(1024) void moe_compact_items_kernel(const int64_t* __restrict__ active_experts,
                                                                 const int64_t* __restrict__ active_slots,
                                                                 int64_t active_count,
                                                                 const int64_t* __restrict__ offsets,
                                                                 int32_t* __restrict__ items) {
  __shared__ int s_wave[16];
  __shared__ int s_base;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) s_base = 0;
  __syncthreads();
  for (int64_t i0 = 0; i0 < active_count; i0 += 1024) {
    const int64_t ai = i0 + threadIdx.x;
    int64_t e = 0, slot = 0, st = 0, en = 0;
    if (ai < active_count) {
      e = active_experts[ai];
      slot = active_slots[ai];
      st = offsets[e];
      en = offsets[e + 1];
    }
    const bool has = ai < active_count && en > st;
    const uint64_t bal = __ballot(has);
    if (lane == 0) s_wave[wave] = __popcll(bal);
    __syncthreads();
    int before = s_base;
    for (int w = 0; w < wave; ++w) before += s_wave[w];
    if (has) {
      int4* dst = (int4*)(items + 4 + 4 * (before + __popcll(bal & ((1ull << lane) - 1ull))));
      *dst = make_int4((int)slot, (int)st, (int)en, 0);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int tot = 0;
      for (int w = 0; w < 16; ++w) tot += s_wave[w];
      s_base += tot;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) items[0] = s_base;
}

}  // namespace

namespace {
template <int HDT, int SDT, int GPB, int NCMAX>
int launch_moe_mlp_nc(const anna_mi_moe_mlp_args& a, hipStream_t st, dim3 g1, dim3 g2) {
  if (a.items) {
    // persistent: at most the workgroups that fit at once (2 per CU for gate/up, 3 for down at
    // these register counts), and no more than there can be items
    const unsigned t1 = g1.x * g1.y, t2 = g2.x * g2.y;
    g1 = dim3(t1 < 512u ? t1 : 512u);
    g2 = dim3(t2 < 768u ? t2 : 768u);
  }
  const size_t lds = (size_t)NCMAX * 16 * MOE_XP * 2;
  const int64_t K = a.hidden_dim;
  if (NCMAX == 1 && HDT != ANNA_MI_F32 && K <= MOE_XF_KMAX && K % 512 == 0) {
    auto kern = moe_int4_mlp_kernel<HDT, SDT, true, GPB, 1, true>;
    const size_t lds_xf = (size_t)16 * (K + 8) * 2;
    static bool attr_set = false;
    if (!attr_set) {
      ANNA_CHECK(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)(16 * (MOE_XF_KMAX + 8) * 2)) == hipSuccess,
                 "moe MLP: cannot raise the LDS limit");
      attr_set = true;
    }
    hipLaunchKernelGGL(kern, g1, dim3(256), lds_xf, st, a);
  } else {
    hipLaunchKernelGGL((moe_int4_mlp_kernel<HDT, SDT, true, GPB, NCMAX>), g1, dim3(256), lds, st, a);
  }
  ANNA_LAUNCH_CHECK("moe_int4_mlp_kernel (gate, up)");
  hipLaunchKernelGGL((moe_int4_mlp_kernel<HDT, SDT, false, GPB, NCMAX>), g2, dim3(256), lds, st, a);
  ANNA_LAUNCH_CHECK("moe_int4_mlp_kernel (down)");
  return ANNA_MI_OK;
}

// One chunk of 16 routes per sweep, whatever sweep_chunks asks: experts with more routes take
// more sweeps over their (then cache-resident) weights.  Measured at the BASELINE MoE shapes,
// the 2- and 4-chunk forms (which keep more routes' x in flight per weight load) lose more to
// their register count (one wave per SIMD) than they save: 316 -> 217 us at 512 tokens.
template <int HDT, int SDT, int GPB>
int launch_moe_mlp(const anna_mi_moe_mlp_args& a, hipStream_t st, dim3 g1, dim3 g2) {
  if constexpr (GPB == 1 && HDT != ANNA_MI_F32) {
    // Weights through LDS rings two steps ahead, x staged once per workgroup (16-bit hidden
    // states, group 128, dims multiples of 256, intermediate <= 512), chosen by the routes per
    // active expert on average (measured at config 5): from 16 (T = 512) the wide gate/up form,
    // which sweeps up to 48 routes per weight pass at the price of a barrier per 256-k pass; from
    // 2 (T = 64) the resident gate/up form, 16 routes with all of K in LDS and no barriers; down
    // resident in both.  Below 2 (T = 8: ~50 of 128 experts with a route or two) the 16-route
    // kernels, whose 64-row tiles keep more CUs busy, stay faster.
    if (a.group_size == 128 && a.hidden_dim % W_PK == 0 && a.intermediate_dim % W_PK == 0 &&
        a.intermediate_dim <= W_DN_KMAX && a.routes >= 2 * a.active_count) {
      const bool many = a.routes >= 16 * a.active_count;
      if (many || a.hidden_dim <= W_GU_KMAX) {
        auto kgw = moe_int4_mlp_wide_kernel<HDT, SDT, true>;
        auto kgr = moe_int4_resident_kernel<HDT, SDT, true>;
        auto kd = moe_int4_resident_kernel<HDT, SDT, false>;
        static bool lds_set = false;
        if (!lds_set) {
          ANNA_CHECK(hipFuncSetAttribute((const void*)kgw, hipFuncAttributeMaxDynamicSharedMemorySize, W_LDS) ==
                             hipSuccess &&
                         hipFuncSetAttribute((const void*)kgr, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             W_RES_LDS) == hipSuccess &&
                         hipFuncSetAttribute((const void*)kd, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             W_RES_LDS) == hipSuccess,
                     "moe MLP: cannot raise the LDS limit");
          lds_set = true;
        }
        auto grid = [](int64_t n) { return dim3((unsigned)(n < 256 ? (n + 7) / 8 * 8 : 256)); };
        const int64_t gtiles = (a.intermediate_dim + W_GU_ROWS - 1) / W_GU_ROWS;
        const int64_t dtiles = (a.hidden_dim + W_DN_ROWS - 1) / W_DN_ROWS;
        if (many) {
          hipLaunchKernelGGL(kgw, grid(a.active_count * gtiles), dim3(512), W_LDS, st, a);
          ANNA_LAUNCH_CHECK("moe_int4_mlp_wide_kernel (gate, up)");
        } else {
          hipLaunchKernelGGL(kgr, grid(a.active_count * ((gtiles + W_GU_TPI - 1) / W_GU_TPI)), dim3(512), W_RES_LDS,
                             st, a);
          ANNA_LAUNCH_CHECK("moe_int4_resident_kernel (gate, up)");
        }
        hipLaunchKernelGGL(kd, grid(a.active_count * ((dtiles + W_DN_TPI - 1) / W_DN_TPI)), dim3(512), W_RES_LDS, st,
                           a);
        ANNA_LAUNCH_CHECK("moe_int4_resident_kernel (down)");
        return ANNA_MI_OK;
      }
    }
  }
  anna_mi_moe_mlp_args b = a;
  b.sweep_chunks = 1;
  return launch_moe_mlp_nc<HDT, SDT, GPB, 1>(b, st, g1, g2);
}}  // namespace
}  // namespace anna

using namespace anna;

extern "C" int anna_mi_moe_router(const void* logits, int logits_dtype, int64_t tokens, int64_t num_experts,
                                  int64_t logits_row_stride, int64_t top_k, int normalize, float* weights,
                                  int64_t* selected, int32_t* usage, void* stream) {
  ANNA_CHECK(weights && selected && usage && (logits || tokens == 0), "anna_mi_moe_router: null pointer");
  ANNA_CHECK(num_experts > 0 && num_experts <= 1024, "anna_mi_moe_router: num_experts must be in [1, 1024]");
  ANNA_CHECK(top_k > 0 && top_k <= num_experts && top_k <= 64, "anna_mi_moe_router: need 0 < top_k <= min(num_experts, 64)");
  ANNA_CHECK(tokens >= 0 && logits_row_stride >= num_experts, "anna_mi_moe_router: bad shape");
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((num_experts + 255) / 256)), dim3(256), 0, st, usage, num_experts);
  ANNA_LAUNCH_CHECK("fill_i32_kernel");
  if (tokens == 0) return ANNA_MI_OK;
  ANNA_DISPATCH_DTYPE(logits_dtype, LDT, {
    ANNA_DISPATCH_MAXV(num_experts, MAXV, {
      hipLaunchKernelGGL((moe_router_kernel<LDT, MAXV>), dim3((unsigned)((tokens + 3) / 4)), dim3(256),
                         4 * route_scratch(num_experts) * sizeof(float), st,
                         (const typename Elem<LDT>::T*)logits, tokens, num_experts, logits_row_stride, top_k, normalize,
                         weights, selected, usage);
    });
  });
  ANNA_LAUNCH_CHECK("moe_router_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_moe_dispatch(const void* hidden, int dtype, int64_t tokens, int64_t hidden_dim,
                                    int64_t hidden_row_stride, const void* routing_weights, int weights_dtype,
                                    const int64_t* selected,
                                    const void* usage, int usage_is_int64, int64_t num_experts, int64_t top_k,
                                    int64_t* sorted_token_idx, int64_t* sorted_route_idx, int64_t* expert_offsets,
                                    void* compact_hidden, void* compact_weights, int64_t* route_pos,
                                    const int64_t* slots, int32_t* items, void* stream) {
  ANNA_CHECK(selected && usage && sorted_token_idx && sorted_route_idx && expert_offsets && compact_hidden &&
                 compact_weights && (hidden || tokens == 0) && (routing_weights || tokens == 0),
             "anna_mi_moe_dispatch: null pointer");
  ANNA_CHECK(num_experts > 0 && top_k > 0 && hidden_dim > 0 && tokens >= 0 && hidden_row_stride >= hidden_dim,
             "anna_mi_moe_dispatch: bad shape");
  ANNA_CHECK(valid_dtype(dtype) && valid_dtype(weights_dtype), "anna_mi_moe_dispatch: bad dtype code");
  ANNA_CHECK((items == nullptr) == (slots == nullptr), "anna_mi_moe_dispatch: items and slots go together");
  ANNA_CHECK(num_experts < (1ll << 30) && tokens * top_k < (1ll << 31), "anna_mi_moe_dispatch: too many routes");
  hipStream_t st = as_stream(stream);
  const int64_t routes = tokens * top_k;
  if (usage_is_int64) {
    hipLaunchKernelGGL((moe_order_kernel<int64_t>), dim3((unsigned)num_experts), dim3(256), 0, st, selected, routes,
                       top_k, (const int64_t*)usage, num_experts, expert_offsets, sorted_token_idx, sorted_route_idx,
                       route_pos, slots, items);
  } else {
    hipLaunchKernelGGL((moe_order_kernel<int32_t>), dim3((unsigned)num_experts), dim3(256), 0, st, selected, routes,
                       top_k, (const int32_t*)usage, num_experts, expert_offsets, sorted_token_idx, sorted_route_idx,
                       route_pos, slots, items);
  }
  ANNA_LAUNCH_CHECK("moe_order_kernel");
  if (routes == 0) return ANNA_MI_OK;
  ANNA_DISPATCH_DTYPE(dtype, HDT, {
    ANNA_DISPATCH_DTYPE(weights_dtype, WDT, {
      using T = typename Elem<HDT>::T;
      hipLaunchKernelGGL((moe_gather_kernel<HDT, WDT>), dim3((unsigned)routes), dim3(64), 0, st, (const T*)hidden,
                         hidden_dim, hidden_row_stride, (const typename Elem<WDT>::T*)routing_weights, sorted_route_idx,
                         top_k, (T*)compact_hidden, (T*)compact_weights);
    });
  });
  ANNA_LAUNCH_CHECK("moe_gather_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_moe_route_small(const void* logits, int logits_dtype, int64_t tokens, int64_t num_experts,
                                       int64_t logits_row_stride, int64_t top_k, int normalize, float* weights,
                                       int64_t* selected, int32_t* usage, int64_t* expert_offsets,
                                       int64_t* sorted_token_idx, int64_t* sorted_route_idx, int64_t* route_pos,
                                       const int64_t* slots, int32_t* items, void* stream) {
  ANNA_CHECK(logits && weights && selected && usage && expert_offsets && sorted_token_idx && sorted_route_idx && slots &&
                 items,
             "anna_mi_moe_route_small: null pointer");
  ANNA_CHECK(num_experts > 0 && num_experts <= 1024, "anna_mi_moe_route_small: num_experts must be in [1, 1024]");
  ANNA_CHECK(top_k > 0 && top_k <= num_experts && top_k <= 64, "anna_mi_moe_route_small: need 0 < top_k <= min(num_experts, 64)");
  ANNA_CHECK(tokens > 0 && tokens * top_k <= 1024 && logits_row_stride >= num_experts,
             "anna_mi_moe_route_small: need 0 < tokens * top_k <= 1024 (use the router + dispatch entry points above)");
  ANNA_CHECK(num_experts <= 512, "anna_mi_moe_route_small: num_experts must be <= 512 (LDS)");
  ANNA_DISPATCH_DTYPE(logits_dtype, LDT, {
    ANNA_DISPATCH_MAXV(num_experts, MAXV, {
      hipLaunchKernelGGL((moe_route_small_kernel<LDT, MAXV>), dim3(1), dim3(1024),
                         16 * route_scratch(num_experts) * sizeof(float), as_stream(stream),
                         (const typename Elem<LDT>::T*)logits, tokens, num_experts, logits_row_stride, top_k, normalize,
                         weights, selected, usage, expert_offsets, sorted_token_idx, sorted_route_idx, route_pos, slots,
                         items);
    });
  });
  ANNA_LAUNCH_CHECK("moe_route_small_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_moe_gather(const void* hidden, int dtype, int64_t hidden_dim, int64_t hidden_row_stride,
                                  const void* routing_weights, int weights_dtype, const int64_t* sorted_route_idx,
                                  int64_t routes,
                                  int64_t top_k, void* compact_hidden, void* compact_weights, void* stream) {
  ANNA_CHECK(hidden && routing_weights && sorted_route_idx && compact_hidden && compact_weights,
             "anna_mi_moe_gather: null pointer");
  ANNA_CHECK(routes >= 0 && top_k > 0 && hidden_dim > 0 && hidden_row_stride >= hidden_dim, "anna_mi_moe_gather: bad shape");
  ANNA_CHECK(valid_dtype(dtype) && valid_dtype(weights_dtype), "anna_mi_moe_gather: bad dtype code");
  if (routes == 0) return ANNA_MI_OK;
  ANNA_DISPATCH_DTYPE(dtype, HDT, {
    ANNA_DISPATCH_DTYPE(weights_dtype, WDT, {
      using T = typename Elem<HDT>::T;
      hipLaunchKernelGGL((moe_gather_kernel<HDT, WDT>), dim3((unsigned)routes), dim3(64), 0, as_stream(stream),
                         (const T*)hidden, hidden_dim, hidden_row_stride, (const typename Elem<WDT>::T*)routing_weights,
                         sorted_route_idx, top_k, (T*)compact_hidden, (T*)compact_weights);
    });
  });
  ANNA_LAUNCH_CHECK("moe_gather_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_moe_scatter(const void* compact_outputs, int dtype, int64_t routes, int64_t hidden_dim,
                                   const int64_t* sorted_token_idx, int64_t num_tokens, float* accum, void* out,
                                   void* stream) {
  ANNA_CHECK(accum && out && (routes == 0 || (compact_outputs && sorted_token_idx)), "anna_mi_moe_scatter: null pointer");
  ANNA_CHECK(hidden_dim > 0 && num_tokens >= 0 && routes >= 0, "anna_mi_moe_scatter: bad shape");
  hipStream_t st = as_stream(stream);
  const int64_t n = num_tokens * hidden_dim;
  if (n == 0) return ANNA_MI_OK;
  const unsigned nb = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(fill_f32_kernel, dim3(nb), dim3(256), 0, st, accum, n);
  ANNA_LAUNCH_CHECK("fill_f32_kernel");
  ANNA_DISPATCH_DTYPE(dtype, HDT, {
    using T = typename Elem<HDT>::T;
    if (routes > 0) {
      hipLaunchKernelGGL((moe_scatter_add_kernel<HDT>), dim3((unsigned)routes, (unsigned)((hidden_dim + 255) / 256)),
                         dim3(256), 0, st, (const T*)compact_outputs, hidden_dim, sorted_token_idx, accum);
    }
    hipLaunchKernelGGL((moe_cast_kernel<HDT>), dim3(nb), dim3(256), 0, st, accum, n, (T*)out);
  });
  ANNA_LAUNCH_CHECK("moe_scatter");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_moe_combine(const void* compact_outputs, int dtype, int64_t hidden_dim, const int64_t* route_pos,
                                   int64_t num_tokens, int64_t top_k, void* out, void* stream) {
  ANNA_CHECK(out && (num_tokens == 0 || (compact_outputs && route_pos)), "anna_mi_moe_combine: null pointer");
  ANNA_CHECK(hidden_dim > 0 && num_tokens >= 0 && top_k > 0, "anna_mi_moe_combine: bad shape");
  if (num_tokens == 0) return ANNA_MI_OK;
  ANNA_DISPATCH_DTYPE(dtype, HDT, {
    using T = typename Elem<HDT>::T;
    hipLaunchKernelGGL((moe_combine_kernel<HDT>), dim3((unsigned)num_tokens, (unsigned)((hidden_dim + 255) / 256)),
                       dim3(256), 0, as_stream(stream), (const T*)compact_outputs, hidden_dim, route_pos, top_k, (T*)out);
  });
  ANNA_LAUNCH_CHECK("moe_combine_kernel");
  return ANNA_MI_OK;
}

extern "C" int64_t anna_mi_sizeof_moe_mlp_args(void) { return (int64_t)sizeof(anna_mi_moe_mlp_args); }

extern "C" int anna_mi_moe_grouped_int4_mlp(const anna_mi_moe_mlp_args* ap, void* stream) {
  ANNA_CHECK(ap != nullptr, "anna_mi_moe_grouped_int4_mlp: null args");
  const anna_mi_moe_mlp_args& a = *ap;
  ANNA_CHECK(valid_dtype(a.dtype) && valid_dtype(a.scale_dtype), "anna_mi_moe_grouped_int4_mlp: bad dtype code");
  ANNA_CHECK(a.routes >= 0 && a.hidden_dim > 0 && a.intermediate_dim > 0 && a.active_count > 0,
             "anna_mi_moe_grouped_int4_mlp: bad shape");
  ANNA_CHECK(a.group_size > 0 && a.group_size % 32 == 0, "group_size must be a positive multiple of 32");
  ANNA_CHECK(a.hidden_dim % 128 == 0 && a.intermediate_dim % 128 == 0,
             "anna_mi_moe_grouped_int4_mlp: hidden_dim and intermediate_dim must be multiples of 128");
  ANNA_CHECK(a.hidden_packed_cols * 8 >= a.hidden_dim && a.intermediate_packed_cols * 8 >= a.intermediate_dim,
             "anna_mi_moe_grouped_int4_mlp: packed width smaller than the input dimension");
  ANNA_CHECK(a.hidden_groups * a.group_size >= a.hidden_dim && a.intermediate_groups * a.group_size >= a.intermediate_dim,
             "anna_mi_moe_grouped_int4_mlp: group count too small");
  ANNA_CHECK(a.compact_hidden && a.compact_weights && a.compact_outputs && a.expert_offsets && a.active_experts &&
                 a.active_slots && a.activation && a.gate_qweight && a.gate_qscale && a.gate_qzeros && a.up_qweight &&
                 a.up_qscale && a.up_qzeros && a.down_qweight && a.down_qscale && a.down_qzeros,
             "anna_mi_moe_grouped_int4_mlp: null pointer");
  ANNA_CHECK(a.sweep_chunks >= 1 && a.sweep_chunks <= MOE_MAXC, "anna_mi_moe_grouped_int4_mlp: sweep_chunks must be 1..4");
  if (a.routes == 0) return ANNA_MI_OK;
  hipStream_t st = as_stream(stream);
  ANNA_CHECK(a.active_count < (1ll << 30) && a.routes < (1ll << 31), "anna_mi_moe_grouped_int4_mlp: too many routes");
  if (a.items && !a.items_prefilled) {
    hipLaunchKernelGGL(moe_compact_items_kernel, dim3(1), dim3(1024), 0, st, a.active_experts, a.active_slots,
                       a.active_count, a.expert_offsets, a.items);
    ANNA_LAUNCH_CHECK("moe_compact_items_kernel");
  }
  const dim3 g1((unsigned)((a.intermediate_dim + MOE_ROWS - 1) / MOE_ROWS), (unsigned)a.active_count);
  const dim3 g2((unsigned)((a.hidden_dim + MOE_ROWS - 1) / MOE_ROWS), (unsigned)a.active_count);
  const int gpb = a.group_size >= 128 ? 1 : (int)(128 / a.group_size);
  ANNA_CHECK(a.group_size % 128 == 0 || gpb * a.group_size == 128,
             "anna_mi_moe_grouped_int4_mlp: group_size must be 32, 64 or a multiple of 128");
  ANNA_DISPATCH_DTYPE(a.dtype, HDT, {
    ANNA_DISPATCH_DTYPE(a.scale_dtype, SDT, {
      if (gpb == 1) {
        const int rc = launch_moe_mlp<HDT, SDT, 1>(a, st, g1, g2);
        if (rc != ANNA_MI_OK) return rc;
      } else if (gpb == 2) {
        const int rc = launch_moe_mlp<HDT, SDT, 2>(a, st, g1, g2);
        if (rc != ANNA_MI_OK) return rc;
      } else {
        const int rc = launch_moe_mlp<HDT, SDT, 4>(a, st, g1, g2);
        if (rc != ANNA_MI_OK) return rc;
      }
    });
  });
  return ANNA_MI_OK;
}
