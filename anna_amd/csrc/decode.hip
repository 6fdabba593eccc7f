// Split-KV (flash-decoding) GQA decode attention for one query token per sequence.
//
// Kernel 1 (decode_split_kernel): one workgroup per (block of tokens, KV head, batch).
//   All G = Hq/Hkv query heads of the KV head are processed together, so each K/V
//   element is read (and dequantized) once for the whole group instead of once per
//   q-head.  4 waves share the block's tokens, 4 tokens per wave per step; a lane owns D/64
//   consecutive dims.  The step's token x head dot products are reduced over the wave
//   together (transposed butterfly), the online-softmax state of head h lives in lanes
//   h, h + GM, ..., and the waves are merged through LDS.
//   Output: per (b, q-head, block) the running max, the denominator and the
//   unnormalized accumulator, in the reference's partial_stats / partial_values layout.
// Kernel 1' (decode_split_mfma_kernel): the MFMA form of kernel 1 for 16-bit activations, dense or
//   TQ-MSE keys and dense or min/max values at head_dim 64/128/256: one wave per range of 32-token
//   tiles (described at the kernel).  With TQ-MSE keys the query is rotated first: by the split
//   kernel itself for the randomized Hadamard rotation (16-byte aligned signs), else by a
//   rotation launch (decode_rotate_query_hadamard_kernel / decode_rotate_query_kernel).
// Kernel 2: log-sum-exp merge of the blocks per (b, q-head), optional sigmoid gate.
//   decode_merge_dims_kernel (64 dims per workgroup, the blocks split over 4 waves) when no
//   block holds rotated values and there are at most 256 blocks; decode_merge_kernel (1024
//   threads, dims x block slices, then the un-rotation of TQ-MSE value accumulators) otherwise.
//
// Reference: launch_gqa_decode_splitkv_fused_xpu (gated_delta_fused_op.sycl:4494-4706)
// and launch_gqa_decode_splitkv_turboquant_fused_xpu (sycl:4771-5094).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "int4_frag.hpp"
#include "tq_hadamard.hpp"

namespace anna {
namespace {

constexpr int DEC_WAVES = 4;
constexpr int DEC_TOKENS = 4;  // tokens per wave whose loads are in flight together
constexpr int MERGE_CHUNK = 1024;
constexpr int MERGE_THREADS = 1024;
constexpr int MERGE_PRE = 8;  // partial values per merge thread loaded before the reductions  // merge workgroup: MERGE_THREADS / head_dim block slices per dim  // block weights staged in LDS per pass of the merge

__device__ __forceinline__ float ldv(const void* p, int64_t i, int dt) {
  if (dt == ANNA_MI_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  if (dt == ANNA_MI_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

// Compile-time-dtype load: the hot loop's loads carry no branch, so they can all be in flight.
template <int DT>
__device__ __forceinline__ float ldt(const void* p, int64_t i) {
  if constexpr (DT == ANNA_MI_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  else if constexpr (DT == ANNA_MI_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  else return ((const float*)p)[i];
}

// v_mov_b32 with a DPP lane pattern (all rows and banks enabled).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ void stv(const void* p, int64_t i, int dt, float v) {
  if (dt == ANNA_MI_BF16) ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
  else if (dt == ANNA_MI_F16) ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  else ((float*)p)[i] = v;
}

__device__ __forceinline__ int sbits(int bits) { return bits == 2 ? 2 : 4; }

struct Split {
  int64_t eb, nb1, eb2;  // block size (segment 1 or whole range), blocks of segment 1, residual block size
  int aligned;           // 1: blocks never straddle the two segments
  int vec;               // 1: dense key rows contiguous and aligned for one vector load per lane, and
                         //    a lane's dims share one value scale group
};

// q' = R q for every (b, q-head); grid (Hq, B), D threads.
// q' = R q for every (b, q head), dense R: a workgroup of D threads per query, the query staged
// in LDS, output element i = sum_k R^T[k][i] q[k] with the R^T loads (coalesced over i, not
// dependent on the sum) issued eight at a time.
__global__ __launch_bounds__(1024) void decode_rotate_query_kernel(const anna_mi_decode_args a) {
  __shared__ float s_q[1024];
  const int64_t h = blockIdx.x, b = blockIdx.y, D = a.head_dim;
  const int i = threadIdx.x;
  const int64_t qb = b * a.query.s0 + h * a.query.s1;
  s_q[i] = ldv(a.query.ptr, qb + i * a.query.s3, a.dtype);
  __syncthreads();
  float acc = 0.f;
  int64_t k = 0;
  for (; k + 8 <= D; k += 8) {
    float r[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) r[u] = a.rotation_t[(k + u) * D + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = fmaf(r[u], s_q[k + u], acc);
  }
  for (; k < D; ++k) acc = fmaf(a.rotation_t[k * D + i], s_q[k], acc);
  a.query_rot[(b * a.q_heads + h) * D + i] = acc;
}

// q' = R q with the randomized Hadamard R = H diag(s) / sqrt(D) (a.rotation_signs set, D a power
// of two in [64, 1024]): one wave per (b, q head), lane l holding elements l E .. l E + E - 1 --
// signs, the in-register fast Walsh-Hadamard transform, 1/sqrt(D).
template <int E>
__global__ __launch_bounds__(256) void decode_rotate_query_hadamard_kernel(const anna_mi_decode_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.batch * a.q_heads) return;  // whole wave
  const int64_t b = row / a.q_heads, h = row % a.q_heads;
  const int64_t qb = b * a.query.s0 + h * a.query.s1;
  float v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int64_t d = (int64_t)lane * E + e;
    v[e] = ldv(a.query.ptr, qb + d * a.query.s3, a.dtype) * a.rotation_signs[d];
  }
  fwht_wave<E>(v);
  const float inv = tq_inv_sqrt(64 * E);
#pragma unroll
  for (int e = 0; e < E; ++e) a.query_rot[row * 64 * E + (int64_t)lane * E + e] = v[e] * inv;
}

template <int KF, int VF, int DPL, int GM, int DT>  // GM: max q-heads per KV group held in registers; DT: activation dtype
__global__ __launch_bounds__(64 * DEC_WAVES) void decode_split_kernel(const anna_mi_decode_args a, const Split sp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t blk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = (int)(a.q_heads / a.kv_heads);
  const int64_t D = a.head_dim, L1 = a.len1, L = a.len1 + a.len2;
  // tokens of this row in the two segments (the segments' capacities without seq_lengths)
  int64_t n1 = L1, n2 = a.len2;
  if (a.seq_lengths) {
    const int64_t n = a.seq_lengths[b];
    n2 = n < a.len2 ? n : a.len2;
    n1 = n - n2 < L1 ? n - n2 : L1;
  }

  int64_t t0, t1;
  if (sp.aligned && blk >= sp.nb1) {
    t0 = L1 + (blk - sp.nb1) * sp.eb2;
    t1 = t0 + sp.eb2 < L ? t0 + sp.eb2 : L;
  } else {
    t0 = blk * sp.eb;
    const int64_t lim = sp.aligned ? L1 : L;
    t1 = t0 + sp.eb < lim ? t0 + sp.eb : lim;
  }

  __shared__ float s_m[DEC_WAVES][16], s_l[DEC_WAVES][16];
  extern __shared__ float s_acc[];  // [G][D]
  for (int64_t i = threadIdx.x; i < (int64_t)G * D; i += blockDim.x) s_acc[i] = 0.f;

  // With TQ-MSE keys blocks never straddle the segments: the whole block scores either
  // rotated codes (against q' = R q) or dense residual keys (against q).
  const bool rot_block = KF == ANNA_MI_KEYS_TQ_MSE && t0 < L1;
  // All query loads are issued before any is used (heads beyond G read head G-1 and are
  // then zeroed), so their latencies overlap.
  float qv[GM][DPL];
  if (rot_block) {
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      const int64_t hq = kvh * G + (h < G ? h : G - 1);
#pragma unroll
      for (int j = 0; j < DPL; ++j) qv[h][j] = a.query_rot[(b * a.q_heads + hq) * D + lane * DPL + j];
    }
  } else {
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      const int64_t hq = kvh * G + (h < G ? h : G - 1);
#pragma unroll
      for (int j = 0; j < DPL; ++j)
        qv[h][j] = ldt<DT>(a.query.ptr, b * a.query.s0 + hq * a.query.s1 + (lane * DPL + j) * a.query.s3);
    }
  }
#pragma unroll
  for (int h = 0; h < GM; ++h)
#pragma unroll
    for (int j = 0; j < DPL; ++j)
      if (h >= G) qv[h][j] = 0.f;
  // Online-softmax state: lane L keeps the running max and denominator of head L % GM
  // (log2 units); every lane keeps the accumulators of its dims for all heads.
  float m_run = -INFINITY, l_run = 0.f, acc[GM][DPL];
#pragma unroll
  for (int h = 0; h < GM; ++h)
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[h][j] = 0.f;

  const int ksb = sbits(a.key_bits), kper = 8 / ksb;
  const int vsb = sbits(a.value_bits), vper = 8 / vsb;
  // Per-lane element offsets within one token's row.  They do not depend on the token, so
  // the divisions (packed codes per byte, scale group) are done once, outside the loop.
  // 32-bit: the host checks head_dim * stride < 2^31 for every view read here.
  int32_t koff[DPL], voff[DPL], soff[DPL], zoff[DPL], rkoff[DPL], rvoff[DPL];
  int kshift[DPL], vshift[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int64_t d = lane * DPL + j;
    if constexpr (KF == ANNA_MI_KEYS_TQ_MSE) {
      koff[j] = (int32_t)((d / kper) * a.key.s3);
      kshift[j] = ksb * (int)(d % kper);
    } else {
      koff[j] = (int32_t)(d * a.key.s3);
      kshift[j] = 0;
    }
    if constexpr (VF == ANNA_MI_VALUES_DENSE) {
      voff[j] = (int32_t)(d * a.value.s3);
      vshift[j] = 0;
    } else {
      voff[j] = (int32_t)((d / vper) * a.value.s3);
      vshift[j] = vsb * (int)(d % vper);
    }
    if constexpr (VF == ANNA_MI_VALUES_MINMAX) {
      const int64_t g = d / a.value_group_size;
      soff[j] = (int32_t)(g * a.value_scales.s3);
      zoff[j] = (int32_t)(g * a.value_zeros.s3);
    } else {
      soff[j] = zoff[j] = 0;
    }
    rkoff[j] = (int32_t)(d * a.residual_key.s3);
    rvoff[j] = (int32_t)(d * a.residual_value.s3);
  }
  const uint32_t kmask = (1u << ksb) - 1u, vmask = (1u << vsb) - 1u;
  const float scale2 = a.scaling * 1.4426950408889634f;  // scores in log2 units
  // Loads one token's K and V rows (dequantized) into registers: every load of the token is
  // issued before any value is used.
  // VEC: the key row slice of a lane is one aligned vector load (dense keys) and the lane's
  // dims share one scale/zero (min/max values); the host sets it when the views allow it.
  auto load_packed = [&](int64_t t, float (&kv)[DPL], float (&vv)[DPL], auto vec_tag) {
    constexpr bool VEC = decltype(vec_tag)::value;
    {
      const int64_t kb = b * a.key.s0 + kvh * a.key.s1 + t * a.key.s2;
      const int64_t vb = b * a.value.s0 + kvh * a.value.s1 + t * a.value.s2;
      if constexpr (KF == ANNA_MI_KEYS_TQ_MSE) {
        const float nk = f16_bits_to_f32(((const uint16_t*)a.key_norms.ptr)[b * a.key_norms.s0 + kvh * a.key_norms.s1 +
                                                                            t * a.key_norms.s2]);
        uint32_t kc[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) kc[j] = ((const uint8_t*)a.key.ptr)[kb + koff[j]];
#pragma unroll
        for (int j = 0; j < DPL; ++j) kv[j] = a.key_centroids[(kc[j] >> kshift[j]) & kmask] * nk;
      } else if constexpr (VEC) {
        using E = typename std::conditional<DT == ANNA_MI_F32, uint32_t, uint16_t>::type;
        struct alignas(sizeof(E) * DPL) Row { E x[DPL]; };
        const Row r = *(const Row*)((const E*)a.key.ptr + kb + lane * DPL);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          if constexpr (DT == ANNA_MI_BF16) kv[j] = bf16_bits_to_f32(r.x[j]);
          else if constexpr (DT == ANNA_MI_F16) kv[j] = f16_bits_to_f32(r.x[j]);
          else kv[j] = __uint_as_float(r.x[j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < DPL; ++j) kv[j] = ldt<DT>(a.key.ptr, kb + koff[j]);
      }
      if constexpr (VF == ANNA_MI_VALUES_DENSE) {
#pragma unroll
        for (int j = 0; j < DPL; ++j) vv[j] = ldt<DT>(a.value.ptr, vb + voff[j]);
      } else if constexpr (VF == ANNA_MI_VALUES_MINMAX) {
        const int64_t sb0 = b * a.value_scales.s0 + kvh * a.value_scales.s1 + t * a.value_scales.s2;
        const int64_t zb0 = b * a.value_zeros.s0 + kvh * a.value_zeros.s1 + t * a.value_zeros.s2;
        uint32_t vc[DPL];
        float sc[DPL], zc[DPL];
        if constexpr (VEC) {
          const float s0 = ldt<DT>(a.value_scales.ptr, sb0 + soff[0]), z0 = ldt<DT>(a.value_zeros.ptr, zb0 + zoff[0]);
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            vc[j] = ((const uint8_t*)a.value.ptr)[vb + voff[j]];
            sc[j] = s0;
            zc[j] = z0;
          }
        } else {
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            vc[j] = ((const uint8_t*)a.value.ptr)[vb + voff[j]];
            sc[j] = ldt<DT>(a.value_scales.ptr, sb0 + soff[j]);
            zc[j] = ldt<DT>(a.value_zeros.ptr, zb0 + zoff[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < DPL; ++j) vv[j] = (float)((vc[j] >> vshift[j]) & vmask) * sc[j] + zc[j];
      } else {
        const float nv = f16_bits_to_f32(((const uint16_t*)a.value_scales.ptr)[b * a.value_scales.s0 +
                                                                               kvh * a.value_scales.s1 +
                                                                               t * a.value_scales.s2]);
        uint32_t vc[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) vc[j] = ((const uint8_t*)a.value.ptr)[vb + voff[j]];
#pragma unroll
        for (int j = 0; j < DPL; ++j) vv[j] = a.value_centroids[(vc[j] >> vshift[j]) & vmask] * nv;
      }
    }
  };
  auto load_residual = [&](int64_t t, float (&kv)[DPL], float (&vv)[DPL]) {
    {
      const anna_mi_view& rk = a.residual_key;
      const anna_mi_view& rv = a.residual_value;
      const int64_t tr = t - L1;
      const int64_t kb = b * rk.s0 + kvh * rk.s1 + tr * rk.s2, vb = b * rv.s0 + kvh * rv.s1 + tr * rv.s2;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        kv[j] = ldt<DT>(rk.ptr, kb + rkoff[j]);
        vv[j] = ldt<DT>(rv.ptr, vb + rvoff[j]);
      }
    }
  };
  // Scores DEC_TOKENS tokens (token u valid when t + u * DEC_WAVES < hi) for every head.
  // The NV = DEC_TOKENS * GM per-lane partial dot products are summed over the wave by a
  // transposed butterfly: stage k exchanges across lane bit k and halves the list (a lane
  // keeps the half selected by that bit), so after log2(NV) stages lane L holds the full dot
  // product of value (L % NV) = u * GM + h.  The softmax update then runs one (u, h) per lane
  // and the weights reach all lanes as scalars (readlane).
  constexpr int NV = DEC_TOKENS * GM;
  static_assert(NV == 32 || NV == 64, "butterfly sized for 32 or 64 values");
  const int my_h = lane % GM, my_u = (lane / GM) % DEC_TOKENS;
  auto score_step = [&](const float (&kv)[DEC_TOKENS][DPL], const float (&vv)[DEC_TOKENS][DPL], int64_t t,
                        int64_t hi) {
    float v[NV];
#pragma unroll
    for (int u = 0; u < DEC_TOKENS; ++u)
#pragma unroll
      for (int h = 0; h < GM; ++h) {
        float p = 0.f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) p = fmaf(qv[h][j], kv[u][j], p);
        v[u * GM + h] = p;
      }
#pragma unroll
    for (int k = 0; (NV >> k) > 1; ++k) {
      const bool hi_half = (lane >> k) & 1;
#pragma unroll
      for (int i = 0; i < (NV >> k) / 2; ++i) {
        const float keep = hi_half ? v[2 * i + 1] : v[2 * i];
        const float send = hi_half ? v[2 * i] : v[2 * i + 1];
        float got;
        if (k == 0) got = dpp_f32<0xB1>(send);       // lane ^ 1 (quad_perm [1,0,3,2])
        else if (k == 1) got = dpp_f32<0x4E>(send);  // lane ^ 2 (quad_perm [2,3,0,1])
        else got = __shfl_xor(send, 1 << k, 64);
        v[i] = keep + got;
      }
    }
    float sc = v[0];
    if constexpr (NV == 32) sc += __shfl_xor(sc, 32, 64);  // the two half-waves hold partial sums
    sc = t + my_u * DEC_WAVES < hi ? sc * scale2 : -INFINITY;
    float mb = fmaxf(sc, __shfl_xor(sc, GM, 64));
    mb = fmaxf(mb, __shfl_xor(mb, 2 * GM, 64));
    const float nm = fmaxf(m_run, mb);
    const float alpha = l_run == 0.f ? 0.f : __builtin_amdgcn_exp2f(m_run - nm);
    const float e = __builtin_amdgcn_exp2f(sc - nm);
    float es = e + __shfl_xor(e, GM, 64);
    es = es + __shfl_xor(es, 2 * GM, 64);
    l_run = l_run * alpha + es;
    m_run = nm;
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      if (h >= G) continue;
      const float ah = lane_f32(alpha, h);
      float eu[DEC_TOKENS];
#pragma unroll
      for (int u = 0; u < DEC_TOKENS; ++u) eu[u] = lane_f32(e, u * GM + h);
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        float x = acc[h][j] * ah;
#pragma unroll
        for (int u = 0; u < DEC_TOKENS; ++u) x = fmaf(eu[u], vv[u][j], x);
        acc[h][j] = x;
      }
    }
  };
  // Wave w scores tokens t0 + w, t0 + w + 4, ... in ascending order.  The packed segment
  // and the residual segment run as two loops so neither loop body branches on the segment;
  // each step loads DEC_TOKENS tokens, then scores them together.
  auto sweep = [&](int64_t lo, int64_t hi, auto&& load) {
    int64_t t = t0 + wave;
    if (t < lo) t += (lo - t + DEC_WAVES - 1) / DEC_WAVES * DEC_WAVES;
    for (; t < hi; t += DEC_TOKENS * DEC_WAVES) {
      float kv[DEC_TOKENS][DPL], vv[DEC_TOKENS][DPL];
#pragma unroll
      for (int u = 0; u < DEC_TOKENS; ++u) {
        const int64_t tu = t + u * DEC_WAVES;
        load(tu < hi ? tu : t, kv[u], vv[u]);  // unconditional: no branch between the loads
      }
      score_step(kv, vv, t, hi);
    }
  };
  if (sp.vec) {
    sweep(t0, t1 < n1 ? t1 : n1,
          [&](int64_t t, float (&kv)[DPL], float (&vv)[DPL]) { load_packed(t, kv, vv, std::true_type{}); });
  } else {
    sweep(t0, t1 < n1 ? t1 : n1,
          [&](int64_t t, float (&kv)[DPL], float (&vv)[DPL]) { load_packed(t, kv, vv, std::false_type{}); });
  }
  sweep(t0 > L1 ? t0 : L1, t1 < L1 + n2 ? t1 : L1 + n2, load_residual);
  // merge the 4 waves: common max, rescale, ordered sum in LDS
  if (lane < G) {  // lane h < GM holds head h's state
    s_m[wave][lane] = m_run;
    s_l[wave][lane] = l_run;
  }
  __syncthreads();
  // waves add in a fixed order (deterministic sums; each lane owns its entries)
  for (int w = 0; w < DEC_WAVES; ++w) {
    if (wave == w) {
#pragma unroll
      for (int h = 0; h < GM; ++h) {
        if (h >= G) continue;
        float M = -INFINITY;
        for (int w2 = 0; w2 < DEC_WAVES; ++w2) M = fmaxf(M, s_m[w2][h]);
        const float f = s_l[wave][h] == 0.f ? 0.f : __builtin_amdgcn_exp2f(s_m[wave][h] - M);
#pragma unroll
        for (int j = 0; j < DPL; ++j) s_acc[h * D + lane * DPL + j] += acc[h][j] * f;
      }
    }
    __syncthreads();
  }
  for (int64_t i = threadIdx.x; i < (int64_t)G * D; i += blockDim.x) {
    const int h = (int)(i / D);
    const int64_t d = i % D, hq = kvh * G + h;
    const anna_mi_view& pv = a.partial_values;
    ((float*)pv.ptr)[b * pv.s0 + hq * pv.s1 + blk * pv.s2 + d * pv.s3] = s_acc[i];
  }
  if (threadIdx.x < G) {
    const int h = threadIdx.x;
    float M = -INFINITY, S = 0.f;
    for (int w = 0; w < DEC_WAVES; ++w) M = fmaxf(M, s_m[w][h]);
    for (int w = 0; w < DEC_WAVES; ++w)
      if (s_l[w][h] != 0.f) S += s_l[w][h] * __builtin_amdgcn_exp2f(s_m[w][h] - M);
    const anna_mi_view& ps = a.partial_stats;
    const int64_t base = b * ps.s0 + (kvh * G + h) * ps.s1 + blk * ps.s2;
    ((float*)ps.ptr)[base] = M * 0.6931471805599453f;  // back to natural-log units
    ((float*)ps.ptr)[base + ps.s3] = S;
  }
}

// grid (Hq, B), MERGE_THREADS threads.  Blocks [0, nrot) hold rotated (TQ-MSE) value
// accumulators.  Thread t owns dim t % D and the blocks k = t / D (mod MERGE_THREADS / D);
// the slices are then added in slice order, so the result does not depend on timing.
__global__ __launch_bounds__(MERGE_THREADS) void decode_merge_kernel(const anna_mi_decode_args a, int64_t nblk,
                                                                     int64_t nrot) {
  extern __shared__ float s_rot[];  // [D] rotated accumulator
  __shared__ float s_red[MERGE_THREADS];
  __shared__ float s_w[MERGE_CHUNK];
  __shared__ float s_part[2][MERGE_THREADS];
  const int64_t h = blockIdx.x, b = blockIdx.y, D = a.head_dim;
  const int tid = threadIdx.x;
  const anna_mi_view& ps = a.partial_stats;
  const anna_mi_view& pv = a.partial_values;
  const float* st = (const float*)ps.ptr + b * ps.s0 + h * ps.s1;
  const float* va = (const float*)pv.ptr + b * pv.s0 + h * pv.s1;
  // Block tid's stats and this thread's first MERGE_PRE partial values are loaded up front,
  // so their latency overlaps the reductions below (later blocks are read as needed).
  const int ks = (int)(MERGE_THREADS / D), slice = tid / (int)D;
  const int64_t d = tid % D;
  const float* vd = va + d * pv.s3;
  const int64_t kn0 = nblk < MERGE_CHUNK ? nblk : MERGE_CHUNK;
  float pre[MERGE_PRE];
#pragma unroll
  for (int i = 0; i < MERGE_PRE; ++i) {
    const int64_t k = slice + (int64_t)i * ks;
    pre[i] = k < kn0 ? vd[k * pv.s2] : 0.f;
  }
  float m0 = -INFINITY, d0 = 0.f;
  if (tid < nblk) {
    m0 = st[(int64_t)tid * ps.s2];
    d0 = st[(int64_t)tid * ps.s2 + ps.s3];
  }
  float mx = m0;
  for (int64_t k = tid + MERGE_THREADS; k < nblk; k += MERGE_THREADS) mx = fmaxf(mx, st[k * ps.s2]);
  s_red[tid] = mx;
  __syncthreads();
  for (int s = MERGE_THREADS / 2; s > 0; s >>= 1) {
    if (tid < s) s_red[tid] = fmaxf(s_red[tid], s_red[tid + s]);
    __syncthreads();
  }
  const float M = s_red[0];
  __syncthreads();
  const float w0 = d0 == 0.f ? 0.f : expf(m0 - M);  // weight of block tid
  float den = d0 == 0.f ? 0.f : d0 * w0;
  for (int64_t k = tid + MERGE_THREADS; k < nblk; k += MERGE_THREADS) {
    const float dk = st[k * ps.s2 + ps.s3];
    if (dk != 0.f) den += dk * expf(st[k * ps.s2] - M);
  }
  s_red[tid] = den;
  __syncthreads();
  for (int s = MERGE_THREADS / 2; s > 0; s >>= 1) {
    if (tid < s) s_red[tid] += s_red[tid + s];
    __syncthreads();
  }
  const float denom = s_red[0];
  // Block weights exp(m_k - M) go through LDS a chunk at a time (0 for empty blocks).  Thread
  // (slice, d) sums blocks slice, slice + ks, ... in ascending order.
  float ar = 0.f, aq = 0.f;
  for (int64_t kc = 0; kc < nblk; kc += MERGE_CHUNK) {
    const int64_t kn = nblk - kc < MERGE_CHUNK ? nblk - kc : MERGE_CHUNK;
    if (kc == 0) {
      if (tid < kn) s_w[tid] = w0;
    } else {
      for (int64_t k = tid; k < kn; k += MERGE_THREADS) {
        const int64_t kk = kc + k;
        const float dk = st[kk * ps.s2 + ps.s3];
        s_w[k] = dk == 0.f ? 0.f : expf(st[kk * ps.s2] - M);
      }
    }
    __syncthreads();
    const int64_t kr = nrot - kc < 0 ? 0 : (nrot - kc < kn ? nrot - kc : kn);  // [0, kr) rotated blocks
    auto add = [&](int64_t k, float v) {
      const float w = s_w[k];
      if (w != 0.f) {
        if (k < kr) ar += w * v;
        else aq += w * v;
      }
    };
    int64_t k = slice;
    if (kc == 0) {
#pragma unroll
      for (int i = 0; i < MERGE_PRE; ++i, k += ks)
        if (k < kn) add(k, pre[i]);
    }
#pragma unroll 8
    for (; k < kn; k += ks) add(k, vd[(kc + k) * pv.s2]);
    __syncthreads();
  }
  s_part[0][tid] = ar;
  s_part[1][tid] = aq;
  __syncthreads();
  if (tid < D) {
    float r = 0.f, q = 0.f;
    for (int i = 0; i < ks; ++i) {
      r += s_part[0][i * D + tid];
      q += s_part[1][i * D + tid];
    }
    if (nrot > 0) s_rot[tid] = r;
    aq = q;
  }
  if (nrot > 0) __syncthreads();
  if (tid < D) {
    float o = aq;
    if (nrot > 0) {
      float u = 0.f;
      for (int64_t i = 0; i < D; ++i) u = fmaf(a.rotation[i * D + d], s_rot[i], u);
      o += u;
    }
    o = denom > 0.f ? o / denom : 0.f;
    if (a.gate_layout == ANNA_MI_GATE_FLAT) {
      o *= 1.f / (1.f + expf(-ldv(a.gate.ptr, b * a.gate.s0 + (h * D + d) * a.gate.s2, a.dtype)));
    } else if (a.gate_layout == ANNA_MI_GATE_HEADS) {
      o *= 1.f / (1.f + expf(-ldv(a.gate.ptr, b * a.gate.s0 + h * a.gate.s1 + d * a.gate.s3, a.dtype)));
    }
    stv(a.out.ptr, b * a.out.s0 + h * a.out.s1 + d * a.out.s3, a.dtype, o);
  }
}

// grid (D / 64, Hq, B), 256 threads: the merge when no block holds rotated accumulators and
// there are at most MERGE_DIM_MAXBLK blocks.  Thread t loads the stats of block t while every
// lane's first MERGE_DIM_PRE partial values are in flight; the max, the block weights
// exp(m_k - M) (LDS) and the denominator take two barriers.  Lane l of each wave owns dim
// 64 blockIdx.x + l; wave w sums the contiguous blocks [w n4, w n4 + n4) in ascending order and
// the four sums are added in wave order, so the result does not depend on timing.
constexpr int MERGE_DIM_WAVES = 4;
constexpr int MERGE_DIM_MAXBLK = 64 * MERGE_DIM_WAVES;
constexpr int MERGE_DIM_PRE = 32;  // partial values per lane loaded before the reductions

__global__ __launch_bounds__(64 * MERGE_DIM_WAVES) void decode_merge_dims_kernel(const anna_mi_decode_args a,
                                                                                 int64_t nblk) {
  __shared__ float s_w[MERGE_DIM_MAXBLK];
  __shared__ float s_red[2][MERGE_DIM_WAVES];
  __shared__ float s_sum[MERGE_DIM_WAVES][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t h = blockIdx.y, b = blockIdx.z, d = (int64_t)blockIdx.x * 64 + lane;
  const anna_mi_view& ps = a.partial_stats;
  const anna_mi_view& pv = a.partial_values;
  const float* st = (const float*)ps.ptr + b * ps.s0 + h * ps.s1;
  const float* vd = (const float*)pv.ptr + b * pv.s0 + h * pv.s1 + d * pv.s3;
  const int n = (int)nblk, n4 = (n + MERGE_DIM_WAVES - 1) / MERGE_DIM_WAVES;
  const int k0 = wave * n4, k1 = k0 + n4 < n ? k0 + n4 : n;
  float pre[MERGE_DIM_PRE];
#pragma unroll
  for (int i = 0; i < MERGE_DIM_PRE; ++i) pre[i] = k0 + i < k1 ? vd[(int64_t)(k0 + i) * pv.s2] : 0.f;
  float mk = -INFINITY, dk = 0.f;
  if (tid < n) {
    mk = st[(int64_t)tid * ps.s2];
    dk = st[(int64_t)tid * ps.s2 + ps.s3];
  }
  float mx = mk;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
  if (lane == 0) s_red[0][wave] = mx;
  __syncthreads();
  float M = s_red[0][0];
#pragma unroll
  for (int w = 1; w < MERGE_DIM_WAVES; ++w) M = fmaxf(M, s_red[0][w]);
  const float wk = dk == 0.f ? 0.f : expf(mk - M);
  s_w[tid] = wk;
  float den = dk * wk;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) den += __shfl_xor(den, m, 64);
  if (lane == 0) s_red[1][wave] = den;
  __syncthreads();
  den = s_red[1][0];
#pragma unroll
  for (int w = 1; w < MERGE_DIM_WAVES; ++w) den += s_red[1][w];

  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < MERGE_DIM_PRE; ++i) {
    if (k0 + i < k1) {
      const float w = s_w[k0 + i];
      if (w != 0.f) acc += w * pre[i];
    }
  }
#pragma unroll 8
  for (int k = k0 + MERGE_DIM_PRE; k < k1; ++k) {
    const float v = vd[(int64_t)k * pv.s2];
    const float w = s_w[k];
    if (w != 0.f) acc += w * v;
  }
  s_sum[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  float o = s_sum[0][lane];
#pragma unroll
  for (int w = 1; w < MERGE_DIM_WAVES; ++w) o += s_sum[w][lane];
  o = den > 0.f ? o / den : 0.f;
  if (a.gate_layout == ANNA_MI_GATE_FLAT) {
    o *= 1.f / (1.f + expf(-ldv(a.gate.ptr, b * a.gate.s0 + (h * a.head_dim + d) * a.gate.s2, a.dtype)));
  } else if (a.gate_layout == ANNA_MI_GATE_HEADS) {
    o *= 1.f / (1.f + expf(-ldv(a.gate.ptr, b * a.gate.s0 + h * a.gate.s1 + d * a.gate.s3, a.dtype)));
  }
  stv(a.out.ptr, b * a.out.s0 + h * a.out.s1 + d * a.out.s3, a.dtype, o);
}

// ------------------------------------------------------------------ MFMA split kernel
//
// Fast path of the split kernel for 16-bit activations, dense keys (packed segment and window)
// and dense or min/max-packed values, head_dim 64/128/256, G <= 16 query heads per KV head.
// One wave per workgroup owns a range of `range` tokens of one (KV head, batch) and walks it in
// 32-token tiles.  The range is chosen on the host (a multiple of 32, about 1536 waves in all, no
// more partials than the caller's workspace holds), independently of the caller's block size.
//   * S^T = K Q^T by v_mfma_f32_16x16x32 (A = 16 key rows x 32 dims straight from memory, B = the
//     query heads' fragments, kept in registers; two MFMAs per 32 dims for tokens r and 16 + r).
//   * Online softmax in base 2, rescaled lazily; the probabilities' accumulator layout is already
//     the A operand of O = P V (16 heads x 32 tokens, token k of lane (head, kq) = 4 kq + e
//     (e < 4) or 16 + 4 kq + e - 4), so P never leaves registers.
//   * V of the tile is staged in LDS transposed, [dim][token] in the activation dtype (min/max
//     codes dequantized as q * scale + zero on the way; window tokens copied), so that the B
//     operand of lane (dim, kq) is two 8-byte reads.
//   * With a fixed tile count (1..4) all of the range's loads are issued at the start, one
//     register set per tile; otherwise two sets hold tiles n and n + 1 and tile n + 2's loads go
//     into set n % 2 right after tile n's scores.  Two tiles per wave run two waves per SIMD
//     (228 registers); three or four run one; TQ-MSE keys at head_dim <= 128 run two (within 256
//     registers and no spills since the packed tiles' addressing is 32-bit: 28.7 -> 27.7 us for
//     TurboQuantRowsCache at D = 128), at 256 one.
// Each wave writes its range's partial from registers in the reference layout (natural-log max,
// denominator, unnormalized values), so the merge kernels take it as they take the VALU
// kernel's blocks.
constexpr int MF_TILE = 32;         // tokens per tile
constexpr int MF_VT = MF_TILE + 4;  // LDS pitch (elements) of the transposed V tile: 18 words,
                                    // so the 16 dims of a B-operand read hit distinct banks
constexpr int64_t MF_WAVES_TARGET = 1536;  // about 6 waves per CU (NT = 2 runs two waves per SIMD)
constexpr int64_t MF_WAVES_TQ2 = 2048;     // 8 per CU: the TQ-MSE-key instances at head_dim <= 128
constexpr int64_t MF_WAVES_TQ1 = 1024;     // 4 per CU: the TQ-MSE-key instances at head_dim 256

// Two floats rounded to nearest-even into the activation dtype, lo in bits 0..15 (one
// v_cvt_pk_bf16_f32 for bf16).
template <int DT>
__device__ __forceinline__ uint32_t pack2_16(float lo, float hi) {
  if constexpr (DT == ANNA_MI_BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
}

// Loads of one tile: key rows, and the raw min/max codes of the lane's two staging tokens (the
// lane's QD dims of a token are one CW-word vector load) with their scales and zeros (span i of
// 32 dims, token u; one zero-extended 16-bit load each, so nothing is combined before use).
// KSB (TQ-MSE keys): the code words of tokens r and 16 + r (the lane's D / 4 dims) and the norms
// of the lane's eight score rows.
template <int D, int SB, int KSB>
struct MfmaTileRegs {
  static constexpr int NST = D / 32, QD = D / 4, NSP = QD >= 32 ? QD / 32 : 1;
  static constexpr int CW = SB == 0 ? 1 : (QD * SB / 8 + 3) / 4;  // 32-bit words of codes per token
  static constexpr int KCW = KSB == 0 ? 1 : QD * KSB / 32;         // 32-bit words of key codes per lane
  u32x4 ka[NST], kb[NST];
  uint32_t vc[2][CW], vsc[NSP][2], vzr[NSP][2];
  uint32_t kc[2][KCW];
  uint32_t kn[8];
};

// n 32-bit words from p (aligned to min(4 n, 16) bytes) as whole-vector non-temporal loads (the
// cache's codes are read once per call).
typedef uint32_t u32x2w __attribute__((ext_vector_type(2)));
template <int N>
__device__ __forceinline__ void load_words(uint32_t (&w)[N], const uint8_t* p) {
  if constexpr (N == 1) {
    w[0] = __builtin_nontemporal_load((const uint32_t*)p);
  } else if constexpr (N == 2) {
    const u32x2w v = __builtin_nontemporal_load((const u32x2w*)p);
    w[0] = v[0];
    w[1] = v[1];
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x4 v = __builtin_nontemporal_load((const u32x4*)(p + 16 * i));
#pragma unroll
      for (int e = 0; e < 4; ++e) w[4 * i + e] = v[e];
    }
  }
}


// SB: storage bits of a min/max code (2, or 4 for 3- and 4-bit values); 0 for dense values.
// NT: tiles per range, fixed (1..4: every load is issued unconditionally, from clamped rows past
// the range's end, so the compiler waits for exactly the loads each step uses), or 0 (any count,
// runtime loop).
// KSB: 0 for dense keys; 2 or 4 for TQ-MSE key codes in fields of that many bits.  Then the
// ranges are aligned to the segments (the first nr1 cover the packed tokens, the rest the window):
// a packed range scores its codes, turned into fp16 centroids by a 256-entry LDS table (code byte
// -> its 2 or 4 centroids), against the rotated query q' = R q (fp16 fragments, lane (head, kq) of
// step st: dims QD kq + 8 st .. + 7) and scales each score by its token's norm; a window range
// runs as with dense keys.
// SEQ: per-row lengths (a.seq_lengths): row b's valid tokens are the first n1 packed slots and
// the first n2 window slots; a range with none of them writes an empty partial.
template <int DT, int VF, int SB, int D, int NT, int KSB, bool SEQ>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(NT == 2 || (KSB > 0 && D <= 128) ? 2 : 1, NT == 2 || (KSB > 0 && D <= 128) ? 2 : 1))) void decode_split_mfma_kernel(
    const anna_mi_decode_args a, const int64_t range, const int64_t nr1) {
  using Regs = MfmaTileRegs<D, SB, KSB>;
  constexpr int NST = Regs::NST, NSP = Regs::NSP, QD = Regs::QD, CW = Regs::CW, KCW = Regs::KCW;
  constexpr int NDT = D / 16;  // 16-dim tiles of the value product
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float LAZY = 4.0f;
  const int lane = threadIdx.x;
  const int r = lane & 15, kq = lane >> 4;
  const int p = lane & 15, qr = lane >> 4;  // staging role: tokens 2p, 2p + 1, dims QD qr ..
  const int64_t blk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = (int)(a.q_heads / a.kv_heads);
  const int64_t L1 = a.len1, L = a.len1 + a.len2;
  int64_t t0, t1;
  bool packed_rng = false;  // (TQ-MSE keys) a range of packed tokens
  if (KSB > 0 && blk < nr1) {
    t0 = blk * range;
    t1 = t0 + range < L1 ? t0 + range : L1;
    packed_rng = true;
  } else {
    t0 = KSB > 0 ? L1 + (blk - nr1) * range : blk * range;
    t1 = t0 + range < L ? t0 + range : L;
  }
  // row b's valid tokens: [0, n1) and [L1, L1 + n2)
  int64_t n1 = L1, n2 = a.len2;
  if constexpr (SEQ) {
    const int64_t n = a.seq_lengths[b];
    n2 = n < a.len2 ? n : a.len2;
    n1 = n - n2 < L1 ? n - n2 : L1;
  }
  // TQ-MSE keys: the ranges are aligned to the segments, so a token of the range is valid below
  // one limit (32-bit compares: the host keeps token indices below 2^31)
  const int vlim = (int)(packed_rng ? (t1 < n1 ? t1 : n1) : (t1 < L1 + n2 ? t1 : L1 + n2));
  auto valid = [&](int64_t t) {
    if constexpr (KSB > 0) return (int)t < vlim;
    else return t < t1 && (!SEQ || t < n1 || (t >= L1 && t < L1 + n2));
  };
  const bool live = !SEQ || t0 < n1 || (t1 > L1 && t0 < L1 + n2);
  const int ntiles = NT > 0 ? NT : (int)((t1 - t0 + MF_TILE - 1) / MF_TILE);
  // raw-code staging: scale groups of whole 32-dim spans, code vectors aligned for one load
  constexpr uintptr_t CA = 4 * CW < 16 ? 4 * CW : 16;
  const bool rawok = VF == ANNA_MI_VALUES_MINMAX && a.value_group_size % 32 == 0 && a.value.s3 == 1 &&
                     ((uintptr_t)a.value.ptr | (uintptr_t)a.value.s0 | (uintptr_t)a.value.s1 |
                      (uintptr_t)a.value.s2) % CA == 0;

  // Row bases and strides of this (batch, KV head), uniform: a per-lane choice between the packed
  // segment and the window then selects between two computed addresses (a select between the
  // views themselves would load the strides per lane).
  const uint16_t* const key0 = (const uint16_t*)a.key.ptr + b * a.key.s0 + kvh * a.key.s1;
  const uint16_t* const rkey0 = (const uint16_t*)a.residual_key.ptr + b * a.residual_key.s0 + kvh * a.residual_key.s1;
  // values: 16-bit elements (dense) or code bytes (min/max); vb0 and vbs2 in bytes
  constexpr int VESZ = VF == ANNA_MI_VALUES_DENSE ? 2 : 1;
  const uint8_t* const vb0 = (const uint8_t*)a.value.ptr + VESZ * (b * a.value.s0 + kvh * a.value.s1);
  const int64_t vbs2 = VESZ * a.value.s2;
  const uint16_t* const rval0 = (const uint16_t*)a.residual_value.ptr + b * a.residual_value.s0 + kvh * a.residual_value.s1;
  const int64_t ks2 = a.key.s2, rks2 = a.residual_key.s2, rvs2 = a.residual_value.s2;
  auto key_row = [&](int64_t t) { return t < L1 ? key0 + t * ks2 : rkey0 + (t - L1) * rks2; };
  // a 16-byte aligned row that is always there (the host checks the key rows' alignment when
  // there is a packed segment, the window's otherwise): the target of loads that feed nothing
  const uint16_t* const safe16 = L1 > 0 ? key0 : rkey0;
  // TQ-MSE packed ranges with raw values: per-lane 32-bit byte offsets (from the uniform row
  // bases) of what tile 0 loads; tile n adds n tiles of stride, and the clamp into the range is a
  // min on the offset (offsets grow with the token).  The host keeps each (batch, KV head) slice
  // of these arrays below 2^31 bytes.
  const bool tqfast = KSB > 0 && packed_rng;  // (the host sends TQ-MSE keys only with raw-ready values)
  const uint8_t* const sb0 = (const uint8_t*)a.value_scales.ptr + 2 * (b * a.value_scales.s0 + kvh * a.value_scales.s1);
  const uint8_t* const zb0 = (const uint8_t*)a.value_zeros.ptr + 2 * (b * a.value_zeros.s0 + kvh * a.value_zeros.s1);
  const uint8_t* const kcb0 = (const uint8_t*)a.key.ptr + b * a.key.s0 + kvh * a.key.s1;
  uint32_t o_v0 = 0, o_v1 = 0, o_s0 = 0, o_s1 = 0, o_z0 = 0, o_z1 = 0, o_ka = 0, o_kb = 0, lim_v = 0, lim_k = 0;
  const uint32_t inc_v = (uint32_t)(MF_TILE * vbs2), inc_s = (uint32_t)(2 * MF_TILE * a.value_scales.s2),
                 inc_z = (uint32_t)(2 * MF_TILE * a.value_zeros.s2), inc_k = (uint32_t)(MF_TILE * a.key.s2);
  const uint32_t lim_s = (uint32_t)(2 * (t1 - 1) * a.value_scales.s2), lim_z = (uint32_t)(2 * (t1 - 1) * a.value_zeros.s2);
  if (tqfast) {
    const uint32_t cv = (uint32_t)(QD * qr * SB / 8), ck = (uint32_t)(QD * kq * KSB / 8);
    const int64_t t = t0 + 2 * p;
    o_v0 = (uint32_t)(t * vbs2) + cv;
    o_v1 = o_v0 + (uint32_t)vbs2;
    o_s0 = (uint32_t)(2 * t * a.value_scales.s2);
    o_s1 = o_s0 + (uint32_t)(2 * a.value_scales.s2);
    o_z0 = (uint32_t)(2 * t * a.value_zeros.s2);
    o_z1 = o_z0 + (uint32_t)(2 * a.value_zeros.s2);
    lim_v = (uint32_t)((t1 - 1) * vbs2) + cv;
    o_ka = (uint32_t)((t0 + r) * a.key.s2) + ck;
    o_kb = (uint32_t)((t0 + 16 + r) * a.key.s2) + ck;
    lim_k = (uint32_t)((t1 - 1) * a.key.s2) + ck;
  }
  // byte offset of the lane's scale / zero group of span i (32 dims)
  auto gofs = [&](int i, int64_t s3) { return (uint32_t)(2 * ((QD * qr + 32 * i) / a.value_group_size) * s3); };

  __shared__ __attribute__((aligned(16))) uint16_t s_vt[D * MF_VT];
  __shared__ u32x4 s_qf[NST][64];
  // TQ-MSE keys: code byte -> fp16 centroids of its codes, lowest field first (4-bit fields: 2 per
  // entry; 2-bit: 4 per entry)
  __shared__ uint32_t s_klut[KSB == 0 ? 1 : KSB == 4 ? 256 : 512];
  if constexpr (KSB > 0) {
    const uint32_t cmask = (1u << a.key_bits) - 1u;  // 3-bit codes in 4-bit fields stay below 8
    auto c16 = [&](uint32_t c) { return (uint32_t)f32_to_f16_bits(a.key_centroids[c & cmask]); };
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t e = (uint32_t)(lane + 64 * i);
      if constexpr (KSB == 4) {
        s_klut[e] = c16(e & 15u) | (c16(e >> 4) << 16);
      } else {
        s_klut[2 * e] = c16(e & 3u) | (c16((e >> 2) & 3u) << 16);
        s_klut[2 * e + 1] = c16((e >> 4) & 3u) | (c16(e >> 6) << 16);
      }
    }
  }
  uint32_t* vw = (uint32_t*)s_vt;  // word (d, p) at d * MF_VT / 2 + p: dim d of tokens 2p, 2p + 1

  // the raw path takes tiles whose tokens are all packed (min/max); others are staged by the
  // chunked loop below
  auto raw_tile = [&](int64_t tt0) { return rawok && (tt0 + MF_TILE <= L1 || t1 <= L1); };
  // PK (TQ-MSE keys): the tile belongs to a packed range.  Packed and window ranges run separate
  // instances of the loads and of the tile step, so that neither carries the other's code.  (A
  // third instance for dense-key ranges inside the packed segment pushed the row-API kernel past
  // 256 registers into scratch: 22.2 -> 25.8 us.)
  using PkT = std::integral_constant<bool, true>;
  using PkF = std::integral_constant<bool, false>;
  auto issue = [&](Regs& R, int n, auto pk) __attribute__((always_inline)) {
    constexpr bool PK = KSB > 0 && decltype(pk)::value;
    const int64_t tt0 = t0 + (int64_t)MF_TILE * n;
    if constexpr (KSB > 0) {
      // packed ranges: codes, scales and zeros of the lane's two staging tokens, the key codes of
      // tokens r and 16 + r, one add and one min per address (window ranges: dense keys below,
      // no value codes)
      const uint32_t nn = (uint32_t)n;
      if constexpr (PK) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t tv = min((u ? o_v1 : o_v0) + nn * inc_v, lim_v);
        load_words<CW>(R.vc[u], vb0 + tv);
        const uint32_t ts = min((u ? o_s1 : o_s0) + nn * inc_s, lim_s), tz = min((u ? o_z1 : o_z0) + nn * inc_z, lim_z);
#pragma unroll
        for (int i = 0; i < NSP; ++i) {
          R.vsc[i][u] = *(const uint16_t*)(sb0 + ts + gofs(i, a.value_scales.s3));
          R.vzr[i][u] = *(const uint16_t*)(zb0 + tz + gofs(i, a.value_zeros.s3));
        }
      }
      load_words<KCW>(R.kc[0], kcb0 + min(o_ka + nn * inc_k, lim_k));
      load_words<KCW>(R.kc[1], kcb0 + min(o_kb + nn * inc_k, lim_k));
      }
    } else if constexpr (VF == ANNA_MI_VALUES_MINMAX) {
      // tokens clamped into the range and the packed segment; a tile that is not staged from
      // these registers still loads them (from the first packed token, or from safe16 when
      // there is none or the codes are not aligned) when NT is fixed, so the load count never
      // varies
      if (NT > 0 || raw_tile(tt0)) {
        const bool real = raw_tile(tt0);
        int64_t t[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          t[u] = tt0 + 2 * p + u < t1 ? tt0 + 2 * p + u : t1 - 1;
          t[u] = real ? t[u] : 0;
          const uint8_t* cp = vb0 + t[u] * vbs2 + QD * qr * SB / 8;
          load_words<CW>(R.vc[u], real || (L1 > 0 && rawok) ? cp : (const uint8_t*)safe16);
        }
        const anna_mi_view &vs = a.value_scales, &vz = a.value_zeros;
        const uint16_t* sp0 = (const uint16_t*)vs.ptr + b * vs.s0 + kvh * vs.s1;
        const uint16_t* zp0 = (const uint16_t*)vz.ptr + b * vz.s0 + kvh * vz.s1;
        const bool any = L1 > 0;
#pragma unroll
        for (int i = 0; i < NSP; ++i) {
          const int64_t g = (QD * qr + 32 * i) / a.value_group_size;
          const uint16_t* sp = any ? sp0 + g * vs.s3 : safe16;
          const uint16_t* zp = any ? zp0 + g * vz.s3 : safe16;
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            R.vsc[i][u] = sp[any ? t[u] * vs.s2 : 0];
            R.vzr[i][u] = zp[any ? t[u] * vz.s2 : 0];
          }
        }
      }
    }
    // key rows of tokens tt0 + r and tt0 + 16 + r (clamped into the range; masked below)
    const int64_t ta = tt0 + r < t1 ? tt0 + r : t1 - 1, tb = tt0 + 16 + r < t1 ? tt0 + 16 + r : t1 - 1;
    if constexpr (PK) {
      // (the key code words are loaded above) the norms of the lane's score rows (tokens
      // 4 kq + i, 16 + 4 kq + i, clamped into the range: the last tile may pass the segment)
      const uint16_t* kn0 = (const uint16_t*)a.key_norms.ptr + b * a.key_norms.s0 + kvh * a.key_norms.s1;
      if (tt0 + MF_TILE <= t1 && a.key_norms.s2 == 1 && (uintptr_t)kn0 % 8 == 0) {
        // a whole tile of contiguous norms: the lane's two runs of four as two 8-byte loads
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const uint2 w = *(const uint2*)(kn0 + tt0 + 16 * hh + 4 * kq);
          R.kn[4 * hh] = w.x & 0xFFFFu;
          R.kn[4 * hh + 1] = w.x >> 16;
          R.kn[4 * hh + 2] = w.y & 0xFFFFu;
          R.kn[4 * hh + 3] = w.y >> 16;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int64_t t = tt0 + 16 * (i >> 2) + 4 * kq + (i & 3);
          R.kn[i] = kn0[(t < t1 ? t : t1 - 1) * a.key_norms.s2];
        }
      }
    } else {
      const uint16_t* ra = key_row(ta);
      const uint16_t* rb = key_row(tb);
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        R.ka[st] = *(const u32x4*)(ra + 32 * st + 8 * kq);
        R.kb[st] = *(const u32x4*)(rb + 32 * st + 8 * kq);
      }
    }
  };

  // fixed NT: every tile's loads are issued here, one register set per tile; otherwise two sets
  // take turns (tile n + 2's loads go into tile n's set after its scores)
  constexpr int NB = NT > 0 ? NT : 2;
  Regs buf[NB];
  // query fragments: lane (head r, kq) of step st holds q[head][32 st + 8 kq .. + 7] (0 for
  // r >= G); they go through registers to LDS once and are read back per tile
  u32x4 qf[NST];
  {
    const bool qvec = a.query.s3 == 1 && (uintptr_t)a.query.ptr % 16 == 0 && a.query.s0 % 8 == 0 && a.query.s1 % 8 == 0;
    // Packed ranges with the randomized Hadamard rotation (16-byte aligned signs: the host then
    // launches no rotation): q' = H diag(s) q / sqrt(D) here, in the operation order of the
    // rotation kernel (signs, butterflies over index bits 0, 1, .. in ascending order, the scale),
    // so the same bits.  Lane (head r, kq) holds dims QD kq .. + QD - 1: index bits below
    // log2(QD) pair up inside the lane, the top two across lanes 16 and 32 apart.
    const bool rot_here = KSB > 0 && a.rotation_signs && (uintptr_t)a.rotation_signs % 16 == 0;
    u32x4 qrot[NST];
    if constexpr (KSB > 0) {
      if (packed_rng && rot_here) {
        float v[1][QD];
        const int64_t qb = b * a.query.s0 + (kvh * G + (r < G ? r : 0)) * a.query.s1;
        const uint16_t* q = (const uint16_t*)a.query.ptr;
#pragma unroll
        for (int j = 0; j < QD; j += 8) {
          const int64_t d0 = QD * kq + j;
          const float4 s0 = *(const float4*)(a.rotation_signs + d0), s1 = *(const float4*)(a.rotation_signs + d0 + 4);
          const float sg[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
          uint16_t h[8];
          if (qvec) {
            const u32x4 w = *(const u32x4*)(q + qb + d0);
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = q[qb + (d0 + e) * a.query.s3];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e)
            v[0][j + e] = (DT == ANNA_MI_BF16 ? bf16_bits_to_f32(h[e]) : f16_bits_to_f32(h[e])) * sg[e];
        }
#pragma unroll
        for (int hb = 1; hb < QD; hb <<= 1) {
#pragma unroll
          for (int e = 0; e < QD; ++e) {
            if ((e & hb) == 0) {
              const float x = v[0][e], y = v[0][e + hb];
              v[0][e] = x + y;
              v[0][e + hb] = x - y;
            }
          }
        }
        fwht_lane_stage<16>(v, (lane & 16) != 0);
        fwht_lane_stage<32>(v, (lane & 32) != 0);
        const float inv = tq_inv_sqrt(D);
#pragma unroll
        for (int st = 0; st < NST; ++st) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            qrot[st][e] = pack2_16<ANNA_MI_F16>(v[0][8 * st + 2 * e] * inv, v[0][8 * st + 2 * e + 1] * inv);
        }
      }
    }
    const int64_t qb = b * a.query.s0 + (kvh * G + (r < G ? r : 0)) * a.query.s1;
    const uint16_t* q = (const uint16_t*)a.query.ptr;
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      if (KSB > 0 && packed_rng && rot_here) {
        qf[st] = qrot[st];
      } else if (KSB > 0 && packed_rng) {
        // q' = R q (fp32, written by the rotation launch) as fp16, dims QD kq + 8 st .. + 7
        const float* qrow = a.query_rot + (b * a.q_heads + kvh * G + (r < G ? r : 0)) * D + QD * kq + 8 * st;
        const float4 lo = *(const float4*)qrow, hi = *(const float4*)(qrow + 4);
        qf[st] = u32x4{pack2_16<ANNA_MI_F16>(lo.x, lo.y), pack2_16<ANNA_MI_F16>(lo.z, lo.w),
                       pack2_16<ANNA_MI_F16>(hi.x, hi.y), pack2_16<ANNA_MI_F16>(hi.z, hi.w)};
      } else if (qvec) {
        qf[st] = *(const u32x4*)(q + qb + 32 * st + 8 * kq);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t d = 32 * st + 8 * kq + 2 * e;
          qf[st][e] = (uint32_t)q[qb + d * a.query.s3] | ((uint32_t)q[qb + (d + 1) * a.query.s3] << 16);
        }
      }
    }
  }

  const float scale2 = a.scaling * LOG2E;
  float m_run = -INFINITY, l_run = 0.f;  // of head r (lane column), replicated over kq
  f32x4 acc[NDT];
#pragma unroll
  for (int j = 0; j < NDT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto process = [&](Regs& R, int n, auto pk) __attribute__((always_inline)) {
    constexpr bool PK = KSB > 0 && decltype(pk)::value;
    const int64_t tt0 = t0 + (int64_t)MF_TILE * n;
    // ---- V of the tile into LDS, transposed.  With per-row lengths the slots past a row's length
    // (stale memory, possibly not finite) stage as zeros: their probabilities are 0, but 0 * NaN
    // would not be.
    const bool keep0 = !SEQ || valid(tt0 + 2 * p), keep1 = !SEQ || valid(tt0 + 2 * p + 1);
    // (with TQ-MSE keys exactly the packed ranges' tiles are raw: the host guarantees raw-ready
    // values, and window tiles never are)
    if (KSB > 0 ? PK : raw_tile(tt0)) {
      if constexpr (VF == ANNA_MI_VALUES_MINMAX) {
        constexpr uint32_t mask = (1u << SB) - 1u;
#pragma unroll
        for (int c = 0; c < QD / 8; ++c) {
          const int i = QD >= 32 ? c / 4 : 0;
          float v[2][8];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const uint16_t sh = (uint16_t)R.vsc[i][u], zh = (uint16_t)R.vzr[i][u];
            float sc = DT == ANNA_MI_BF16 ? bf16_bits_to_f32(sh) : f16_bits_to_f32(sh);
            float zc = DT == ANNA_MI_BF16 ? bf16_bits_to_f32(zh) : f16_bits_to_f32(zh);
            if constexpr (SEQ) {
              // a slot past the row's length stages as q * 0 + 0 = 0 (its scale and zero may be
              // stale, not finite; the codes are small integers)
              const bool k = u ? keep1 : keep0;
              sc = k ? sc : 0.f;
              zc = k ? zc : 0.f;
            }
            if constexpr (SB == 4) {
              // one word holds the 8 codes: split into the even and odd codes' bytes, each then
              // one byte-to-float conversion
              const uint32_t w = R.vc[u][c], lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                v[u][2 * e] = (float)((lo >> (8 * e)) & 0xFFu) * sc + zc;
                v[u][2 * e + 1] = (float)((hi >> (8 * e)) & 0xFFu) * sc + zc;
              }
            } else if constexpr (SB == 2) {
              // one word holds the codes of chunks 2 (c / 2) and + 1: code j sits in byte j / 4 of
              // plane j % 4 (planes = the word's 2-bit fields masked apart), one byte-to-float
              // conversion each; this chunk's codes are bytes 2 (c % 2) and + 1
              const uint32_t w = R.vc[u][c >> 1];
              const int hb = 2 * (c & 1);
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const uint32_t plane = (w >> (2 * (e & 3))) & 0x03030303u;
                v[u][e] = (float)((plane >> (8 * (hb + (e >> 2)))) & 0xFFu) * sc + zc;
              }
            } else {
              // codes of dims 8c .. 8c + 7 of the lane's quarter: 8 SB bits from bit 8 SB c
              const uint32_t w = R.vc[u][(8 * SB * c) / 32] >> ((8 * SB * c) % 32);
#pragma unroll
              for (int e = 0; e < 8; ++e) v[u][e] = (float)((w >> (SB * e)) & mask) * sc + zc;
            }
          }
          const int d0 = QD * qr + 8 * c;
#pragma unroll
          for (int e = 0; e < 8; ++e) vw[(d0 + e) * (MF_VT / 2) + p] = pack2_16<DT>(v[0][e], v[1][e]);
        }
      }
    } else {
      // lane (p, quarter) takes tokens 2p, 2p + 1 and dims [QD quarter, QD quarter + QD); a
      // 32-bit LDS word holds one dim of both tokens
      int64_t tu[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) tu[u] = tt0 + 2 * p + u < t1 ? tt0 + 2 * p + u : t1 - 1;
      const bool dense0 = VF == ANNA_MI_VALUES_DENSE || tu[0] >= L1, dense1 = VF == ANNA_MI_VALUES_DENSE || tu[1] >= L1;
      if (dense0 && dense1) {
        // 16-bit rows (window tokens, or dense values): interleave the two tokens' halves
        const uint16_t* row[2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
          row[u] = (tu[u] >= L1 ? rval0 + (tu[u] - L1) * rvs2 : (const uint16_t*)(vb0 + tu[u] * vbs2)) + QD * qr;
#pragma unroll 2
        for (int c = 0; c < QD / 8; ++c) {
          u32x4 w0 = *(const u32x4*)(row[0] + 8 * c), w1 = *(const u32x4*)(row[1] + 8 * c);
          if constexpr (SEQ) {
            w0 = keep0 ? w0 : u32x4{0u, 0u, 0u, 0u};
            w1 = keep1 ? w1 : u32x4{0u, 0u, 0u, 0u};
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int d = QD * qr + 8 * c + 2 * e;
            vw[d * (MF_VT / 2) + p] = __builtin_amdgcn_perm(w1[e], w0[e], 0x05040100u);
            vw[(d + 1) * (MF_VT / 2) + p] = __builtin_amdgcn_perm(w1[e], w0[e], 0x07060302u);
          }
        }
      } else {
        // at least one packed token: dequantize q * scale + zero per 8 dims (one group)
        constexpr int sb = SB == 2 ? 2 : 4;
        constexpr uint32_t mask = (1u << sb) - 1u;
#pragma unroll 2
        for (int c = 0; c < QD / 8; ++c) {
          const int d0 = QD * qr + 8 * c;
          float v[2][8];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int64_t t = tu[u];
            if (t >= L1) {
              const uint16_t* row = rval0 + (t - L1) * rvs2 + d0;
              const u32x4 w = *(const u32x4*)row;
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                v[u][e] = DT == ANNA_MI_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
              }
            } else {
              const uint8_t* codes = vb0 + t * vbs2;
              const int64_t g = d0 / a.value_group_size;
              const float sc = ldt<DT>(a.value_scales.ptr, b * a.value_scales.s0 + kvh * a.value_scales.s1 +
                                                                 t * a.value_scales.s2 + g * a.value_scales.s3);
              const float zc = ldt<DT>(a.value_zeros.ptr, b * a.value_zeros.s0 + kvh * a.value_zeros.s1 +
                                                                t * a.value_zeros.s2 + g * a.value_zeros.s3);
              const uint32_t bits = sb == 2 ? (uint32_t)*(const uint16_t*)(codes + d0 / 4) : *(const uint32_t*)(codes + d0 / 2);
#pragma unroll
              for (int e = 0; e < 8; ++e) v[u][e] = (float)((bits >> (sb * e)) & mask) * sc + zc;
            }
          }
#pragma unroll
          for (int e = 0; e < 8; ++e)
            vw[(d0 + e) * (MF_VT / 2) + p] = pack2_16<DT>(keep0 ? v[0][e] : 0.f, keep1 ? v[1][e] : 0.f);
        }
      }
    }
    // ---- scores: st0 rows = tokens tt0 + 0..15, st1 rows = tt0 + 16..31; columns = heads
    f32x4 st0 = {0.f, 0.f, 0.f, 0.f}, st1 = st0;
    float kscale[8];
    if constexpr (PK) {
      // the codes of dims QD kq + 8 st .. + 7 through the table
      auto frag = [&](const uint32_t (&kc)[KCW], int st) -> u32x4 {
        if constexpr (KSB == 4) {
          const uint32_t w = kc[st];
          return u32x4{s_klut[w & 0xFFu], s_klut[(w >> 8) & 0xFFu], s_klut[(w >> 16) & 0xFFu], s_klut[w >> 24]};
        } else {
          const uint32_t w = kc[st >> 1] >> (16 * (st & 1));
          const uint2 lo = ((const uint2*)s_klut)[w & 0xFFu], hi = ((const uint2*)s_klut)[(w >> 8) & 0xFFu];
          return u32x4{lo.x, lo.y, hi.x, hi.y};
        }
      };
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        const u32x4 qs = s_qf[st][lane];
        st0 = mfma16<ANNA_MI_F16>(frag(R.kc[0], st), qs, st0);
        st1 = mfma16<ANNA_MI_F16>(frag(R.kc[1], st), qs, st1);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) kscale[i] = f16_bits_to_f32((uint16_t)R.kn[i]) * scale2;
    } else {
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        const u32x4 qs = s_qf[st][lane];
        st0 = mfma16<DT>(R.ka[st], qs, st0);
        st1 = mfma16<DT>(R.kb[st], qs, st1);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) kscale[i] = scale2;
    }
    // this buffer is free again: tile n + 2 goes in flight
    if (NT == 0 && n + 2 < ntiles) issue(R, n + 2, pk);
    float s[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = valid(tt0 + 4 * kq + i) ? st0[i] * kscale[i] : -INFINITY;
      s[4 + i] = valid(tt0 + 16 + 4 * kq + i) ? st1[i] * kscale[4 + i] : -INFINITY;
    }
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i]);
    mx = fmaxf(mx, lane_xor16(mx));
    mx = fmaxf(mx, lane_xor32(mx));
    if (__any(mx > m_run + LAZY)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 while m_run is -inf
      l_run *= alpha;
      // acc[j][i] belongs to head 4 kq + i: its factor comes from lane column 4 kq + i
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, (lane & ~15) | (4 * kq + i), 64);
#pragma unroll
      for (int j = 0; j < NDT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] *= al[i];
      m_run = m_new;
    }
    u32x4 pf;
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      float p0 = __builtin_amdgcn_exp2f(s[i] - m_run), p1 = __builtin_amdgcn_exp2f(s[i + 1] - m_run);
      float p2 = __builtin_amdgcn_exp2f(s[4 + i] - m_run), p3 = __builtin_amdgcn_exp2f(s[5 + i] - m_run);
      if constexpr (SEQ) {  // a tile can be all masked while m_run is still -inf
        p0 = s[i] == -INFINITY ? 0.f : p0;
        p1 = s[i + 1] == -INFINITY ? 0.f : p1;
        p2 = s[4 + i] == -INFINITY ? 0.f : p2;
        p3 = s[5 + i] == -INFINITY ? 0.f : p3;
      }
      l_run += (p0 + p1) + (p2 + p3);
      pf[i >> 1] = pack2_16<DT>(p0, p1);
      pf[2 + (i >> 1)] = pack2_16<DT>(p2, p3);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the V tile is in LDS
    // ---- O[heads x dims] += P[heads x tokens] V[tokens x dims], one MFMA per 16 dims
#pragma unroll
    for (int j = 0; j < NDT; ++j) {
      const uint16_t* col = s_vt + (16 * j + r) * MF_VT;
      const uint2 lo = *(const uint2*)(col + 4 * kq), hi = *(const uint2*)(col + 16 + 4 * kq);
      const u32x4 vf = {lo.x, lo.y, hi.x, hi.y};
      acc[j] = mfma16<DT>(pf, vf, acc[j]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next tile's writes
  };

  // The tile loads (after the query's: a wait for those never waits for the tiles), the query
  // fragments into LDS, the tile loop -- one instance per tag, chosen once, so that the tile
  // registers are written from one place in each (written from two branches, the compiler kept
  // them in scratch memory).
  auto run = [&](auto pk) __attribute__((always_inline)) {
    if (live) {
      if constexpr (NT > 0) {
#pragma unroll
        for (int n = 0; n < NT; ++n) issue(buf[n], n, pk);
      } else {
        issue(buf[0], 0, pk);
        if (ntiles > 1) issue(buf[1], 1, pk);
      }
    }
    // the first use of a loaded value (the padding heads' zeros included) stays below every load:
    // a use above them made the compiler wait for all loads issued so far before issuing the rest
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < NST; ++st) s_qf[st][lane] = r < G ? qf[st] : u32x4{0u, 0u, 0u, 0u};
    if (live) {
      if constexpr (NT > 0) {
#pragma unroll
        for (int n = 0; n < NT; ++n) process(buf[n], n, pk);
      } else {
        for (int n = 0; n < ntiles; n += 2) {
          process(buf[0], n, pk);
          if (n + 1 < ntiles) process(buf[1], n + 1, pk);
        }
      }
    }
  };
  if (KSB > 0 && packed_rng) run(PkT{});
  else run(PkF{});

  // ---- the range's partial: stats of head r from lanes (r, kq = 0), values [b, hq, blk, d] from
  // the accumulators (lane (dim 16 j + r, kq) holds heads 4 kq + i)
  l_run += lane_xor16(l_run);
  l_run += lane_xor32(l_run);
  if (kq == 0 && r < G) {
    const anna_mi_view& ps = a.partial_stats;
    const int64_t base = b * ps.s0 + (kvh * G + r) * ps.s1 + blk * ps.s2;
    ((float*)ps.ptr)[base] = m_run * 0.6931471805599453f;  // back to natural-log units
    ((float*)ps.ptr)[base + ps.s3] = l_run;
  }
  // a range with no valid token (per-row lengths) leaves its values unwritten: the merges weigh
  // a block with denominator 0 by 0 and never read its values into a sum
  if (!live) return;
  const anna_mi_view& pv = a.partial_values;
  float* out = (float*)pv.ptr + b * pv.s0 + blk * pv.s2 + r * pv.s3;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * kq + i;
    if (h < G) {
      float* oh = out + (kvh * G + h) * pv.s1;
#pragma unroll
      for (int j = 0; j < NDT; ++j) __builtin_nontemporal_store(acc[j][i], oh + 16 * j * pv.s3);  // read once, by the merge
    }
  }
}

Split make_split(const anna_mi_decode_args& a) {
  Split sp{};
  const int64_t bs = a.block_size < 16 ? 16 : a.block_size;
  const int64_t L = a.len1 + a.len2;
  sp.aligned = a.value_format == ANNA_MI_VALUES_TQ_MSE || a.key_format == ANNA_MI_KEYS_TQ_MSE;
  if (sp.aligned) {
    sp.eb = a.len1 > 0 ? (bs < a.len1 ? bs : a.len1) : 1;
    sp.nb1 = a.len1 > 0 ? (a.len1 + sp.eb - 1) / sp.eb : 0;
    sp.eb2 = a.len2 > 0 ? (bs < a.len2 ? bs : a.len2) : 1;
  } else {
    sp.eb = bs < L ? bs : L;
    sp.nb1 = 0;
    sp.eb2 = 1;
  }
  return sp;
}

int64_t total_blocks(const anna_mi_decode_args& a, const Split& sp) {
  if (sp.aligned) return sp.nb1 + (a.len2 > 0 ? (a.len2 + sp.eb2 - 1) / sp.eb2 : 0);
  const int64_t L = a.len1 + a.len2;
  return (L + sp.eb - 1) / sp.eb;
}


// The MFMA split kernel takes 16-bit activations, dense or TQ-MSE keys, dense or min/max values
// and aligned rows (the layouts of the reference's caches and of TurboQuantRowsCache), with or
// without per-row lengths; anything else runs on the VALU kernel.
bool mfma_path_ok(const anna_mi_decode_args& a, const Split& sp) {
  if (a.dtype == ANNA_MI_F32) return false;
  if (a.value_format != ANNA_MI_VALUES_DENSE && a.value_format != ANNA_MI_VALUES_MINMAX) return false;
  if (a.head_dim != 64 && a.head_dim != 128 && a.head_dim != 256) return false;
  if (a.q_heads / a.kv_heads > 16) return false;
  const bool tqk = a.key_format == ANNA_MI_KEYS_TQ_MSE;
  if (!tqk && (a.key_format != ANNA_MI_KEYS_DENSE || sp.aligned)) return false;
  if (tqk && a.value_format != ANNA_MI_VALUES_MINMAX) return false;  // the forms instantiated
  auto rows16 = [](const anna_mi_view& v) {  // 8 x 16-bit elements per aligned 16-byte load
    return v.s3 == 1 && (uintptr_t)v.ptr % 16 == 0 && v.s0 % 8 == 0 && v.s1 % 8 == 0 && v.s2 % 8 == 0;
  };
  if (a.len1 > 0 && tqk) {
    // code fields of 2 or 4 bits (3-bit codes take 4); the lane's D / 4 dims of a token in one
    // aligned load of up to 16 bytes; the rotated query rows 16-byte aligned
    if (a.key_bits < 2 || a.key_bits > 4 || !a.query_rot || !a.key_centroids || (uintptr_t)a.query_rot % 16) return false;
    const int64_t ksb = a.key_bits == 2 ? 2 : 4, al = std::min<int64_t>(a.head_dim / 4 * ksb / 8, 16);
    const anna_mi_view& k = a.key;
    if (k.s3 != 1 || (uintptr_t)k.ptr % al || k.s0 % al || k.s1 % al || k.s2 % al) return false;
    // the packed ranges address a (batch, KV head) slice of the codes, scales and zeros with 32-bit
    // byte offsets, and tokens with 32-bit indices
    auto slice31 = [&](const anna_mi_view& v, int64_t esz, int64_t groups) {
      return v.s2 >= 0 && v.s3 >= 0 && (a.len1 * v.s2 + groups * v.s3 + a.head_dim) * esz < (1ll << 31);
    };
    const int64_t ng = a.value_group_size > 0 ? a.head_dim / a.value_group_size + 1 : 1;
    if (a.len1 + a.len2 >= (1ll << 31) || !slice31(k, 1, 0) || !slice31(a.value, 1, 0) ||
        !slice31(a.value_scales, 2, ng) || !slice31(a.value_zeros, 2, ng))
      return false;
    // and stages the packed values from raw codes (whole 32-dim scale groups, the lane's codes of a
    // token one aligned vector load), which the kernel then takes as given
    const int64_t vsb = a.value_bits == 2 ? 2 : 4, vca = std::min<int64_t>((a.head_dim / 4 * vsb / 8 + 3) / 4 * 4, 16);
    const anna_mi_view& v = a.value;
    if (a.value_group_size % 32 != 0 || v.s3 != 1 || (uintptr_t)v.ptr % vca || v.s0 % vca || v.s1 % vca || v.s2 % vca)
      return false;
  } else if (a.len1 > 0) {
    if (!rows16(a.key)) return false;
  }
  if (a.len1 > 0) {
    if (a.value_format == ANNA_MI_VALUES_DENSE) {
      if (!rows16(a.value)) return false;
    } else {
      const int64_t al = a.value_bits == 2 ? 2 : 4;  // the 8 codes of a group chunk in one load
      const anna_mi_view& v = a.value;
      if (v.s3 != 1 || (uintptr_t)v.ptr % al || v.s0 % al || v.s1 % al || v.s2 % al) return false;
      if (a.value_group_size % 8 != 0) return false;
    }
  }
  if (a.len2 > 0 && (!rows16(a.residual_key) || !rows16(a.residual_value))) return false;
  return true;
}

// Tokens per wave of the MFMA split kernel: whole tiles, about MF_WAVES_TARGET waves over all
// (batch, KV head) rows, and no more ranges per row than the caller's workspace holds.  With
// TQ-MSE keys the ranges are aligned to the segments (mfma_ranges counts both).
int64_t mfma_ranges(const anna_mi_decode_args& a, int64_t range, int64_t* nr1) {
  const bool aligned = a.key_format == ANNA_MI_KEYS_TQ_MSE;
  const int64_t L = a.len1 + a.len2;
  *nr1 = aligned ? (a.len1 + range - 1) / range : 0;
  return aligned ? *nr1 + (a.len2 + range - 1) / range : (L + range - 1) / range;
}

int64_t mfma_range(const anna_mi_decode_args& a) {
  const int64_t L = a.len1 + a.len2;
  const int64_t tiles = a.batch * a.kv_heads * ((L + MF_TILE - 1) / MF_TILE);
  // TQ-MSE keys at head_dim <= 128 run two waves per SIMD: eight per CU (TurboQuantRowsCache
  // D = 128: 26.7 -> 25.0 us against 1536 waves; 2560 no better); at 256 one: four per CU (D = 256:
  // 46.1 -> 45.1 us; 768 or 2048 waves 50.2 / 53.9)
  const bool tqk = a.key_format == ANNA_MI_KEYS_TQ_MSE;
  const int64_t wt = tqk ? (a.head_dim <= 128 ? MF_WAVES_TQ2 : MF_WAVES_TQ1) : MF_WAVES_TARGET;
  int64_t range = (tiles + wt - 1) / wt * MF_TILE;
  if (range < MF_TILE) range = MF_TILE;
  int64_t nr1 = 0;
  while (mfma_ranges(a, range, &nr1) > a.partial_capacity && range < L) range += MF_TILE;
  return range;
}

void launch_split_mfma(const anna_mi_decode_args& a, int64_t range, int64_t nranges, int64_t nr1, hipStream_t st) {
  const dim3 grid((unsigned)nranges, (unsigned)a.kv_heads, (unsigned)a.batch), blk(64);
  const int64_t nt = range / MF_TILE;
  const bool seq = a.seq_lengths != nullptr, tqk = a.key_format == ANNA_MI_KEYS_TQ_MSE;
  auto go = [&](auto dt_tag, auto vf_tag, auto sb_tag, auto ksb_tag, auto seq_tag) {
    constexpr int DT = decltype(dt_tag)::value, VF = decltype(vf_tag)::value, SB = decltype(sb_tag)::value;
    constexpr int KSB = decltype(ksb_tag)::value;
    constexpr bool SEQ = decltype(seq_tag)::value;
    auto by_nt = [&](auto d_tag) {
      constexpr int D = decltype(d_tag)::value;
      // per-row lengths or TQ-MSE keys: the runtime tile loop only (fewer instantiations)
      const int64_t n = KSB > 0 || SEQ ? 0 : nt;
      switch (n) {
        case 1: hipLaunchKernelGGL((decode_split_mfma_kernel<DT, VF, SB, D, 1, 0, false>), grid, blk, 0, st, a, range, nr1); break;
        case 2: hipLaunchKernelGGL((decode_split_mfma_kernel<DT, VF, SB, D, 2, 0, false>), grid, blk, 0, st, a, range, nr1); break;
        case 3: hipLaunchKernelGGL((decode_split_mfma_kernel<DT, VF, SB, D, 3, 0, false>), grid, blk, 0, st, a, range, nr1); break;
        case 4: hipLaunchKernelGGL((decode_split_mfma_kernel<DT, VF, SB, D, 4, 0, false>), grid, blk, 0, st, a, range, nr1); break;
        default: hipLaunchKernelGGL((decode_split_mfma_kernel<DT, VF, SB, D, 0, KSB, SEQ>), grid, blk, 0, st, a, range, nr1); break;
      }
    };
    switch (a.head_dim) {
      case 64: by_nt(std::integral_constant<int, 64>{}); break;
      case 128: by_nt(std::integral_constant<int, 128>{}); break;
      default: by_nt(std::integral_constant<int, 256>{}); break;
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S2 = std::integral_constant<int, 2>;
  using S4 = std::integral_constant<int, 4>;
  using BF = std::integral_constant<int, ANNA_MI_BF16>;
  using HF = std::integral_constant<int, ANNA_MI_F16>;
  using VD = std::integral_constant<int, ANNA_MI_VALUES_DENSE>;
  using VM = std::integral_constant<int, ANNA_MI_VALUES_MINMAX>;
  using Y = std::integral_constant<bool, true>;
  using N = std::integral_constant<bool, false>;
  const bool dense = a.value_format == ANNA_MI_VALUES_DENSE, two = a.value_bits == 2;
  auto go_k = [&](auto dt, auto vf, auto sb) {
    if (!tqk) {
      seq ? go(dt, vf, sb, S0{}, Y{}) : go(dt, vf, sb, S0{}, N{});
    } else if constexpr (decltype(vf)::value == ANNA_MI_VALUES_MINMAX) {
      // TQ-MSE keys come with min/max values (TurboQuantRowsCache, the row API)
      if (a.key_bits == 2) seq ? go(dt, vf, sb, S2{}, Y{}) : go(dt, vf, sb, S2{}, N{});
      else seq ? go(dt, vf, sb, S4{}, Y{}) : go(dt, vf, sb, S4{}, N{});
    }
  };
  if (a.dtype == ANNA_MI_BF16) {
    if (dense) go_k(BF{}, VD{}, S0{});
    else if (two) go_k(BF{}, VM{}, S2{});
    else go_k(BF{}, VM{}, S4{});
  } else {
    if (dense) go_k(HF{}, VD{}, S0{});
    else if (two) go_k(HF{}, VM{}, S2{});
    else go_k(HF{}, VM{}, S4{});
  }
}

template <int KF, int VF, int DT>
void launch_split_dt(const anna_mi_decode_args& a, const Split& sp, int64_t nblk, hipStream_t st) {
  dim3 grid((unsigned)nblk, (unsigned)a.kv_heads, (unsigned)a.batch);
  const int64_t G = a.q_heads / a.kv_heads;
  const size_t lds = (size_t)G * a.head_dim * 4;
  const dim3 blk(64 * DEC_WAVES);
#define ANNA_SPLIT(DPL, GM) hipLaunchKernelGGL((decode_split_kernel<KF, VF, DPL, GM, DT>), grid, blk, lds, st, a, sp)
  const bool small = G <= 8;
  switch (a.head_dim) {
    case 64: if (small) ANNA_SPLIT(1, 8); else ANNA_SPLIT(1, 16); break;
    case 128: if (small) ANNA_SPLIT(2, 8); else ANNA_SPLIT(2, 16); break;
    case 256: if (small) ANNA_SPLIT(4, 8); else ANNA_SPLIT(4, 16); break;
    default: ANNA_SPLIT(8, 8); break;
  }
#undef ANNA_SPLIT
}

template <int KF, int VF>
void launch_split(const anna_mi_decode_args& a, const Split& sp, int64_t nblk, hipStream_t st) {
  if (a.dtype == ANNA_MI_BF16) launch_split_dt<KF, VF, ANNA_MI_BF16>(a, sp, nblk, st);
  else if (a.dtype == ANNA_MI_F16) launch_split_dt<KF, VF, ANNA_MI_F16>(a, sp, nblk, st);
  else launch_split_dt<KF, VF, ANNA_MI_F32>(a, sp, nblk, st);
}

}  // namespace
}  // namespace anna

using namespace anna;

extern "C" int64_t anna_mi_sizeof_decode_args(void) { return (int64_t)sizeof(anna_mi_decode_args); }

extern "C" int64_t anna_mi_decode_num_blocks(const anna_mi_decode_args* a) {
  if (!a || a->len1 + a->len2 <= 0) return 0;
  return total_blocks(*a, make_split(*a));
}

static int gqa_decode_splitkv_impl(const anna_mi_decode_args& a, void* stream) {
  ANNA_CHECK(valid_dtype(a.dtype), "anna_mi_gqa_decode_splitkv: bad dtype code");
  ANNA_CHECK(a.batch > 0 && a.q_heads > 0 && a.kv_heads > 0, "anna_mi_gqa_decode_splitkv: empty batch or heads");
  ANNA_CHECK(a.q_heads % a.kv_heads == 0, "query heads must be divisible by kv_heads");
  ANNA_CHECK(a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256 || a.head_dim == 512,
             "anna_mi_gqa_decode_splitkv: head_dim must be 64, 128, 256 or 512 (got %lld)", (long long)a.head_dim);
  const int64_t G = a.q_heads / a.kv_heads;
  const int64_t gmax = a.head_dim == 512 ? 8 : 16;
  ANNA_CHECK(G <= gmax, "anna_mi_gqa_decode_splitkv: %lld query heads per KV head exceed %lld", (long long)G, (long long)gmax);
  ANNA_CHECK(a.len1 >= 0 && a.len2 >= 0 && a.len1 + a.len2 >= 1, "key_len must be positive");
  ANNA_CHECK(a.block_size >= 16, "block_size must be at least 16");
  ANNA_CHECK(a.key_format == ANNA_MI_KEYS_DENSE || a.key_format == ANNA_MI_KEYS_TQ_MSE, "bad key_format");
  ANNA_CHECK(a.value_format >= ANNA_MI_VALUES_DENSE && a.value_format <= ANNA_MI_VALUES_TQ_MSE, "bad value_format");
  ANNA_CHECK(a.query.ptr && a.out.ptr && a.partial_stats.ptr && a.partial_values.ptr, "null query/out/workspace");
  if (a.len1 > 0) ANNA_CHECK(a.key.ptr && a.value.ptr, "null key/value");
  if (a.len2 > 0) ANNA_CHECK(a.residual_key.ptr && a.residual_value.ptr, "null residual key/value");
  if (a.value_format == ANNA_MI_VALUES_MINMAX && a.len1 > 0) {
    ANNA_CHECK(a.value_bits == 2 || a.value_bits == 3 || a.value_bits == 4, "TurboQuant value_bits must be 2, 3, or 4");
    ANNA_CHECK(a.value_group_size > 0 && a.head_dim % a.value_group_size == 0,
               "TurboQuant value_group_size must evenly divide head_dim");
    ANNA_CHECK(a.value_scales.ptr && a.value_zeros.ptr, "null value scales/zeros");
  }
  if (a.key_format == ANNA_MI_KEYS_TQ_MSE && a.len1 > 0)
    ANNA_CHECK(a.key_norms.ptr && a.rotation_t && a.key_centroids && a.query_rot, "TQ-MSE keys need norms, rotation_t, centroids and query_rot");
  if (a.value_format == ANNA_MI_VALUES_TQ_MSE && a.len1 > 0)
    ANNA_CHECK(a.value_scales.ptr && a.rotation && a.value_centroids, "TQ-MSE values need norms, rotation and centroids");
  if (a.gate_layout != ANNA_MI_GATE_NONE) ANNA_CHECK(a.gate.ptr != nullptr, "null gate");
  for (const anna_mi_view* v : {&a.key, &a.value, &a.value_scales, &a.value_zeros, &a.residual_key, &a.residual_value})
    ANNA_CHECK(v->s3 >= 0 && v->s3 < ((int64_t)1 << 31) / a.head_dim,
               "anna_mi_gqa_decode_splitkv: innermost stride %lld too large", (long long)v->s3);
  Split sp = make_split(a);
  {
    const int64_t dpl = a.head_dim / 64, esz = a.dtype == ANNA_MI_F32 ? 4 : 2;
    const anna_mi_view& k = a.key;
    const bool kvec = a.key_format != ANNA_MI_KEYS_DENSE ||
                      (k.s3 == 1 && k.s0 % dpl == 0 && k.s1 % dpl == 0 && k.s2 % dpl == 0 &&
                       (uintptr_t)k.ptr % (uintptr_t)(dpl * esz) == 0);
    const bool svec = a.value_format != ANNA_MI_VALUES_MINMAX || a.value_group_size % dpl == 0;
    sp.vec = kvec && svec;
  }
  const int64_t nblk = total_blocks(a, sp);
  ANNA_CHECK(nblk <= a.partial_capacity, "partial_stats/partial_values capacity %lld is smaller than %lld blocks",
             (long long)a.partial_capacity, (long long)nblk);
  hipStream_t st = as_stream(stream);
  const bool kq = a.key_format == ANNA_MI_KEYS_TQ_MSE;
  int64_t nmerge = nblk;  // partials written by the split kernel
  int64_t mf_range = 0, mf_nr1 = 0, mf_n = 0;
  if (mfma_path_ok(a, sp)) {
    mf_range = mfma_range(a);
    mf_n = mfma_ranges(a, mf_range, &mf_nr1);
  }
  const bool use_mfma = mf_n > 0 && mf_n <= a.partial_capacity;  // (two aligned segments take two ranges at least)
  // the MFMA kernel rotates the query itself with 16-byte aligned Hadamard signs (the same
  // condition as in the kernel)
  const bool rot_in_split = use_mfma && kq && a.rotation_signs && (uintptr_t)a.rotation_signs % 16 == 0;
  if (kq && a.len1 > 0 && !rot_in_split) {
    const int64_t D = a.head_dim;
    if (a.rotation_signs && (D == 64 || D == 128 || D == 256 || D == 512 || D == 1024)) {
      const dim3 grid((unsigned)((a.batch * a.q_heads + 3) / 4));
      switch (D) {
        case 64: hipLaunchKernelGGL(decode_rotate_query_hadamard_kernel<1>, grid, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(decode_rotate_query_hadamard_kernel<2>, grid, dim3(256), 0, st, a); break;
        case 256: hipLaunchKernelGGL(decode_rotate_query_hadamard_kernel<4>, grid, dim3(256), 0, st, a); break;
        case 512: hipLaunchKernelGGL(decode_rotate_query_hadamard_kernel<8>, grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL(decode_rotate_query_hadamard_kernel<16>, grid, dim3(256), 0, st, a); break;
      }
      ANNA_LAUNCH_CHECK("decode_rotate_query_hadamard_kernel");
    } else {
      hipLaunchKernelGGL(decode_rotate_query_kernel, dim3((unsigned)a.q_heads, (unsigned)a.batch),
                         dim3((unsigned)a.head_dim), 0, st, a);
      ANNA_LAUNCH_CHECK("decode_rotate_query_kernel");
    }
  }
  if (use_mfma) {
    nmerge = mf_n;
    launch_split_mfma(a, mf_range, nmerge, mf_nr1, st);
  } else switch (a.value_format) {
    case ANNA_MI_VALUES_DENSE:
      kq ? launch_split<1, 0>(a, sp, nblk, st) : launch_split<0, 0>(a, sp, nblk, st);
      break;
    case ANNA_MI_VALUES_MINMAX:
      kq ? launch_split<1, 1>(a, sp, nblk, st) : launch_split<0, 1>(a, sp, nblk, st);
      break;
    default:
      kq ? launch_split<1, 2>(a, sp, nblk, st) : launch_split<0, 2>(a, sp, nblk, st);
      break;
  }
  ANNA_LAUNCH_CHECK("decode_split_kernel");
  const int64_t nrot = a.value_format == ANNA_MI_VALUES_TQ_MSE ? sp.nb1 : 0;
  if (nrot == 0 && nmerge <= MERGE_DIM_MAXBLK) {
    hipLaunchKernelGGL(decode_merge_dims_kernel, dim3((unsigned)(a.head_dim / 64), (unsigned)a.q_heads, (unsigned)a.batch),
                       dim3(64 * MERGE_DIM_WAVES), 0, st, a, nmerge);
    ANNA_LAUNCH_CHECK("decode_merge_dims_kernel");
  } else {
    hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)a.q_heads, (unsigned)a.batch), dim3(MERGE_THREADS),
                       (size_t)a.head_dim * 4, st, a, nmerge, nrot);
    ANNA_LAUNCH_CHECK("decode_merge_kernel");
  }
  return ANNA_MI_OK;
}

extern "C" int anna_mi_gqa_decode_splitkv(const anna_mi_decode_args* ap, void* stream) {
  ANNA_CHECK(ap != nullptr, "anna_mi_gqa_decode_splitkv: null args");
  return gqa_decode_splitkv_impl(*ap, stream);
}

// ------------------------------------------------------------------ allocation-free variant
//
// The workspace of anna_mi_gqa_decode_splitkv (partial stats, partial values and, with TQ-MSE
// keys, the rotated query) lives in one file-scope device array per GPU instead of caller
// tensors.  Every call on a GPU shares that GPU's array: calls that overlap on one GPU (two
// streams, two threads) race.  Nothing in it has to start at zero: the split kernel writes
// every partial the merge reads, and the rotation kernel every rotated query entry.
namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;  // 32 MiB per GPU
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once per device; the array's
// host-side name is not a device address).
int scratch_of_current_device(unsigned char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "anna_mi_gqa_decode_splitkv_noalloc: hipGetDevice");
  ANNA_CHECK(dev >= 0 && dev < kMaxDevices, "anna_mi_gqa_decode_splitkv_noalloc: device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail_hip(e, "anna_mi_gqa_decode_splitkv_noalloc: hipGetSymbolAddress(scratch)");
    ANNA_CHECK(p != nullptr, "anna_mi_gqa_decode_splitkv_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = (unsigned char*)p;
  }
  *out = g_scratch_ptr[dev];
  return ANNA_MI_OK;
}

}  // namespace

extern "C" int64_t anna_mi_gqa_decode_splitkv_noalloc_capacity(void) { return (int64_t)kNoAllocScratchBytes; }

extern "C" int anna_mi_gqa_decode_splitkv_noalloc(const anna_mi_decode_args* ap, void* stream) {
  ANNA_CHECK(ap != nullptr, "anna_mi_gqa_decode_splitkv_noalloc: null args");
  anna_mi_decode_args a = *ap;
  ANNA_CHECK(a.batch > 0 && a.q_heads > 0 && a.head_dim > 0 && a.len1 >= 0 && a.len2 >= 0 && a.len1 + a.len2 >= 1,
             "anna_mi_gqa_decode_splitkv_noalloc: empty batch, heads or keys");
  const int64_t nblk = total_blocks(a, make_split(a));
  const int64_t rows = a.batch * a.q_heads;
  const bool qrot = a.key_format == ANNA_MI_KEYS_TQ_MSE && a.len1 > 0;
  // [B][Hq][nblk][2] stats, [B][Hq][nblk][D] values, [B][Hq][D] rotated query (fp32, 256-byte aligned parts)
  auto up = [](int64_t n) { return (n + 63) / 64 * 64; };
  const int64_t n_stats = up(rows * nblk * 2), n_values = up(rows * nblk * a.head_dim);
  const int64_t n_qrot = qrot ? up(rows * a.head_dim) : 0;
  const int64_t need = (n_stats + n_values + n_qrot) * 4;
  ANNA_CHECK(need <= (int64_t)kNoAllocScratchBytes,
             "anna_mi_gqa_decode_splitkv_noalloc: workspace of %lld bytes (batch %lld, %lld heads, %lld blocks, head_dim "
             "%lld) exceeds the %lld-byte static scratch; use anna_mi_gqa_decode_splitkv with a caller workspace",
             (long long)need, (long long)a.batch, (long long)a.q_heads, (long long)nblk, (long long)a.head_dim,
             (long long)kNoAllocScratchBytes);
  unsigned char* base = nullptr;
  int rc = scratch_of_current_device(&base);
  if (rc != ANNA_MI_OK) return rc;
  float* f = (float*)base;
  a.partial_stats = anna_mi_view{f, a.q_heads * nblk * 2, nblk * 2, 2, 1};
  a.partial_values = anna_mi_view{f + n_stats, a.q_heads * nblk * a.head_dim, nblk * a.head_dim, a.head_dim, 1};
  a.partial_capacity = nblk;
  a.query_rot = qrot ? f + n_stats + n_values : nullptr;
  return gqa_decode_splitkv_impl(a, stream);
}
