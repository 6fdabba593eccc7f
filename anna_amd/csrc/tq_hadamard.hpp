// Randomized Hadamard rotation of TQ-MSE (power-of-two head_dim): y = R x with
// R = (1/sqrt(D)) H_D diag(s), H_D the Sylvester Hadamard matrix (H[i][j] = (-1)^popcount(i & j))
// and s a seeded sign vector.  One wave transforms one vector: lane l holds the E = D / 64
// consecutive elements l*E .. l*E + E - 1.
//
// The arithmetic order is fixed so that the CPU oracle reproduces every bit:
//   * signs are applied first (exact), then butterfly stages over index bits b = 0, 1, ...,
//     log2(D) - 1 in ascending order; a stage maps the pair (i, i | 2^b), bit b of i clear,
//     to (x_i + x_j, x_i - x_j); then every element is multiplied by fp32(1/sqrt(D));
//   * |x|^2 is, per lane, an fma chain over its E elements in ascending order starting from 0,
//     then an xor tree over lanes with masks 1, 2, 4, 8, 16, 32 (p_l <- p_l + p_{l ^ m});
//   * the norm is the correctly rounded fp32 sqrt of that sum; code_i counts the thresholds
//     t_j with y_i >= fl(t_j * norm).
#pragma once

#include "common.hpp"

namespace anna {

// Bits of the sign vector: s_i = -1 where bit (i % 64) of the (i / 64)-th splitmix64 output of
// the seed is set.
inline uint64_t tq_splitmix64(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline void tq_hadamard_signs(int64_t D, uint64_t seed, float* out) {
  uint64_t s = seed, w = 0;
  for (int64_t i = 0; i < D; ++i) {
    if (i % 64 == 0) w = tq_splitmix64(s);
    out[i] = ((w >> (i % 64)) & 1u) ? -1.0f : 1.0f;
  }
}

// n standard-normal values from the splitmix64 stream of `seed` by Box-Muller in fp64: each
// pair (u1, u2) of 53-bit uniforms in (0, 1) gives r cos(2 pi u2), r sin(2 pi u2) with
// r = sqrt(-2 ln u1).
inline void tq_gaussian(int64_t n, uint64_t seed, double* g) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; i += 2) {
    double u1 = ((double)(tq_splitmix64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    double u2 = ((double)(tq_splitmix64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    double r = __builtin_sqrt(-2.0 * __builtin_log(u1));
    g[i] = r * __builtin_cos(6.283185307179586 * u2);
    if (i + 1 < n) g[i + 1] = r * __builtin_sin(6.283185307179586 * u2);
  }
}

__host__ __device__ constexpr bool tq_is_pow2(int64_t d) { return d > 0 && (d & (d - 1)) == 0; }

// fp32(1/sqrt(D)) (exact for D a power of 4)
__host__ __device__ inline float tq_inv_sqrt(int64_t D) {
  int l = 0;
  while ((int64_t(1) << l) < D) ++l;
  if ((l & 1) == 0) return 1.0f / (float)(int64_t(1) << (l / 2));
  return (float)(1.0 / __builtin_sqrt((double)D));
}

// Value of lane (lane ^ M) for the wave's 64 lanes: LDS swizzles (quad-permute mode for M = 1,
// 2, bit mode inside 32-lane halves for 4, 8, 16) and a bpermute for 32.  They run on the LDS
// pipe, not the VALU (a DPP move would take a VALU slot per element; the transforms here are
// VALU-bound).  Exact copies, so the arithmetic around them is the same whichever exchange is
// used.
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
  if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x80B1));
  else if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x804E));
  else if constexpr (M < 32) return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (M << 10) | 0x1F));
  else return __shfl_xor(v, 32, 64);
}

// One butterfly stage across lanes: the lower lane of a pair keeps x_i + x_j, the upper one
// x_i - x_j.  Written as fma(v, +-1, partner): the product is exact and the one rounding is
// that of the add or subtract (signed zeros included: fma(x, -1, x) = +0 = x - x), so the
// result is bit-identical to the two-branch form at one instruction per element.
template <int M, int NV, int E>
__device__ __forceinline__ void fwht_lane_stage(float (&v)[NV][E], bool upper) {
  const float sg = upper ? -1.0f : 1.0f;
#pragma unroll
  for (int n = 0; n < NV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) v[n][e] = __builtin_fmaf(v[n][e], sg, xor_lane<M>(v[n][e]));
}

// In-place FWHT of NV vectors at once (independent chains), E elements of each per lane (stages
// as above, no scaling).
template <int NV, int E>
__device__ __forceinline__ void fwht_wave_n(float (&v)[NV][E]) {
  // stages inside a lane: index bits 0 .. log2(E) - 1
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int n = 0; n < NV; ++n)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if ((e & h) == 0) {
          const float a = v[n][e], c = v[n][e + h];
          v[n][e] = a + c;
          v[n][e + h] = a - c;
        }
      }
  }
  // stages across lanes: index bits log2(E) .. log2(E) + 5 = lane bits 0 .. 5
  const int lane = threadIdx.x & 63;
  fwht_lane_stage<1>(v, (lane & 1) != 0);
  fwht_lane_stage<2>(v, (lane & 2) != 0);
  fwht_lane_stage<4>(v, (lane & 4) != 0);
  fwht_lane_stage<8>(v, (lane & 8) != 0);
  fwht_lane_stage<16>(v, (lane & 16) != 0);
  fwht_lane_stage<32>(v, (lane & 32) != 0);
}

template <int E>
__device__ __forceinline__ void fwht_wave(float (&v)[E]) {
  float w[1][E];
#pragma unroll
  for (int e = 0; e < E; ++e) w[0][e] = v[e];
  fwht_wave_n<1, E>(w);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = w[0][e];
}

// |x|^2 of NV vectors in the fixed order above (every lane gets the totals).
template <int NV, int E>
__device__ __forceinline__ void sumsq_wave_n(const float (&x)[NV][E], float (&out)[NV]) {
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    float p = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) p = __builtin_fmaf(x[n][e], x[n][e], p);
    out[n] = p;
  }
#pragma unroll
  for (int n = 0; n < NV; ++n) out[n] = out[n] + xor_lane<1>(out[n]);
#pragma unroll
  for (int n = 0; n < NV; ++n) out[n] = out[n] + xor_lane<2>(out[n]);
#pragma unroll
  for (int n = 0; n < NV; ++n) out[n] = out[n] + xor_lane<4>(out[n]);
#pragma unroll
  for (int n = 0; n < NV; ++n) out[n] = out[n] + xor_lane<8>(out[n]);
#pragma unroll
  for (int n = 0; n < NV; ++n) out[n] = out[n] + xor_lane<16>(out[n]);
#pragma unroll
  for (int n = 0; n < NV; ++n) out[n] = out[n] + xor_lane<32>(out[n]);
}

// Quantize NV vectors of the wave (lane's E elements each, fp32 values of the input): the lane's
// E codes per vector (1 byte each) and the norms (all lanes).
template <int NV, int E>
__device__ __forceinline__ void hadamard_codes_wave_n(const float (&x)[NV][E], const float* __restrict__ signs,
                                                      const float* __restrict__ thr, int nthr, float inv,
                                                      uint32_t (&code)[NV][E], float (&nrm)[NV]) {
  const int lane = threadIdx.x & 63;
  float ss[NV];
  sumsq_wave_n<NV, E>(x, ss);
#pragma unroll
  for (int n = 0; n < NV; ++n) nrm[n] = __builtin_sqrtf(ss[n]);
  float sg[E];
#pragma unroll
  for (int e = 0; e < E; ++e) sg[e] = signs[lane * E + e];
  float v[NV][E];
#pragma unroll
  for (int n = 0; n < NV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) v[n][e] = x[n][e] * sg[e];
  fwht_wave_n<NV, E>(v);
#pragma unroll
  for (int n = 0; n < NV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float y = v[n][e] * inv;
      uint32_t c = 0;
      for (int j = 0; j < nthr; ++j) c += y >= __fmul_rn(thr[j], nrm[n]) ? 1u : 0u;
      code[n][e] = c;
    }
}

template <int E>
__device__ __forceinline__ float hadamard_codes_wave(const float (&x)[E], const float* __restrict__ signs,
                                                     const float* __restrict__ thr, int nthr, float inv,
                                                     uint32_t (&code)[E]) {
  float xv[1][E], nrm[1];
  uint32_t c[1][E];
#pragma unroll
  for (int e = 0; e < E; ++e) xv[0][e] = x[e];
  hadamard_codes_wave_n<1, E>(xv, signs, thr, nthr, inv, c, nrm);
#pragma unroll
  for (int e = 0; e < E; ++e) code[e] = c[0][e];
  return nrm[0];
}

}  // namespace anna
