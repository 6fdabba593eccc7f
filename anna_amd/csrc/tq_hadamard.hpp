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

__host__ __device__ constexpr bool tq_is_pow2(int64_t d) { return d > 0 && (d & (d - 1)) == 0; }

// fp32(1/sqrt(D)) (exact for D a power of 4)
__host__ __device__ inline float tq_inv_sqrt(int64_t D) {
  int l = 0;
  while ((int64_t(1) << l) < D) ++l;
  if ((l & 1) == 0) return 1.0f / (float)(int64_t(1) << (l / 2));
  return (float)(1.0 / __builtin_sqrt((double)D));
}

// In-place FWHT of the E elements each lane holds (stages as above, no scaling).
template <int E>
__device__ __forceinline__ void fwht_wave(float (&v)[E]) {
  // stages inside a lane: index bits 0 .. log2(E) - 1
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if ((e & h) == 0) {
        const float a = v[e], c = v[e + h];
        v[e] = a + c;
        v[e + h] = a - c;
      }
    }
  }
  // stages across lanes: index bits log2(E) .. log2(E) + 5 = lane bits 0 .. 5
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const bool upper = (lane & m) != 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float p = __shfl_xor(v[e], m, 64);
      v[e] = upper ? p - v[e] : v[e] + p;
    }
  }
}

// |x|^2 of the wave's vector in the fixed order above (every lane gets the total).
template <int E>
__device__ __forceinline__ float sumsq_wave(const float (&x)[E]) {
  float p = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) p = __builtin_fmaf(x[e], x[e], p);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) p = p + __shfl_xor(p, m, 64);
  return p;
}

// Quantize the wave's vector x (lane's E elements, fp32 values of the input): the lane's E codes
// (1 byte each) and the norm (all lanes).
template <int E>
__device__ __forceinline__ float hadamard_codes_wave(const float (&x)[E], const float* __restrict__ signs,
                                                     const float* __restrict__ thr, int nthr, float inv,
                                                     uint32_t (&code)[E]) {
  const int lane = threadIdx.x & 63;
  const float nrm = __builtin_sqrtf(sumsq_wave<E>(x));
  float v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = x[e] * signs[lane * E + e];
  fwht_wave<E>(v);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float y = v[e] * inv;
    uint32_t c = 0;
    for (int j = 0; j < nthr; ++j) c += y >= __fmul_rn(thr[j], nrm) ? 1u : 0u;
    code[e] = c;
  }
  return nrm;
}

}  // namespace anna
