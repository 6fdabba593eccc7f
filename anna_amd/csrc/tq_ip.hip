// TurboQuant inner-product keys (TurboQuant_prod: an MSE stage plus a 1-bit QJL sketch of its
// residual) on gfx950: quantize, dequantize, and attention scores straight from the codes.
//
// This build's definition of the third-party TurboQuantIP(dim, bits, seed) that the reference
// calls (src/anna/model/turboquant.py:84-92, 255-332; the package is absent), following the
// published algorithm (Zandieh et al., "TurboQuant: Online Vector Quantization with
// Near-optimal Distortion Rate", 2025, Algorithm 2):
//   norm = |x|, y = R x (the randomized Hadamard rotation of TQ-MSE, tq_hadamard.hpp),
//   code_i = #{j : y_i >= fl(t_j * norm)} with the (bits-1)-bit Lloyd-Max thresholds t,
//   rho_i = fma(-c[code_i], norm, y_i)           (residual of the MSE stage, rotated, scaled by norm),
//   gamma = sqrt(|rho|^2) (the fixed order of tq_hadamard.hpp), residual_norm = gamma / norm,
//   z = G rho with G a seeded D x D standard-normal matrix, qjl_i = (z_i >= 0).
// Reconstruction:  x~ = norm * R^T (c[code] + k0 * residual_norm * G^T (2 qjl - 1)),
//   k0 = fl(sqrt(pi/2) / D).  In the reference's terms S = G R: the QJL signs are those of
//   S (x / norm - R^T c[code]), and its score formula (turboquant.py:311-332) becomes
//   q . x~ = norm * ((R q) . c[code] + k0 * residual_norm * (G R q) . (2 qjl - 1)),
// which is what tq_ip_scores_kernel evaluates: the query is rotated and projected once, the
// keys are never expanded.
//
// Arithmetic order (fixed so that the CPU oracle reproduces quantize and dequantize bit for bit):
//   every matrix-vector product out_j = sum_k M[k][j] v_k is one fma chain from 0 in ascending k;
//   dequantize: u = fma(k0 * rn, w, c[code]), t = FWHT(u)_k * fl(1/sqrt(D)), t = t * s_k, out = norm * t.
#include <math.h>

#include <vector>

#include "common.hpp"
#include "tq_hadamard.hpp"

namespace anna {
namespace {

constexpr int IPNV = 4;  // vectors per wave

// out[n][e] (index lane*E + e) = sum_k M[k*D + lane*E + e] * vl[n*D + k], k ascending (one fma
// chain from 0).  vl: the wave's vectors in LDS.
template <int NV, int E>
__device__ __forceinline__ void matvec_wave_n(const float* __restrict__ M, const float* vl, int64_t D,
                                              float (&out)[NV][E]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int n = 0; n < NV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) out[n][e] = 0.f;
  const float* col = M + lane * E;
#pragma unroll 4
  for (int64_t k = 0; k < D; ++k) {
    float g[E];
    if constexpr (E % 4 == 0) {
#pragma unroll
      for (int e = 0; e < E; e += 4) {
        const float4 v = *(const float4*)(col + k * D + e);
        g[e] = v.x, g[e + 1] = v.y, g[e + 2] = v.z, g[e + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) g[e] = col[k * D + e];
    }
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const float vk = vl[n * D + k];
#pragma unroll
      for (int e = 0; e < E; ++e) out[n][e] = __builtin_fmaf(g[e], vk, out[n][e]);
    }
  }
}

// y = fl(1/sqrt(D)) * FWHT(s .* x), as the TQ-MSE quantizer forms it
template <int NV, int E>
__device__ __forceinline__ void rotate_wave_n(const float (&x)[NV][E], const float* __restrict__ signs, float inv,
                                              float (&y)[NV][E]) {
  const int lane = threadIdx.x & 63;
  float sg[E];
#pragma unroll
  for (int e = 0; e < E; ++e) sg[e] = signs[lane * E + e];
#pragma unroll
  for (int n = 0; n < NV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) y[n][e] = x[n][e] * sg[e];
  fwht_wave_n<NV, E>(y);
#pragma unroll
  for (int n = 0; n < NV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) y[n][e] = y[n][e] * inv;
}

// 4 waves per 256-thread workgroup, IPNV vectors per wave, lane l holds elements l*E .. l*E+E-1.
// Every wave reaches the barrier (a wave past the end works on clamped copies and stores nothing).
template <int XDT, int E>
__global__ __launch_bounds__(256) void tq_ip_quantize_kernel(
    const typename Elem<XDT>::T* __restrict__ x, int64_t nvec, int64_t D, int64_t xs,
    const float* __restrict__ signs, const float* __restrict__ thr, const float* __restrict__ cent, int nthr,
    const float* __restrict__ gt, uint8_t* __restrict__ idx_out, uint8_t* __restrict__ qjl_out,
    float* __restrict__ norm_out, float* __restrict__ rn_out) {
  __shared__ float rl[4][IPNV * 64 * E];
  const int wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t v0 = ((int64_t)blockIdx.x * 4 + wave) * IPNV;
  float xv[IPNV][E];
#pragma unroll
  for (int n = 0; n < IPNV; ++n) {
    int64_t v = v0 + n < nvec ? v0 + n : nvec - 1;
#pragma unroll
    for (int e = 0; e < E; ++e) xv[n][e] = Elem<XDT>::load(x, v * xs + lane * E + e);
  }
  float ss[IPNV], nrm[IPNV];
  sumsq_wave_n<IPNV, E>(xv, ss);
#pragma unroll
  for (int n = 0; n < IPNV; ++n) nrm[n] = __builtin_sqrtf(ss[n]);
  float y[IPNV][E];
  rotate_wave_n<IPNV, E>(xv, signs, tq_inv_sqrt(D), y);
  uint32_t code[IPNV][E];
  float rho[IPNV][E];
#pragma unroll
  for (int n = 0; n < IPNV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      uint32_t c = 0;
      for (int j = 0; j < nthr; ++j) c += y[n][e] >= __fmul_rn(thr[j], nrm[n]) ? 1u : 0u;
      code[n][e] = c;
      rho[n][e] = __builtin_fmaf(-cent[c], nrm[n], y[n][e]);
    }
  float gg[IPNV];
  sumsq_wave_n<IPNV, E>(rho, gg);
  float* my = rl[wave];
#pragma unroll
  for (int n = 0; n < IPNV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) my[n * D + lane * E + e] = rho[n][e];
  __syncthreads();
  float z[IPNV][E];
  matvec_wave_n<IPNV, E>(gt, my, D, z);
#pragma unroll
  for (int n = 0; n < IPNV; ++n) {
    const int64_t v = v0 + n;
    if (v >= nvec) break;
    uint8_t* ib = idx_out + v * D + lane * E;
    uint8_t* qb = qjl_out + v * D + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      ib[e] = (uint8_t)code[n][e];
      qb[e] = z[n][e] >= 0.f ? 1 : 0;
    }
    if (lane == 0) {
      norm_out[v] = nrm[n];
      rn_out[v] = nrm[n] > 0.f ? __fdiv_rn(__builtin_sqrtf(gg[n]), nrm[n]) : 0.f;
    }
  }
}

template <int ODT, int E>
__global__ __launch_bounds__(256) void tq_ip_dequant_kernel(
    const uint8_t* __restrict__ idx, const uint8_t* __restrict__ qjl, const float* __restrict__ norms,
    const float* __restrict__ rn, int64_t nvec, int64_t D, const float* __restrict__ signs,
    const float* __restrict__ cent, const float* __restrict__ g, float k0, typename Elem<ODT>::T* __restrict__ out,
    int64_t os) {
  __shared__ float sl[4][IPNV * 64 * E];
  const int wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t v0 = ((int64_t)blockIdx.x * 4 + wave) * IPNV;
  float* my = sl[wave];
  float c[IPNV][E];
#pragma unroll
  for (int n = 0; n < IPNV; ++n) {
    const int64_t v = v0 + n < nvec ? v0 + n : nvec - 1;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      c[n][e] = cent[idx[v * D + lane * E + e]];
      my[n * D + lane * E + e] = qjl[v * D + lane * E + e] ? 1.f : -1.f;
    }
  }
  __syncthreads();
  float w[IPNV][E];
  matvec_wave_n<IPNV, E>(g, my, D, w);
  const float inv = tq_inv_sqrt(D);
  float sg[E];
#pragma unroll
  for (int e = 0; e < E; ++e) sg[e] = signs[lane * E + e];
  float nrm[IPNV];
#pragma unroll
  for (int n = 0; n < IPNV; ++n) {
    const int64_t v = v0 + n < nvec ? v0 + n : nvec - 1;
    const float coef = k0 * rn[v];
    nrm[n] = norms[v];
#pragma unroll
    for (int e = 0; e < E; ++e) w[n][e] = __builtin_fmaf(coef, w[n][e], c[n][e]);
  }
  fwht_wave_n<IPNV, E>(w);
#pragma unroll
  for (int n = 0; n < IPNV; ++n) {
    const int64_t v = v0 + n;
    if (v >= nvec) break;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float t = w[n][e] * inv;
      t = t * sg[e];
      out[v * os + lane * E + e] = Elem<ODT>::cvt(nrm[n] * t);
    }
  }
}

// One wave per query row r = hq * Lq + lq: ws[r][0][:] = R q, ws[r][1][:] = G R q (fp32).
template <int QDT, int E>
__global__ __launch_bounds__(256) void tq_ip_query_kernel(const typename Elem<QDT>::T* __restrict__ q, int64_t rows,
                                                          int64_t Lq, int64_t D, int64_t sh, int64_t sl_,
                                                          const float* __restrict__ signs,
                                                          const float* __restrict__ gt, float* __restrict__ ws) {
  __shared__ float ql[4][64 * E];
  const int wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t r0 = (int64_t)blockIdx.x * 4 + wave;
  const int64_t r = r0 < rows ? r0 : rows - 1;
  const int64_t hq = r / Lq, lq = r % Lq;
  float xv[1][E], y[1][E];
#pragma unroll
  for (int e = 0; e < E; ++e) xv[0][e] = Elem<QDT>::load(q, hq * sh + lq * sl_ + lane * E + e);
  rotate_wave_n<1, E>(xv, signs, tq_inv_sqrt(D), y);
#pragma unroll
  for (int e = 0; e < E; ++e) ql[wave][lane * E + e] = y[0][e];
  __syncthreads();
  float p[1][E];
  matvec_wave_n<1, E>(gt, ql[wave], D, p);
  if (r0 < rows) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      ws[r * 2 * D + lane * E + e] = y[0][e];
      ws[r * 2 * D + D + lane * E + e] = p[0][e];
    }
  }
}

// Scores of 64 tokens x 16 query rows of one KV head per 256-thread workgroup.  Thread (t, rg)
// takes token t and rows 4 rg .. 4 rg + 3.  The keys' centroid values and +-1 signs are staged
// 64 dims at a time into LDS (row stride 65: conflict-free across tokens), with the same 64
// dims of R q and G R q for the 16 rows.
constexpr int SC_TOK = 64, SC_ROWS = 16, SC_DIM = 64;

__global__ __launch_bounds__(256) void tq_ip_scores_kernel(const float* __restrict__ ws, int64_t GL, int64_t D,
                                                           const uint8_t* __restrict__ idx,
                                                           const uint8_t* __restrict__ qjl,
                                                           const float* __restrict__ norms,
                                                           const float* __restrict__ rn, int64_t T,
                                                           const float* __restrict__ cent, float k0, float scaling,
                                                           float* __restrict__ out) {
  __shared__ float cf[SC_TOK][SC_DIM + 1], sf[SC_TOK][SC_DIM + 1];
  __shared__ float qs[SC_ROWS][SC_DIM], ps[SC_ROWS][SC_DIM];
  const int tid = threadIdx.x, t = tid & 63, rg = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * SC_TOK, hkv = blockIdx.y, r0 = (int64_t)blockIdx.z * SC_ROWS;
  float am[4] = {0.f, 0.f, 0.f, 0.f}, aq[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t d0 = 0; d0 < D; d0 += SC_DIM) {
    for (int i = tid; i < SC_TOK * SC_DIM; i += 256) {
      const int tt = i / SC_DIM, kk = i % SC_DIM;
      const int64_t tok = t0 + tt;
      float a = 0.f, b = 0.f;
      if (tok < T) {
        const int64_t o = (hkv * T + tok) * D + d0 + kk;
        a = cent[idx[o]];
        b = qjl[o] ? 1.f : -1.f;
      }
      cf[tt][kk] = a;
      sf[tt][kk] = b;
    }
    for (int i = tid; i < SC_ROWS * SC_DIM; i += 256) {
      const int rr = i / SC_DIM, kk = i % SC_DIM;
      const int64_t row = r0 + rr;
      float a = 0.f, b = 0.f;
      if (row < GL) {
        const float* w = ws + (hkv * GL + row) * 2 * D + d0 + kk;
        a = w[0];
        b = w[D];
      }
      qs[rr][kk] = a;
      ps[rr][kk] = b;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < SC_DIM; ++kk) {
      const float a = cf[t][kk], b = sf[t][kk];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        am[j] = __builtin_fmaf(qs[rg * 4 + j][kk], a, am[j]);
        aq[j] = __builtin_fmaf(ps[rg * 4 + j][kk], b, aq[j]);
      }
    }
    __syncthreads();
  }
  const int64_t tok = t0 + t;
  if (tok >= T) return;
  const float nrm = norms[hkv * T + tok], coef = k0 * rn[hkv * T + tok];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t row = r0 + rg * 4 + j;
    if (row < GL) out[(hkv * GL + row) * T + tok] = scaling * (nrm * __builtin_fmaf(coef, aq[j], am[j]));
  }
}

template <typename F>
void dispatch_e(int64_t D, F&& go) {
  switch (D) {
    case 64: go(std::integral_constant<int, 1>{}); break;
    case 128: go(std::integral_constant<int, 2>{}); break;
    case 256: go(std::integral_constant<int, 4>{}); break;
    case 512: go(std::integral_constant<int, 8>{}); break;
    default: go(std::integral_constant<int, 16>{}); break;
  }
}

bool ip_dim_ok(int64_t D) { return D == 64 || D == 128 || D == 256 || D == 512 || D == 1024; }

float ip_k0(int64_t D) { return (float)(1.2533141373155002512 / (double)D); }

}  // namespace
}  // namespace anna

using namespace anna;

extern "C" int anna_mi_tq_ip_gaussian(int64_t D, uint64_t seed, float* out) {
  ANNA_CHECK(out != nullptr && D > 0 && D <= 4096, "anna_mi_tq_ip_gaussian: bad arguments");
  std::vector<double> g((size_t)(D * D));
  tq_gaussian(D * D, seed, g.data());
  for (int64_t i = 0; i < D * D; ++i) out[i] = (float)g[(size_t)i];
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_ip_quantize(const void* x, int x_dtype, int64_t nvec, int64_t D, int64_t x_row_stride,
                                      const float* signs, const float* thresholds, const float* centroids,
                                      const float* gaussian_t, int bits, uint8_t* mse_indices, uint8_t* qjl_signs,
                                      float* norms, float* residual_norms, void* stream) {
  if (nvec == 0) return ANNA_MI_OK;  // empty state: nothing to read or write
  ANNA_CHECK(x && signs && thresholds && centroids && gaussian_t && mse_indices && qjl_signs && norms && residual_norms,
             "anna_mi_tq_ip_quantize: null pointer");
  ANNA_CHECK(valid_dtype(x_dtype), "anna_mi_tq_ip_quantize: bad dtype code");
  ANNA_CHECK(bits >= 2 && bits <= 4, "anna_mi_tq_ip_quantize: bits must be 2..4");
  ANNA_CHECK(ip_dim_ok(D), "anna_mi_tq_ip_quantize: head_dim must be a power of two in [64, 1024]");
  ANNA_CHECK(x_row_stride >= D, "anna_mi_tq_ip_quantize: row stride smaller than head_dim");
  ANNA_CHECK(nvec > 0, "anna_mi_tq_ip_quantize: negative vector count");
  const dim3 grid((unsigned)((nvec + 4 * IPNV - 1) / (4 * IPNV)));
  const int nthr = (1 << (bits - 1)) - 1;
  ANNA_DISPATCH_DTYPE(x_dtype, XDT, {
    dispatch_e(D, [&](auto e_tag) {
      constexpr int E = decltype(e_tag)::value;
      hipLaunchKernelGGL((tq_ip_quantize_kernel<XDT, E>), grid, dim3(256), 0, as_stream(stream),
                         (const typename Elem<XDT>::T*)x, nvec, D, x_row_stride, signs, thresholds, centroids, nthr,
                         gaussian_t, mse_indices, qjl_signs, norms, residual_norms);
    });
  });
  ANNA_LAUNCH_CHECK("tq_ip_quantize_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_ip_dequant(const uint8_t* mse_indices, const uint8_t* qjl_signs, const float* norms,
                                     const float* residual_norms, int64_t nvec, int64_t D, const float* signs,
                                     const float* centroids, const float* gaussian, int bits, void* out, int out_dtype,
                                     int64_t out_row_stride, void* stream) {
  if (nvec == 0) return ANNA_MI_OK;  // empty state: nothing to read or write
  ANNA_CHECK(mse_indices && qjl_signs && norms && residual_norms && signs && centroids && gaussian && out,
             "anna_mi_tq_ip_dequant: null pointer");
  ANNA_CHECK(valid_dtype(out_dtype), "anna_mi_tq_ip_dequant: bad dtype code");
  ANNA_CHECK(bits >= 2 && bits <= 4, "anna_mi_tq_ip_dequant: bits must be 2..4");
  ANNA_CHECK(ip_dim_ok(D), "anna_mi_tq_ip_dequant: head_dim must be a power of two in [64, 1024]");
  ANNA_CHECK(out_row_stride >= D, "anna_mi_tq_ip_dequant: row stride smaller than head_dim");
  ANNA_CHECK(nvec > 0, "anna_mi_tq_ip_dequant: negative vector count");
  const dim3 grid((unsigned)((nvec + 4 * IPNV - 1) / (4 * IPNV)));
  ANNA_DISPATCH_DTYPE(out_dtype, ODT, {
    dispatch_e(D, [&](auto e_tag) {
      constexpr int E = decltype(e_tag)::value;
      hipLaunchKernelGGL((tq_ip_dequant_kernel<ODT, E>), grid, dim3(256), 0, as_stream(stream), mse_indices, qjl_signs,
                         norms, residual_norms, nvec, D, signs, centroids, gaussian, ip_k0(D),
                         (typename Elem<ODT>::T*)out, out_row_stride);
    });
  });
  ANNA_LAUNCH_CHECK("tq_ip_dequant_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_ip_scores(const void* query, int q_dtype, int64_t Hq, int64_t Lq, int64_t D,
                                    int64_t q_stride_h, int64_t q_stride_l, const uint8_t* mse_indices,
                                    const uint8_t* qjl_signs, const float* norms, const float* residual_norms,
                                    int64_t Hkv, int64_t T, const float* signs, const float* centroids,
                                    const float* gaussian_t, int bits, float scaling, float* workspace, float* out,
                                    void* stream) {
  if (Lq == 0 || T == 0) return ANNA_MI_OK;  // empty query or key state: no scores
  ANNA_CHECK(query && mse_indices && qjl_signs && norms && residual_norms && signs && centroids && gaussian_t &&
                 workspace && out,
             "anna_mi_tq_ip_scores: null pointer");
  ANNA_CHECK(valid_dtype(q_dtype), "anna_mi_tq_ip_scores: bad dtype code");
  ANNA_CHECK(bits >= 2 && bits <= 4, "anna_mi_tq_ip_scores: bits must be 2..4");
  ANNA_CHECK(ip_dim_ok(D), "anna_mi_tq_ip_scores: head_dim must be a power of two in [64, 1024]");
  ANNA_CHECK(Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "anna_mi_tq_ip_scores: query heads must be a multiple of KV heads");
  ANNA_CHECK(Lq > 0 && T > 0, "anna_mi_tq_ip_scores: negative length");
  const int64_t rows = Hq * Lq, GL = (Hq / Hkv) * Lq;
  ANNA_CHECK(GL / SC_ROWS + 1 < 65536 && Hkv < 65536, "anna_mi_tq_ip_scores: too many query rows");
  ANNA_DISPATCH_DTYPE(q_dtype, QDT, {
    dispatch_e(D, [&](auto e_tag) {
      constexpr int E = decltype(e_tag)::value;
      hipLaunchKernelGGL((tq_ip_query_kernel<QDT, E>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                         as_stream(stream), (const typename Elem<QDT>::T*)query, rows, Lq, D, q_stride_h, q_stride_l,
                         signs, gaussian_t, workspace);
    });
  });
  ANNA_LAUNCH_CHECK("tq_ip_query_kernel");
  const dim3 grid((unsigned)((T + SC_TOK - 1) / SC_TOK), (unsigned)Hkv, (unsigned)((GL + SC_ROWS - 1) / SC_ROWS));
  hipLaunchKernelGGL(tq_ip_scores_kernel, grid, dim3(256), 0, as_stream(stream), workspace, GL, D, mse_indices,
                     qjl_signs, norms, residual_norms, T, centroids, ip_k0(D), scaling, out);
  ANNA_LAUNCH_CHECK("tq_ip_scores_kernel");
  return ANNA_MI_OK;
}
