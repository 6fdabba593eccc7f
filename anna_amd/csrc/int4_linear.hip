// Group-wise int4 weight-only linear on gfx950 (W4A16).
//
// Weight layout is the reference's XPUInt4Linear buffer layout
// (src/anna/model/quantization.py:460-487): qweight int32 [N, Kp/8] with nibble k%8
// of word k/8 at bits 4*(k%8), qscale [G, N], qzeros int8 [G, N], w = (q - z) * s.
//
// Kernels
//   int4_gemv_mfma   M <= 16.  HBM-bound.  Each wave owns NT 16-row tiles of W and a
//                    strided share of the K blocks (KW waves split K, reduced through
//                    LDS at the end).  One 128-bit load per lane brings 32 nibbles of
//                    one row; nibbles are turned into bf16/f16 "128+q" / "1024+q"
//                    patterns with one AND-OR per pair (exact small integers), fed to
//                    v_mfma_f32_16x16x32 against x, and the zero point is removed per
//                    128-k block with a row sum of x that a second MFMA against an
//                    all-ones operand produces in the same C layout:
//                       sum_k x (q - z) s = s * (sum_k x (off + q) - (off + z) sum_k x).
//   int4_gemm_mfma   M > 16.  LDS-tiled: a 128x128 tile of W is dequantized once per
//                    workgroup to bf16 ((q - z) * s rounded to bf16, the reference's
//                    dequant numerics) next to a 128x128 tile of x, and 4 waves run
//                    v_mfma_f32_32x32x16_bf16 on it.
//   int4_linear_generic  any dtype / group / alignment; VALU, one wave per output row.
#include "common.hpp"

namespace anna {
namespace {

// ------------------------------------------------------------------ helpers

// Turn 8 nibbles of `w` into 8 exact "off + q" values in the 16-bit float format of
// the MFMA: element 2p is nibble p, element 2p+1 is nibble p+4.
template <int XDT>
__device__ __forceinline__ u32x4 nibbles_to_frag(uint32_t w) {
  constexpr uint32_t MAGIC = XDT == ANNA_MI_BF16 ? 0x43004300u : 0x64006400u;
  u32x4 r;
  r.x = (w & 0x000F000Fu) | MAGIC;
  r.y = ((w >> 4) & 0x000F000Fu) | MAGIC;
  r.z = ((w >> 8) & 0x000F000Fu) | MAGIC;
  r.w = ((w >> 12) & 0x000F000Fu) | MAGIC;
  return r;
}

// Reorder 8 consecutive 16-bit activations (x0..x7) to the nibble order above:
// (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ u32x4 interleave_x(u32x4 v) {
  u32x4 r;
  r.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
  r.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
  r.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  r.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return r;
}

template <int XDT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (XDT == ANNA_MI_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// ------------------------------------------------------------------ GEMV (M <= 16)

constexpr int GEMV_UNROLL = 2;  // K blocks whose loads are issued together

template <int XDT, int SDT, int NT, int KW>
__global__ __launch_bounds__(64 * KW) void int4_gemv_mfma(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t xs,
    const uint32_t* __restrict__ qw, int64_t N, int64_t pc,
    const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz,
    int64_t blocks_per_group, uint16_t* __restrict__ y) {
  constexpr float OFF = XDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
  constexpr uint32_t ONES = XDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int kq = lane >> 4;
  const int64_t n_base = (int64_t)blockIdx.x * (16 * NT);
  const bool m_ok = r < M;
  const uint16_t* xrow = x + (int64_t)r * xs;
  const int64_t nblk = (K + 127) >> 7;
  const u32x4 ones = {ONES, ONES, ONES, ONES};

  const uint32_t* wrow[NT];
  bool n_ok[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n_base + t * 16 + r;
    n_ok[t] = n < N;
    wrow[t] = qw + (n_ok[t] ? n : 0) * pc + kq * 4;
  }

  f32x4 out[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) out[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int64_t b0 = wave; b0 < nblk; b0 += (int64_t)KW * GEMV_UNROLL) {
    u32x4 wv[GEMV_UNROLL][NT];
    u32x4 xa[GEMV_UNROLL][4];
#pragma unroll
    for (int u = 0; u < GEMV_UNROLL; ++u) {
      const int64_t b = b0 + (int64_t)u * KW;
      const bool b_ok = b < nblk;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        wv[u][t] = (b_ok && n_ok[t]) ? __builtin_nontemporal_load((const u32x4*)(wrow[t] + b * 16))
                                     : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int64_t k = b * 128 + kq * 32 + s * 8;
        xa[u][s] = (b_ok && m_ok && k < K) ? *(const u32x4*)(xrow + k) : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < GEMV_UNROLL; ++u) {
      const int64_t b = b0 + (int64_t)u * KW;
      if (b >= nblk) break;
      f32x4 acc[NT];
      f32x4 sx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4 a = interleave_x(xa[u][s]);
        sx = mfma16<XDT>(a, ones, sx);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const uint32_t w = wv[u][t][s];
          acc[t] = mfma16<XDT>(a, nibbles_to_frag<XDT>(w), acc[t]);
        }
      }
      // C layout: lane holds rows m = 4*kq + i of column n = n_base + 16t + r.
      const int64_t g = b / blocks_per_group;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t n = n_base + t * 16 + r;
        const int64_t gi = g * N + (n_ok[t] ? n : 0);
        const float sc = Elem<SDT>::load(qs, gi);
        const float c = OFF + (float)qz[gi];
#pragma unroll
        for (int i = 0; i < 4; ++i) out[t][i] = fmaf(sc, acc[t][i] - c * sx[i], out[t][i]);
      }
    }
  }

  if constexpr (KW > 1) {
    __shared__ float red[KW - 1][NT * 4][64];
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave - 1][t * 4 + i][lane] = out[t][i];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < KW - 1; ++w)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) out[t][i] += red[w][t * 4 + i][lane];
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n_base + t * 16 + r;
    if (!n_ok[t]) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = 4 * kq + i;
      if (m < M) y[m * N + n] = Elem<XDT>::cvt(out[t][i]);
    }
  }
}

// ------------------------------------------------------------------ GEMM (M > 16)

constexpr int GB_M = 128, GB_N = 128, GB_K = 128;
constexpr int G_LDS_PITCH = GB_K + 8;  // 16-bit elements; 16 B pad against bank conflicts

template <int SDT>
__global__ __launch_bounds__(256) void int4_gemm_mfma(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t xs,
    const uint32_t* __restrict__ qw, int64_t N, int64_t pc,
    const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz,
    int64_t gsz, uint16_t* __restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[GB_M * G_LDS_PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t sB[GB_N * G_LDS_PITCH];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 2x2 waves, 64x64 each
  const int64_t m0 = (int64_t)blockIdx.y * GB_M;
  const int64_t n0 = (int64_t)blockIdx.x * GB_N;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int64_t nblk = (K + GB_K - 1) / GB_K;
  for (int64_t b = 0; b < nblk; ++b) {
    const int64_t k0 = b * GB_K;
    // x tile: 128 rows x 128 k, 16 B per thread-load (8 values), 8 loads per thread.
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int idx = it * 256 + tid;  // 0..2047
      const int row = idx >> 4, c8 = (idx & 15) * 8;
      const int64_t m = m0 + row, k = k0 + c8;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < M && k < K) v = *(const u32x4*)(x + m * xs + k);
      *(u32x4*)(sA + row * G_LDS_PITCH + c8) = v;
    }
    // W tile: 128 rows x 16 words; each thread dequantizes 2 x uint4 (64 nibbles).
    const int64_t g = k0 / gsz;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int idx = it * 256 + tid;  // 0..511
      const int row = idx >> 2, q4 = (idx & 3) * 4;
      const int64_t n = n0 + row;
      u32x4 wv = {0u, 0u, 0u, 0u};
      float sc = 0.f, z = 0.f;
      if (n < N) {
        wv = __builtin_nontemporal_load((const u32x4*)(qw + n * pc + b * 16 + q4));
        sc = Elem<SDT>::load(qs, g * N + n);
        z = (float)qz[g * N + n];
      }
      uint16_t* dst = sB + row * G_LDS_PITCH + q4 * 8;
#pragma unroll
      for (int wi = 0; wi < 4; ++wi) {
        const uint32_t w = wv[wi];
        u32x4 o;
        uint32_t* op = (uint32_t*)&o;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float lo = ((float)((w >> (8 * p)) & 0xFu) - z) * sc;
          const float hi = ((float)((w >> (8 * p + 4)) & 0xFu) - z) * sc;
          op[p] = (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
        }
        *(u32x4*)(dst + wi * 8) = o;
      }
    }
    __syncthreads();
    // 8 k-steps of 16 on 32x32x16 MFMA.  A frag: row = lane%32, k = 8*(lane/32)+0..7.
#pragma unroll
    for (int ks = 0; ks < GB_K / 16; ++ks) {
      const int kk = ks * 16 + (lane >> 5) * 8;
      u32x4 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *(const u32x4*)(sA + (wm * 64 + i * 32 + (lane & 31)) * G_LDS_PITCH + kk);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bfr[j] = *(const u32x4*)(sB + (wn * 64 + j * 32 + (lane & 31)) * G_LDS_PITCH + kk);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[i]),
                                                              __builtin_bit_cast(bf16x8, bfr[j]),
                                                              acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  // 32x32 C layout: column = lane%32, row = 8*(e/4) + 4*(lane/32)... (e%4) -- see below.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t m = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (m < M) y[m * N + n] = f32_to_bf16_bits(acc[i][j][e]);
      }
    }
}

// ------------------------------------------------------------------ generic

template <int XDT, int SDT>
__global__ __launch_bounds__(64) void int4_linear_generic(
    const typename Elem<XDT>::T* __restrict__ x, int64_t M, int64_t K, int64_t xs,
    const uint32_t* __restrict__ qw, int64_t N, int64_t pc,
    const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz,
    int64_t gsz, typename Elem<XDT>::T* __restrict__ y) {
  const int64_t n = blockIdx.x;
  const int lane = threadIdx.x;
  for (int64_t m0 = (int64_t)blockIdx.y * 8; m0 < M; m0 += (int64_t)gridDim.y * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t k = lane; k < K; k += 64) {
      const uint32_t word = qw[n * pc + (k >> 3)];
      const int64_t gi = (k / gsz) * N + n;
      const float w = ((float)((word >> (4 * (k & 7))) & 0xFu) - (float)qz[gi]) * Elem<SDT>::load(qs, gi);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (m0 + i < M) acc[i] = fmaf(Elem<XDT>::load(x, (m0 + i) * xs + k), w, acc[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s = wave_sum(acc[i]);
      if (lane == 0 && m0 + i < M) y[(m0 + i) * N + n] = Elem<XDT>::cvt(s);
    }
  }
}

// ------------------------------------------------------------------ quantize / dequant

template <int WDT>
__global__ __launch_bounds__(64) void int4_quantize_kernel(
    const typename Elem<WDT>::T* __restrict__ w, int64_t N, int64_t K, int64_t Kp, int64_t gsz,
    int rounding, uint32_t* __restrict__ qw, float* __restrict__ qs, int8_t* __restrict__ qz) {
  // one wave per (row, group)
  const int64_t G = Kp / gsz;
  const int64_t n = blockIdx.x / G;
  const int64_t g = blockIdx.x % G;
  const int lane = threadIdx.x;
  float amax = 0.f;
  for (int64_t j = lane; j < gsz; j += 64) {
    const int64_t k = g * gsz + j;
    const float v = k < K ? Elem<WDT>::load(w, n * K + k) : 0.f;
    amax = fmaxf(amax, fabsf(v));
  }
  amax = wave_max(amax);
  const float scale = amax > 0.f ? amax / 7.0f : 1.0f;
  if (lane == 0) {
    qs[g * N + n] = scale;
    qz[g * N + n] = 8;
  }
  for (int64_t wd = lane; wd < gsz / 8; wd += 64) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = g * gsz + wd * 8 + j;
      const float v = k < K ? Elem<WDT>::load(w, n * K + k) : 0.f;
      float t = __fdiv_rn(v, scale);
      t = __fadd_rn(t, 8.0f);
      float rq = rounding == 0 ? rintf(t) : roundf(t);
      rq = fminf(fmaxf(rq, 0.f), 15.f);
      word |= ((uint32_t)rq & 0xFu) << (4 * j);
    }
    qw[n * (Kp / 8) + (g * gsz) / 8 + wd] = word;
  }
}

__global__ __launch_bounds__(256) void autoround_repack_kernel(
    const uint32_t* __restrict__ gq, const uint32_t* __restrict__ gz, const uint16_t* __restrict__ sc16,
    int64_t K, int64_t N, int64_t gsz, int64_t G, int64_t Kp, uint32_t* __restrict__ qw,
    float* __restrict__ qs, int8_t* __restrict__ qz) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n8 = (N + 7) / 8;
  const int64_t pc = Kp / 8;
  if (idx < G * N) {
    const int64_t g = idx / N, n = idx % N;
    const int z = (int)((gz[g * n8 + n / 8] >> (4 * (n % 8))) & 0xFu) + 1;
    qz[idx] = (int8_t)z;
    qs[idx] = f16_bits_to_f32(sc16[idx]);
  }
  if (idx < N * pc) {
    const int64_t n = idx / pc, kw = idx % pc;
    int64_t tail_g = K / gsz;
    if (tail_g > G - 1) tail_g = G - 1;
    const int tail_z = (int)((gz[tail_g * n8 + n / 8] >> (4 * (n % 8))) & 0xFu) + 1;
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = kw * 8 + j;
      uint32_t q;
      if (k < K) q = (gq[(k / 8) * N + n] >> (4 * (k % 8))) & 0xFu;
      else q = (uint32_t)tail_z & 0xFu;
      word |= q << (4 * j);
    }
    qw[idx] = word;
  }
}

template <int SDT, int ODT>
__global__ __launch_bounds__(256) void int4_dequant_kernel(
    const uint32_t* __restrict__ qw, int64_t N, int64_t pc, const typename Elem<SDT>::T* __restrict__ qs,
    const int8_t* __restrict__ qz, int64_t gsz, int64_t K, typename Elem<ODT>::T* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one word
  const int64_t kw_per_row = (K + 7) / 8;
  if (idx >= N * kw_per_row) return;
  const int64_t n = idx / kw_per_row, kw = idx % kw_per_row;
  const uint32_t word = qw[n * pc + kw];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t k = kw * 8 + j;
    if (k >= K) break;
    const int64_t gi = (k / gsz) * N + n;
    const float v = ((float)((word >> (4 * j)) & 0xFu) - (float)qz[gi]) * Elem<SDT>::load(qs, gi);
    out[n * K + k] = Elem<ODT>::cvt(v);
  }
}

template <int XDT, int SDT, int NT, int KW>
void launch_gemv(const void* x, int64_t M, int64_t K, int64_t xs, const int32_t* qw, int64_t N,
                 int64_t pc, const void* qs, const int8_t* qz, int64_t gsz, void* y, hipStream_t st) {
  dim3 grid((unsigned)((N + 16 * NT - 1) / (16 * NT)), 1, 1);
  hipLaunchKernelGGL((int4_gemv_mfma<XDT, SDT, NT, KW>), grid, dim3(64 * KW), 0, st,
                     (const uint16_t*)x, M, K, xs, (const uint32_t*)qw, N, pc,
                     (const typename Elem<SDT>::T*)qs, qz, gsz / 128, (uint16_t*)y);
}

}  // namespace
}  // namespace anna

using namespace anna;

extern "C" int anna_mi_int4_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t xs,
                                   const int32_t* qweight, int64_t N, int64_t pc, const void* qscale,
                                   int scale_dtype, const int8_t* qzeros, int64_t G, int64_t gsz,
                                   void* y, void* stream) {
  ANNA_CHECK(x && qweight && qscale && qzeros && y, "anna_mi_int4_linear: null pointer");
  ANNA_CHECK(valid_dtype(x_dtype) && valid_dtype(scale_dtype), "anna_mi_int4_linear: bad dtype code");
  ANNA_CHECK(M > 0 && N > 0 && K > 0, "anna_mi_int4_linear: M, N, K must be positive (got %lld, %lld, %lld)",
             (long long)M, (long long)N, (long long)K);
  ANNA_CHECK(gsz > 0, "anna_mi_int4_linear: group_size must be positive");
  ANNA_CHECK(pc * 8 >= K, "anna_mi_int4_linear: qweight packed columns (%lld) are smaller than in_features (%lld)",
             (long long)pc, (long long)K);
  ANNA_CHECK(G * gsz >= K, "anna_mi_int4_linear: qscale group count is smaller than in_features");
  ANNA_CHECK(xs >= K, "anna_mi_int4_linear: x row stride smaller than K");
  hipStream_t st = as_stream(stream);
  const bool x16 = x_dtype != ANNA_MI_F32;
  const bool aligned = ((uintptr_t)x % 16 == 0) && (xs % 8 == 0) && (K % 8 == 0) &&
                       ((uintptr_t)qweight % 16 == 0) && (pc % 4 == 0) && (gsz % 128 == 0);
  if (x16 && aligned && M <= 16) {
    ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
      if (x_dtype == ANNA_MI_BF16)
        launch_gemv<ANNA_MI_BF16, SDT, 1, 4>(x, M, K, xs, qweight, N, pc, qscale, qzeros, gsz, y, st);
      else
        launch_gemv<ANNA_MI_F16, SDT, 1, 4>(x, M, K, xs, qweight, N, pc, qscale, qzeros, gsz, y, st);
    });
    ANNA_LAUNCH_CHECK("int4_gemv_mfma");
    return ANNA_MI_OK;
  }
  if (x_dtype == ANNA_MI_BF16 && aligned && M > 16) {
    dim3 grid((unsigned)((N + GB_N - 1) / GB_N), (unsigned)((M + GB_M - 1) / GB_M), 1);
    ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
      hipLaunchKernelGGL((int4_gemm_mfma<SDT>), grid, dim3(256), 0, st, (const uint16_t*)x, M, K, xs,
                         (const uint32_t*)qweight, N, pc, (const typename Elem<SDT>::T*)qscale, qzeros,
                         gsz, (uint16_t*)y);
    });
    ANNA_LAUNCH_CHECK("int4_gemm_mfma");
    return ANNA_MI_OK;
  }
  dim3 grid((unsigned)N, (unsigned)((M + 7) / 8 < 64 ? (M + 7) / 8 : 64), 1);
  ANNA_DISPATCH_DTYPE(x_dtype, XDT, {
    ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
      hipLaunchKernelGGL((int4_linear_generic<XDT, SDT>), grid, dim3(64), 0, st,
                         (const typename Elem<XDT>::T*)x, M, K, xs, (const uint32_t*)qweight, N, pc,
                         (const typename Elem<SDT>::T*)qscale, qzeros, gsz, (typename Elem<XDT>::T*)y);
    });
  });
  ANNA_LAUNCH_CHECK("int4_linear_generic");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_int4_dequant(const int32_t* qweight, int64_t N, int64_t pc, const void* qscale,
                                    int scale_dtype, const int8_t* qzeros, int64_t G, int64_t gsz, int64_t K,
                                    void* w_out, int out_dtype, void* stream) {
  ANNA_CHECK(qweight && qscale && qzeros && w_out, "anna_mi_int4_dequant: null pointer");
  ANNA_CHECK(valid_dtype(scale_dtype) && valid_dtype(out_dtype), "anna_mi_int4_dequant: bad dtype code");
  ANNA_CHECK(N > 0 && K > 0 && gsz > 0 && pc * 8 >= K && G * gsz >= K, "anna_mi_int4_dequant: bad shape");
  const int64_t total = N * ((K + 7) / 8);
  dim3 grid((unsigned)((total + 255) / 256));
  ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
    ANNA_DISPATCH_DTYPE(out_dtype, ODT, {
      hipLaunchKernelGGL((int4_dequant_kernel<SDT, ODT>), grid, dim3(256), 0, as_stream(stream),
                         (const uint32_t*)qweight, N, pc, (const typename Elem<SDT>::T*)qscale, qzeros, gsz, K,
                         (typename Elem<ODT>::T*)w_out);
    });
  });
  ANNA_LAUNCH_CHECK("int4_dequant_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_int4_quantize(const void* w, int w_dtype, int64_t N, int64_t K, int64_t Kp, int64_t gsz,
                                     int rounding, int32_t* qweight, float* qscale, int8_t* qzeros, void* stream) {
  ANNA_CHECK(w && qweight && qscale && qzeros, "anna_mi_int4_quantize: null pointer");
  ANNA_CHECK(valid_dtype(w_dtype), "anna_mi_int4_quantize: bad dtype code");
  ANNA_CHECK(N > 0 && K > 0 && gsz > 0 && gsz % 8 == 0, "anna_mi_int4_quantize: bad shape");
  ANNA_CHECK(Kp >= K && Kp % gsz == 0 && Kp % 8 == 0, "anna_mi_int4_quantize: padded_in_features must cover K and be a multiple of group_size and 8");
  ANNA_CHECK(rounding == 0 || rounding == 1, "anna_mi_int4_quantize: rounding must be 0 or 1");
  const int64_t G = Kp / gsz;
  ANNA_CHECK(N * G < (1ll << 31), "anna_mi_int4_quantize: too many groups");
  ANNA_DISPATCH_DTYPE(w_dtype, WDT, {
    hipLaunchKernelGGL((int4_quantize_kernel<WDT>), dim3((unsigned)(N * G)), dim3(64), 0, as_stream(stream),
                       (const typename Elem<WDT>::T*)w, N, K, Kp, gsz, rounding, (uint32_t*)qweight, qscale, qzeros);
  });
  ANNA_LAUNCH_CHECK("int4_quantize_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_autoround_to_int4(const int32_t* gq, const int32_t* gz, const uint16_t* sc16, int64_t K,
                                         int64_t N, int64_t gsz, int64_t G, int64_t Kp, int32_t* qweight,
                                         float* qscale, int8_t* qzeros, void* stream) {
  ANNA_CHECK(gq && gz && sc16 && qweight && qscale && qzeros, "anna_mi_autoround_to_int4: null pointer");
  ANNA_CHECK(K > 0 && N > 0 && gsz > 0 && G > 0 && Kp >= K && Kp % 8 == 0, "anna_mi_autoround_to_int4: bad shape");
  const int64_t total = G * N > N * (Kp / 8) ? G * N : N * (Kp / 8);
  hipLaunchKernelGGL(autoround_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, as_stream(stream),
                     (const uint32_t*)gq, (const uint32_t*)gz, sc16, K, N, gsz, G, Kp, (uint32_t*)qweight, qscale,
                     qzeros);
  ANNA_LAUNCH_CHECK("autoround_repack_kernel");
  return ANNA_MI_OK;
}
