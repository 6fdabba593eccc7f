// Group-wise int4 weight-only linear on gfx950 (W4A16).
//
// Weight layout is the reference's XPUInt4Linear buffer layout
// (src/anna/model/quantization.py:460-487): qweight int32 [N, Kp/8] with nibble k%8
// of word k/8 at bits 4*(k%8), qscale [G, N], qzeros int8 [G, N], w = (q - z) * s.
//
// Kernels
//   int4_gemv_dot2   M <= 2 (16-bit x).  HBM-bound.  Each wave owns 4 output rows; a lane
//                    loads 16 bytes (32 weights) of a row per buffer load, turns nibble pairs
//                    into bf16/f16 "off + q" with one AND-OR, accumulates v_dot2 in fp32 against
//                    the pre-interleaved x and removes the zero point once per group; partials
//                    are reduced with swizzle/DPP steps.  XCD-aware workgroup -> row map.
//   int4_gemv_mfma   other M < 64 (16-bit x, K <= 4096 for M > 16).  HBM-bound.  Each wave owns NT
//                    16-row tiles of W and a strided share of the K blocks (KW waves split K, reduced through
//                    LDS at the end).  One 128-bit load per lane brings 32 nibbles of
//                    one row; nibbles are turned into bf16/f16 "128+q" / "1024+q"
//                    patterns with one AND-OR per pair (exact small integers), fed to
//                    v_mfma_f32_16x16x32 against x, and the zero point is removed per
//                    128-k block with a row sum of x that a second MFMA against an
//                    all-ones operand produces in the same C layout:
//                       sum_k x (q - z) s = s * (sum_k x (off + q) - (off + z) sum_k x).
//                    For M > 16 the 16-row groups of x take turns against the weights,
//                    which stay in registers (W is read once for all of M).
//   (16 < M <= 64 with group 128 and at most 256 workgroups of 32 x 48: int4_gemm_skinny_kernel;
//    M >= 64, or 16 < M < 64 with K > 4096, 16-bit activations, K % 64 == 0:
//    int4_gemm_tiled_kernel; both in int4_gemm.hip)
//   int4_gemm_mfma   other M > 16.  LDS-tiled: a 128x128 tile of W is dequantized once per
//                    workgroup to bf16 ((q - z) * s rounded to bf16, the reference's
//                    dequant numerics) next to a 128x128 tile of x, and 4 waves run
//                    v_mfma_f32_32x32x16_bf16 on it.
//   int4_linear_generic  any dtype / group / alignment; VALU, one wave per output row.
#include <stdlib.h>

#include <type_traits>

#include "common.hpp"
#include "int4_frag.hpp"
#include "int4_gemm.hpp"

namespace anna {
namespace {

constexpr uint32_t OOB = 0x80000000u;  // buffer offset past any num_records: the load returns 0

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// ------------------------------------------------------------------ GEMV (M <= 16)

// K blocks (128 k each) one wave keeps in flight per pass (BPW, a template parameter: 8, or 4
// when the K split over the waves leaves at most 4 per wave): all of them are loaded before any
// is consumed, so a wave has BPW x 16 B x NT per lane outstanding.  Loads past the wave's share
// would be clamped duplicates that still cost registers, hence BPW = 4 when 4 suffice: it lets
// two 8-wave workgroups share a CU.

// x is read through L1/L2 (staging it in LDS first was measured slower at every M).
// MG > 1 (M up to 16 MG, one pass per wave only): the wave's weights stay in registers and the
// 16-row groups of x take turns against them, so W is read from memory once for all of M.
template <int XDT, int SDT, int NT, int KW, int GEMV_BPW, int MG = 1>
__global__ __launch_bounds__(64 * KW) void int4_gemv_mfma(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t xs,
    const uint32_t* __restrict__ qw, int64_t N, int64_t pc,
    const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz,
    int64_t blocks_per_group, uint16_t* __restrict__ y, int contiguous, int nontemporal) {
  constexpr float OFF = XDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
  constexpr uint32_t ONES = XDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int kq = lane >> 4;
  const int64_t n_base = xcd_tile(blockIdx.x, gridDim.x) * (16 * NT);
  const int64_t nblk = (K + 127) >> 7;
  const u32x4 ones = {ONES, ONES, ONES, ONES};
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  const bool bpg1 = blocks_per_group == 1;

  const uint32_t* wrow[NT];
  bool n_ok[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n_base + t * 16 + r;
    n_ok[t] = n < N;
    wrow[t] = qw + (n_ok[t] ? n : 0) * pc + kq * 4;
  }

  f32x4 out[MG][NT];
#pragma unroll
  for (int g = 0; g < MG; ++g)
#pragma unroll
    for (int t = 0; t < NT; ++t) out[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Block j of a pass: interleaved (b = p0 + wave + KW*j) or contiguous per wave
  // (b = p0 + wave*BPW + j, so one wave reads whole 128 B lines back to back).
  const int64_t bw0 = contiguous ? (int64_t)wave * GEMV_BPW : wave;
  const int64_t bstep = contiguous ? 1 : KW;
  // One pass = GEMV_BPW blocks per wave (one pass covers K = 4096 at 8 waves).
  // Buffer loads: lanes of padding rows (row >= M) and past K take an offset beyond the
  // buffer and read 0 without touching memory (a clamped load plus a select had fetched a real
  // row for them: at M = 8, x traffic through L1 exceeded the weights').  The host keeps the
  // buffer below 2^31 bytes.
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)(((M - 1) * xs + K) * 2));
  auto load_x = [&](int64_t b, int s, int g) -> u32x4 {
    const int64_t k = b * 128 + kq * 32 + s * 8;
    const int64_t row = 16 * g + r;
    const bool ok = b < nblk && row < M && k < K;
    const uint32_t off = ok ? (uint32_t)((row * xs + k) * 2) : OOB;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
  };
  // With 4 blocks per wave and pass, the x fragments of all of them are loaded first (64
  // VGPRs): a fragment fetched one block ahead was sunk by the compiler next to its use, and
  // each block then waited a full round trip for x.
  // Several row groups (MG > 1): the x fragments of the next block are fetched while the
  // current block computes instead (half the registers), pinned ahead of the MFMAs by a
  // scheduling barrier, so that three 16-row tiles per wave still fit without spills.
  constexpr bool XALL = GEMV_BPW <= 4 && MG == 1;
  static_assert(MG == 1 || GEMV_BPW <= 4, "several row groups need the 4-block pass");
  auto pass = [&](int64_t p0) {
    u32x4 xall[XALL ? GEMV_BPW : 1][4];
    if constexpr (XALL) {
#pragma unroll
      for (int j = 0; j < GEMV_BPW; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) xall[j][s] = load_x(p0 + bw0 + bstep * j, s, 0);
    }
    // Issue every global load of the pass up front: weights, scales, zero points.
    u32x4 wv[GEMV_BPW][NT];
    float scv[GEMV_BPW][NT];
    float cv[GEMV_BPW][NT];
    // Loads are unconditional (addresses clamped into range, results selected after):
    // predicated loads would split the pass into branches with a full vmcnt wait each.
#pragma unroll
    for (int j = 0; j < GEMV_BPW; ++j) {
      const int64_t b = p0 + bw0 + bstep * j;
      const int64_t bc = b < nblk ? b : nblk - 1;
      // 32-bit (K / 128 < 2^31 here), and none at all for 128-wide groups: a 64-bit division
      // is ~100 instructions in front of each block's loads
      const int64_t g = bpg1 ? bc : (int64_t)((uint32_t)bc / (uint32_t)blocks_per_group);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t gi = g * N + (n_ok[t] ? n_base + t * 16 + r : 0);
        const u32x4* src = (const u32x4*)(wrow[t] + bc * 16);
        wv[j][t] = nontemporal ? __builtin_nontemporal_load(src) : *src;
        scv[j][t] = Elem<SDT>::load(qs, gi);
        cv[j][t] = (float)qz[gi];
      }
    }
#pragma unroll
    for (int j = 0; j < GEMV_BPW; ++j)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (!n_ok[t]) wv[j][t] = zero4;
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) {
      if (mg > 0 && 16 * mg >= M) break;
      // otherwise the x fragments of the next block are fetched while the current block computes
      u32x4 xa[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) xa[s] = XALL ? xall[0][s] : load_x(p0 + bw0, s, mg);
#pragma unroll
      for (int j = 0; j < GEMV_BPW; ++j) {
        const int64_t b = p0 + bw0 + bstep * j;
        if (b >= nblk) break;
        u32x4 xn[4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
          xn[s] = j + 1 < GEMV_BPW ? (XALL ? xall[j + 1 < GEMV_BPW ? j + 1 : 0][s] : load_x(b + bstep, s, mg)) : zero4;
        if constexpr (MG > 1) __builtin_amdgcn_sched_barrier(0);
        f32x4 acc[NT];
        f32x4 sx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const u32x4 a = interleave_x(xa[s]);
          sx = mfma16<XDT>(a, ones, sx);
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[t] = mfma16<XDT>(a, nibbles_to_frag<XDT>(wv[j][t][s]), acc[t]);
        }
        // C layout: lane holds rows m = 16 mg + 4 kq + i of column n = n_base + 16t + r.
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const float c = OFF + cv[j][t];
#pragma unroll
          for (int i = 0; i < 4; ++i) out[mg][t][i] = fmaf(scv[j][t], acc[t][i] - c * sx[i], out[mg][t][i]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) xa[s] = xn[s];
      }
    }
  };
  for (int64_t p0 = 0; p0 < nblk; p0 += (int64_t)KW * GEMV_BPW) pass(p0);

#pragma unroll
  for (int mg = 0; mg < MG; ++mg) {
    if (16 * mg >= M) break;
    if constexpr (KW > 1) {
      __shared__ float red[KW - 1][NT * 4][64];
      if (mg > 0) __syncthreads();  // wave 0 is done reading the previous group's sums
      if (wave > 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) red[wave - 1][t * 4 + i][lane] = out[mg][t][i];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w = 0; w < KW - 1; ++w)
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) out[mg][t][i] += red[w][t * 4 + i][lane];
      }
    }
    if (wave == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t n = n_base + t * 16 + r;
        if (!n_ok[t]) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t m = 16 * mg + 4 * kq + i;
          if (m < M) y[m * N + n] = Elem<XDT>::cvt(out[mg][t][i]);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ GEMV, VALU dot2 (M <= 2)
//
// Streaming kernel for the bandwidth-critical M = 1..2 case.  A load instruction covers
// 64/LPR rows x (LPR x 16 B) contiguous bytes of each (whole 128 B lines).  Wave w of a
// workgroup owns the k-slice [w*LPR*32, (w+1)*LPR*32) of RW = 4 RG rows; a lane keeps its 32 x
// values in registers (loaded first, so they never wait behind weights) and walks RG row
// groups whose loads are all issued up front (RG = 4, or 2 where four would leave fewer than
// three workgroups per compute unit).  Per 8 nibbles: 7 ALU ops build the bf16
// pairs (128+q_i, 128+q_{i+4}) and 4 v_dot2c_f32_bf16 accumulate; per 32 k the zero point
// and scale are applied as s * (acc - (128 + z) * sum(x)).  Lanes of a row and the waves of
// the workgroup are reduced at the end.


template <int XDT>
__device__ __forceinline__ float sum8_16bit(u32x4 v) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = v[i];
    if constexpr (XDT == ANNA_MI_BF16) {
      s += __uint_as_float(w << 16) + __uint_as_float(w & 0xFFFF0000u);
    } else {
      s += f16_bits_to_f32((uint16_t)(w & 0xFFFFu)) + f16_bits_to_f32((uint16_t)(w >> 16));
    }
  }
  return s;
}

constexpr int DOT2_MAX_WAVES = 16;

// v_mov_b32 with a DPP lane pattern (all rows and banks enabled).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Lane (sub, c) of a wave: c = lane % 16 owns k [k0 + 32 c, k0 + 32 c + 32) of the wave's
// 512-k slice, sub = lane / 16 the rows n0 + RG sub + g of its RG (1, 2 or 4) row groups g.  One
// load instruction (fixed g) covers 4 rows x 256 contiguous bytes; a lane's RG rows are
// consecutive, so its scales and zero points are one load each (RG x 2 or 4 bytes, RG bytes).  Every load of a slice is issued before any value is converted: a conversion
// placed right after its load made the compiler wait for that load before issuing the next.
template <int XDT, int SDT, int MR, int WMAX, bool VEC_SZ, int RG>
__global__ __launch_bounds__(64 * WMAX) void int4_gemv_dot2(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t xs,
    const uint32_t* __restrict__ qw, int64_t N, int64_t pc,
    const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz,
    int gshift, uint16_t* __restrict__ y) {
  static_assert(RG == 1 || RG == 2 || RG == 4, "row groups (loads of W) per lane and slice");
  constexpr int RW = 4 * RG;    // rows per workgroup
  constexpr int KSL = 512;      // k per wave slice
  constexpr float OFF = XDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
  constexpr uint32_t ONES = XDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr int SB = (int)sizeof(typename Elem<SDT>::T);
  const int lane = threadIdx.x & 63;
  const int wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kw = blockDim.x >> 6;
  const int sub = lane >> 4, c = lane & 15;
  const int64_t n0 = xcd_tile(blockIdx.x, gridDim.x) * RW;
  const int64_t G = (K + (1 << gshift) - 1) >> gshift;
  // Weight rows of this workgroup; rows >= N fall outside num_records and read 0.
  const int64_t rows_here = N - n0 < RW ? N - n0 : RW;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(qw + n0 * pc, (uint32_t)(rows_here * pc * 4));
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(qs, (uint32_t)(G * N * SB));
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(qz, (uint32_t)(G * N));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)(((M - 1) * xs + K) * 2));
  // VEC_SZ: one vector load of a lane's 4 scales / zero points (N % 4 == 0: 4-row aligned rows)

  float yacc[MR][RG];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int g = 0; g < RG; ++g) yacc[m][g] = 0.f;

  // x of a pass (kw * 512 k) is staged in LDS once per workgroup, already in nibble-pair order,
  // with the sum of every 32-k chunk (the zero-point term): thread t loads x[8 t .. 8 t + 7].
  __shared__ u32x4 s_x[MR][64 * WMAX];
  __shared__ float s_xsum[MR][16 * WMAX];
  auto pass = [&](int64_t p0) {
    const int64_t k0 = p0 + (int64_t)wave * KSL;
    const int64_t kl = k0 + c * 32;
    const bool k_ok = kl < K;
    u32x4 xg[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const int64_t kx = p0 + 8 * (int64_t)threadIdx.x;
      const uint32_t xo = (kx < K && m < M) ? (uint32_t)((m * xs + kx) * 2) : OOB;
      xg[m] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0));
    }
    // scales and zero points (small, ahead of the weights they scale), kept raw
    const int64_t grp = k_ok ? kl >> gshift : 0;
    const uint32_t so = k_ok ? (uint32_t)(grp * N + n0 + RG * sub) : OOB / 4;
    u32x4 svec = {0u, 0u, 0u, 0u};
    uint32_t zvec = 0, sg[RG], zg[RG];
    if constexpr (VEC_SZ) {
      // RG consecutive scales (RG * 2 or RG * 4 bytes) and zero points (RG bytes)
      if constexpr (RG * SB == 16) {
        svec = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, so * SB, 0, 0));
      } else if constexpr (RG * SB == 8) {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, so * SB, 0, 0));
        svec.x = v.x, svec.y = v.y;
      } else if constexpr (RG * SB == 4) {
        svec.x = __builtin_amdgcn_raw_buffer_load_b32(rs, so * SB, 0, 0);
      } else {
        svec.x = __builtin_amdgcn_raw_buffer_load_b16(rs, so * SB, 0, 0);
      }
      if constexpr (RG == 4) zvec = __builtin_amdgcn_raw_buffer_load_b32(rz, so, 0, 0);
      else if constexpr (RG == 2) zvec = __builtin_amdgcn_raw_buffer_load_b16(rz, so, 0, 0);
      else zvec = __builtin_amdgcn_raw_buffer_load_b8(rz, so, 0, 0);
    } else {
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        sg[g] = SDT == ANNA_MI_F32 ? __builtin_amdgcn_raw_buffer_load_b32(rs, so * 4, g * 4, 0)
                                   : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, so * 2, g * 2, 0);
        zg[g] = __builtin_amdgcn_raw_buffer_load_b8(rz, so, g, 0);
      }
    }
    // weights with the non-temporal hint (cache policy 2): the default policy measured 7.5 against
    // 7.06 us at M = 1, N = 12288, K = 4096; adding sc0 or sc1 changed nothing beyond noise
    u32x4 wv[RG];
    const uint32_t wo = k_ok ? (uint32_t)((RG * sub * pc + (kl >> 3)) * 4) : OOB;
#pragma unroll
    for (int g = 0; g < RG; ++g)
      wv[g] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rw, wo, (int)(g * pc * 4), 2 /* slc: streamed once */));
    __builtin_amdgcn_sched_barrier(0);
    if (p0 > 0) __syncthreads();  // the previous pass is done reading s_x
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const u32x4 iv = interleave_x(xg[m]);
      s_x[m][threadIdx.x] = iv;
      float t = dot2_acc<XDT>(iv.x, ONES, 0.f);
      t = dot2_acc<XDT>(iv.y, ONES, t);
      t = dot2_acc<XDT>(iv.z, ONES, t);
      t = dot2_acc<XDT>(iv.w, ONES, t);
      t += dpp_f32<0xB1>(t);  // quad_perm [1, 0, 3, 2]
      t += dpp_f32<0x4E>(t);  // quad_perm [2, 3, 0, 1]
      if ((threadIdx.x & 3) == 0) s_xsum[m][threadIdx.x >> 2] = t;
    }
    __syncthreads();
    uint32_t sraw[RG];
    uint32_t zraw = 0;
    if constexpr (VEC_SZ) {
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        if constexpr (SDT == ANNA_MI_F32) sraw[g] = svec[g];
        else sraw[g] = svec[g >> 1] >> (16 * (g & 1));
      }
      zraw = zvec;
    } else {
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        sraw[g] = sg[g];
        zraw |= (zg[g] & 0xFFu) << (8 * g);
      }
    }
    float sc[RG], cz[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      if constexpr (SDT == ANNA_MI_F32) sc[g] = __uint_as_float(sraw[g]);
      else if constexpr (SDT == ANNA_MI_BF16) sc[g] = __uint_as_float(sraw[g] << 16);
      else sc[g] = f16_bits_to_f32((uint16_t)(sraw[g] & 0xFFFFu));
      cz[g] = OFF + (float)(int8_t)(zraw >> (8 * g));
    }
    // this lane's 32 k: threads 4 (16 wave + c) .. + 3 of the staging
    const int xi = 4 * (16 * wave + c);
    uint32_t xp[MR][16];
    float sx[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const u32x4 iv = s_x[m][xi + s4];
        xp[m][s4 * 4 + 0] = iv.x;
        xp[m][s4 * 4 + 1] = iv.y;
        xp[m][s4 * 4 + 2] = iv.z;
        xp[m][s4 * 4 + 3] = iv.w;
      }
      sx[m] = s_xsum[m][16 * wave + c];
    }
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      float acc[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const u32x4 f = nibbles_to_frag<XDT>(wv[g][s4]);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          acc[m] = dot2_acc<XDT>(xp[m][s4 * 4 + 0], f.x, acc[m]);
          acc[m] = dot2_acc<XDT>(xp[m][s4 * 4 + 1], f.y, acc[m]);
          acc[m] = dot2_acc<XDT>(xp[m][s4 * 4 + 2], f.z, acc[m]);
          acc[m] = dot2_acc<XDT>(xp[m][s4 * 4 + 3], f.w, acc[m]);
        }
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) yacc[m][g] = fmaf(sc[g], fmaf(-cz[g], sx[m], acc[m]), yacc[m][g]);
    }
  };
  // one pass covers K when the workgroup has enough waves (the common case): straight-line code
  if (K <= (int64_t)kw * KSL) {
    pass(0);
  } else {
    for (int64_t p0 = 0; p0 < K; p0 += (int64_t)kw * KSL) pass(p0);
  }
  // Reduce-scatter over the 16 lanes of a DPP row (the lanes c of one sub): each stage pairs a
  // lane with one whose bit b of c differs (row_mirror flips bit 3, row_half_mirror bit 2, quad
  // permutations bits 1 and 0), keeps the half of the list that bit selects and adds the
  // partner's copy of it.  Afterwards lane c holds row group (c >> 3 & 1) * 2 + (c >> 2 & 1)
  // summed over the row.
  float red_v[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float v[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) v[g] = g < RG ? yacc[m][g] : 0.f;
    // with fewer row groups the first stages add the whole list instead of halving it
    if constexpr (RG == 4) {
      const bool up = (c >> 3) & 1;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float mine = up ? v[i + 2] : v[i], give = up ? v[i] : v[i + 2];
        v[i] = mine + dpp_f32<0x140>(give);  // row_mirror
      }
    } else if constexpr (RG == 2) {
      const bool up = (c >> 3) & 1;
      const float mine = up ? v[1] : v[0], give = up ? v[0] : v[1];
      v[0] = mine + dpp_f32<0x140>(give);  // row_mirror
    } else {
      v[0] += dpp_f32<0x140>(v[0]);
    }
    if constexpr (RG == 4) {
      const bool up = (c >> 2) & 1;
      const float mine = up ? v[1] : v[0], give = up ? v[0] : v[1];
      v[0] = mine + dpp_f32<0x141>(give);  // row_half_mirror
    } else {
      v[0] += dpp_f32<0x141>(v[0]);
    }
    v[0] += dpp_f32<0x4E>(v[0]);  // quad_perm [2, 3, 0, 1]
    v[0] += dpp_f32<0xB1>(v[0]);  // quad_perm [1, 0, 3, 2]
    red_v[m] = v[0];
  }
  // the row group lane c holds: bits 3 and 2 of c for four groups, bit 3 for two
  const int gsel = RG == 4 ? ((c >> 3) & 1) * 2 + ((c >> 2) & 1) : RG == 2 ? (c >> 3) & 1 : 0;
  __shared__ float red[WMAX][MR][RW];
  if ((c & (RG == 4 ? 3 : RG == 2 ? 7 : 15)) == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave][m][RG * sub + gsel] = red_v[m];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < MR * RW; i += blockDim.x) {
    const int m = i / RW, row = i % RW;
    float v = 0.f;
    for (int w = 0; w < kw; ++w) v += red[w][m][row];
    const int64_t n = n0 + row;
    if (m < M && n < N) y[m * N + n] = Elem<XDT>::cvt(v);
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

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return (v && *v) ? atoi(v) : dflt;
}
// ANNA_MI_INT4_GEMV_CONTIG / ANNA_MI_INT4_GEMV_NT: block order and nontemporal weight loads.
static const int g_contig = env_int("ANNA_MI_INT4_GEMV_CONTIG", 0);
static const int g_nt = env_int("ANNA_MI_INT4_GEMV_NT", 1);

template <int XDT, int SDT, int NT, int KW, int BPW, int MG = 1>
void launch_gemv(const void* x, int64_t M, int64_t K, int64_t xs, const int32_t* qw, int64_t N,
                 int64_t pc, const void* qs, const int8_t* qz, int64_t gsz, void* y, hipStream_t st) {
  dim3 grid((unsigned)((N + 16 * NT - 1) / (16 * NT)), 1, 1);
  hipLaunchKernelGGL((int4_gemv_mfma<XDT, SDT, NT, KW, BPW, MG>), grid, dim3(64 * KW), 0, st, (const uint16_t*)x, M, K, xs,
                     (const uint32_t*)qw, N, pc, (const typename Elem<SDT>::T*)qs, qz, gsz / 128, (uint16_t*)y,
                     g_contig, g_nt);
}

// Tuning knobs (read once): ANNA_MI_INT4_GEMV_WAVES in {4, 8} splits K across that many
// waves per workgroup; ANNA_MI_INT4_GEMV_TILES in {1, 2, 3, 4} sets 16-row tiles per wave.
// Default tiles: the fewest that put the whole N in one workgroup per compute unit (every
// wave's loads then go out in a single round), e.g. 3 at N = 12288 (256 workgroups; 12.8 us at
// M = 8 against 14.5 us for 384 two-tile workgroups) and 2 at N = 6144; 2 past 256 x 48 rows.

template <int XDT, int SDT>
void dispatch_gemv(const void* x, int64_t M, int64_t K, int64_t xs, const int32_t* qw, int64_t N, int64_t pc,
                   const void* qs, const int8_t* qz, int64_t gsz, void* y, hipStream_t st) {
  static const int env_waves = env_int("ANNA_MI_INT4_GEMV_WAVES", 0);
  static const int env_tiles = env_int("ANNA_MI_INT4_GEMV_TILES", 0);
  const int64_t nblk = (K + 127) / 128;
  const int waves = env_waves ? env_waves : (nblk >= 32 ? 8 : 4);
  int tiles = 2;
  for (int t = 1; t <= 3; ++t)
    if ((N + 16 * t - 1) / (16 * t) <= 256) {
      tiles = t;
      break;
    }
  if (env_tiles) tiles = env_tiles;
  const bool b4 = nblk <= 4 * waves;  // one pass of 4 blocks per wave covers K
#define ANNA_GEMV_GO(T, W)                                                                   \
  (b4 ? launch_gemv<XDT, SDT, T, W, 4>(x, M, K, xs, qw, N, pc, qs, qz, gsz, y, st)           \
      : launch_gemv<XDT, SDT, T, W, 8>(x, M, K, xs, qw, N, pc, qs, qz, gsz, y, st))
  if (waves == 8 && tiles == 3) ANNA_GEMV_GO(3, 8);
  else if (waves == 8 && tiles == 4) ANNA_GEMV_GO(4, 8);
  else if (waves == 8 && tiles == 2) ANNA_GEMV_GO(2, 8);
  else if (waves == 8) ANNA_GEMV_GO(1, 8);
  else if (tiles >= 3) ANNA_GEMV_GO(3, 4);
  else if (tiles == 2) ANNA_GEMV_GO(2, 4);
  else ANNA_GEMV_GO(1, 4);
#undef ANNA_GEMV_GO
}

// 16 < M <= 64 with one 4-block pass per wave (K <= 128 x 4 x waves): the GEMV with MG row
// groups of x against the register-resident weights (W read once).
template <int XDT, int SDT>
void dispatch_gemv_mg(const void* x, int64_t M, int64_t K, int64_t xs, const int32_t* qw, int64_t N, int64_t pc,
                      const void* qs, const int8_t* qz, int64_t gsz, void* y, hipStream_t st) {
  const int64_t nblk = (K + 127) / 128;
  const bool w8 = nblk > 16;
  int tiles = 3;
  for (int t = 1; t <= 3; ++t)
    if ((N + 16 * t - 1) / (16 * t) <= 256) {
      tiles = t;
      break;
    }
  const bool mg2 = M <= 32;
#define ANNA_GEMV_MG(T)                                                                        \
  (w8 ? (mg2 ? launch_gemv<XDT, SDT, T, 8, 4, 2>(x, M, K, xs, qw, N, pc, qs, qz, gsz, y, st)      \
             : launch_gemv<XDT, SDT, T, 8, 4, 4>(x, M, K, xs, qw, N, pc, qs, qz, gsz, y, st))     \
      : (mg2 ? launch_gemv<XDT, SDT, T, 4, 4, 2>(x, M, K, xs, qw, N, pc, qs, qz, gsz, y, st)      \
             : launch_gemv<XDT, SDT, T, 4, 4, 4>(x, M, K, xs, qw, N, pc, qs, qz, gsz, y, st)))
  if (tiles == 1) ANNA_GEMV_MG(1);
  else if (tiles == 2) ANNA_GEMV_MG(2);
  else ANNA_GEMV_MG(3);
#undef ANNA_GEMV_MG
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
  const bool gsz_pow2 = gsz >= 32 && (gsz & (gsz - 1)) == 0;
  if (x16 && aligned && M <= 2 && K % 32 == 0 && gsz_pow2) {
    const int gshift = __builtin_ctzll((unsigned long long)gsz);
    const int64_t ksl = 16 * 32;
    int64_t waves = (K + ksl - 1) / ksl;
    waves = waves > DOT2_MAX_WAVES ? DOT2_MAX_WAVES : waves;
    ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
      auto go = [&](auto xdt_tag, auto mr_tag) {
        constexpr int XDT = decltype(xdt_tag)::value, MR = decltype(mr_tag)::value;
        dim3 grid((unsigned)((N + 15) / 16));
        // 8-wave bound where K allows: a 1024-thread bound and LDS sized for 16 waves cost
        // registers at K = 4096
        auto launch = [&](auto kern) {
          hipLaunchKernelGGL(kern, grid, dim3((unsigned)(64 * waves)), 0, st, (const uint16_t*)x, M, K, xs,
                             (const uint32_t*)qweight, N, pc, (const typename Elem<SDT>::T*)qscale, qzeros, gshift,
                             (uint16_t*)y);
        };
        const bool vec = (N & 3) == 0;
        // four row groups per lane while that still gives three workgroups per compute unit, else
        // two (twice the waves, half the chain per wave): M = 1, N = 6144, K = 2048 3.93 -> 3.72 us,
        // K = 4096 5.25 -> 5.03 us; N = 12288 stays at four (6.8 against 7.8 us with two); one row
        // group per lane measured 3.86 / 5.89 us at N = 6144 (two: 3.74 / 4.83).
        // ANNA_MI_INT4_DOT2_RG = 1 / 2 / 4 forces a count (read on every call, for the tests).
        int rg = (N + 15) / 16 >= 768 ? 4 : 2;
        if (const char* f = getenv("ANNA_MI_INT4_DOT2_RG"); f && (f[0] == '1' || f[0] == '2' || f[0] == '4'))
          rg = f[0] - '0';
        auto go_rg = [&](auto rg_tag) {
          constexpr int RG = decltype(rg_tag)::value;
          grid = dim3((unsigned)((N + 4 * RG - 1) / (4 * RG)));
          if (waves <= 8) {
            if (vec) launch(int4_gemv_dot2<XDT, SDT, MR, 8, true, RG>);
            else launch(int4_gemv_dot2<XDT, SDT, MR, 8, false, RG>);
          } else {
            if (vec) launch(int4_gemv_dot2<XDT, SDT, MR, DOT2_MAX_WAVES, true, RG>);
            else launch(int4_gemv_dot2<XDT, SDT, MR, DOT2_MAX_WAVES, false, RG>);
          }
        };
        if (rg == 1) go_rg(std::integral_constant<int, 1>{});
        else if (rg == 2) go_rg(std::integral_constant<int, 2>{});
        else go_rg(std::integral_constant<int, 4>{});
      };
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using XB = std::integral_constant<int, ANNA_MI_BF16>;
      using XH = std::integral_constant<int, ANNA_MI_F16>;
      if (x_dtype == ANNA_MI_BF16) { if (M == 1) go(XB{}, I1{}); else go(XB{}, I2{}); }
      else { if (M == 1) go(XH{}, I1{}); else go(XH{}, I2{}); }
    });
    ANNA_LAUNCH_CHECK("int4_gemv_dot2");
    return ANNA_MI_OK;
  }
  const bool x31 = ((M - 1) * xs + K) * 2 < ((int64_t)1 << 31);  // x fits one buffer resource
  if (x16 && aligned && x31 && M <= 16) {
    ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
      if (x_dtype == ANNA_MI_BF16)
        dispatch_gemv<ANNA_MI_BF16, SDT>(x, M, K, xs, qweight, N, pc, qscale, qzeros, gsz, y, st);
      else
        dispatch_gemv<ANNA_MI_F16, SDT>(x, M, K, xs, qweight, N, pc, qscale, qzeros, gsz, y, st);
    });
    ANNA_LAUNCH_CHECK("int4_gemv_mfma");
    return ANNA_MI_OK;
  }
  // 16 < M <= 64 (group 128, K a multiple of 1024) when its workgroups (32 rows of x x 48 rows of
  // W each) fit one round of the chip: the skinny GEMM.  M = 64, K = 4096: N = 6144 (256
  // workgroups) 14.5 us against 19.1 for the tiled GEMM; N = 12288 (512) 27 against 22.3, so
  // larger grids stay with the tiled GEMM / the row-group GEMV.  ANNA_MI_INT4_SKINNY_MMAX moves
  // the upper bound of M (0 turns the skinny GEMM off).
  static const int skinny_mmax = env_int("ANNA_MI_INT4_SKINNY_MMAX", 64);
  if (x16 && M > 16 && M <= skinny_mmax && int4_gemm_skinny_workgroups(M, N) <= 256 &&
      int4_gemm_skinny_supported(x_dtype, M, N, K, xs, x, qweight, pc, gsz))
    return int4_gemm_skinny_launch(x, x_dtype, M, K, xs, qweight, N, pc, qscale, scale_dtype, qzeros, y, st);
  // 16 < M < 64: the GEMV with 16-row groups of x against register-resident weights (M = 17..48
  // at N = 12288, K = 4096: 24-35 us, where the LDS-tiled fallback below took ~145 us); from
  // M = 64 the tiled GEMM is faster (27.6 against 46 us at M = 64)
  if (x16 && aligned && x31 && M < 64 && (K + 127) / 128 <= 32) {
    ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
      if (x_dtype == ANNA_MI_BF16)
        dispatch_gemv_mg<ANNA_MI_BF16, SDT>(x, M, K, xs, qweight, N, pc, qscale, qzeros, gsz, y, st);
      else
        dispatch_gemv_mg<ANNA_MI_F16, SDT>(x, M, K, xs, qweight, N, pc, qscale, qzeros, gsz, y, st);
    });
    ANNA_LAUNCH_CHECK("int4_gemv_mfma (row groups)");
    return ANNA_MI_OK;
  }
  if (int4_gemm_tiled_supported(x_dtype, M, N, K, xs, x, qweight, pc, qscale, qzeros, gsz))
    return int4_gemm_tiled_launch(x, x_dtype, M, K, xs, qweight, N, pc, qscale, scale_dtype, qzeros, gsz, y, st);
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
