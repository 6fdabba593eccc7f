// W4A16 GEMM for M >= 64 (and 16 < M < 64 with long K) on gfx950: y[M, N] = x[M, K] . dequant(W)[N, K]^T.
//
// Tile 256 (m) x 192 (n) x 64 (k) per workgroup of 12 waves with two roles (for M >= 1024; the
// same kernel runs 128 x 96 tiles with a 4 x 2 grid of MFMA waves for M >= 256 and 64 x 48 with
// 4 x 1 below, so that every compute unit gets a workgroup):
//   8 MFMA waves   a 2 x 4 grid, each owning 128 x 48 of C as 8 x 3 v_mfma_f32_16x16x32
//                  accumulators; they only read LDS;
//   4 loader waves (one per SIMD) copy the x tile (256 x 64, 16-bit) straight from memory into
//                  LDS (buffer loads with the LDS destination, two k-steps ahead, three
//                  buffers), and load the int4 words of W (192 rows x 64 k) two steps ahead into
//                  registers, dequantize them to (q - z) * s in fp32 rounded to the activation
//                  dtype (the reference's dequant numerics, quantization.py:626-648) and write
//                  them to the LDS buffer of the next step (two buffers).
// The two roles run between the same barriers (one per k-step), so each SIMD issues the
// loaders' VALU work while its MFMA waves keep the matrix core busy.  LDS rows are 64 elements
// (128 B) with the 16-byte chunk c of row r stored at slot c ^ (r & 7): the 16 lanes of an MFMA
// operand read (16 consecutive rows, one chunk) then touch 8 distinct slots per 8 rows, and an
// 8-row block is exactly the 1 KB one wave-wide LDS-destination load writes.  The tile ->
// workgroup map is XCD-aware and m-major: the n-tiles of one m-tile share one XCD, so that XCD's
// L2 holds the m-tile's slice of x (256 x K, 2 MB at K = 4096) and only the small int4 W streams
// in; M = 2048 with N = 12288 gives 512 tiles (two rounds on 256 CUs).
#include <stdlib.h>

#include <type_traits>

#include "common.hpp"
#include "int4_frag.hpp"
#include "int4_gemm.hpp"

namespace anna {
namespace {

constexpr int GM_BK = 64, GM_LOAD_WAVES = 4;
constexpr int GM_LT = 64 * GM_LOAD_WAVES;  // loader threads

constexpr uint32_t GM_OOB = 0x80000000u;   // buffer offset past any num_records: the load returns 0

// Tile shape: BM x BN per workgroup, an MW x NW grid of MFMA waves (wave tile BM/MW x BN/NW),
// SPB k-steps of 64 between two workgroup barriers (a "period"): the smallest tile, whose steps
// hold little MFMA work, pays the barrier and its waits once per two steps.  LDS holds x for
// three periods (the one read, the one landing, the one being loaded) and W for two.
// KS_ = 2: the workgroup holds two such sets of waves (and LDS), each over half of K; the halves
// meet at the same barriers, and the second hands its accumulators to the first at the end.
template <int BM_, int BN_, int MW_, int NW_, int SPB_ = 1, int KS_ = 1>
struct GemmTile {
  static constexpr int BM = BM_, BN = BN_, MW = MW_, NW = NW_, SPB = SPB_, KS = KS_;
  static constexpr int NA = 3 * SPB, NB = 2 * SPB;  // LDS buffers (one k-step each) of x and of W
  static constexpr int MFMA_WAVES = MW * NW, HALF_WAVES = MFMA_WAVES + GM_LOAD_WAVES, THREADS = 64 * KS * HALF_WAVES;
  static constexpr int TM = BM / MW, TN = BN / NW, FM = TM / 16, FN = TN / 16;  // wave tile, fragments
  static constexpr int LDS_A = BM * GM_BK, LDS_B = BN * GM_BK;                   // 16-bit elements per buffer
  static constexpr size_t HALF_ELEMS = (size_t)(NA * LDS_A + NB * LDS_B);  // 16-bit elements of one half
  static constexpr size_t LDS_BYTES = KS * HALF_ELEMS * 2;
  static constexpr int XLD = BM / 8 / GM_LOAD_WAVES;           // 8-row x blocks per loader wave
  static constexpr int WPT = (BN * 4 + GM_LT - 1) / GM_LT;     // W chunks (8 B = 16 nibbles) per loader thread
  // vector-memory loads one loader thread issues per k-step: the x blocks plus word, scale and
  // zero point of each W chunk; the wait before each barrier keeps exactly these outstanding
  static constexpr int LOADS_PER_STEP = XLD + 3 * WPT;
  static_assert(TM % 16 == 0 && TN % 16 == 0 && BM % (8 * GM_LOAD_WAVES) == 0, "tile shape");
  static_assert(SPB == 1 || SPB == 2, "one or two k-steps per period");
  static_assert(KS == 1 || KS == 2, "one or two halves of K");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};
using TileL = GemmTile<256, 192, 2, 4, 1>;  // M >= 1024: 128 x 48 wave tiles, 144 KB LDS
using TileM = GemmTile<128, 96, 4, 2, 1>;   // M >= 256:  32 x 48 wave tiles, 72 KB LDS
using TileS = GemmTile<64, 48, 4, 1, 2>;    // M < 256:   16 x 48 wave tiles, 72 KB LDS, 2 steps per
                                            // period (M = 64, N = 12288: 25.6 -> 23.9 us; the 128 x 96
                                            // tile measured no faster with 2)
using TileM2 = GemmTile<128, 96, 2, 2, 1, 2>;  // TileM's tile with K split over two halves of a
                                               // 16-wave workgroup, 4 MFMA waves of 64 x 48 each
using TileS2 = GemmTile<64, 48, 4, 1, 2, 2>;  // TileS with K split over two halves of a 16-wave
                                              // workgroup (K a multiple of 256), 144 KB LDS

// The loader's end of a k-step: all but its N most recent loads have landed (so the previous
// step's LDS-destination x loads are in LDS), its LDS writes are done, then the workgroup
// barrier.  __syncthreads() would also wait for the loads just issued, since its release fence
// covers LDS-destination loads.  The scheduling barrier in front keeps the machine scheduler
// from moving any load of this step below the wait (a count-based wait is right only while
// every load it counts was issued before it).
template <int N>
__device__ __forceinline__ void loader_barrier() {
  static_assert(N >= 0 && N <= 63, "vmcnt holds 6 bits");
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"i"(N) : "memory");
}

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr;

template <int XDT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (XDT == ANNA_MI_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){lo, hi}, bf16x2v));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){lo, hi}, f16x2v));
  }
}

// element offset of 16-byte chunk c of row r in a swizzled 64-element-row LDS tile
__device__ __forceinline__ int swz(int r, int c) { return r * GM_BK + ((c ^ (r & 7)) << 3); }

template <int XDT, int SDT, class T>
__global__ __launch_bounds__(T::THREADS) void int4_gemm_tiled_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t xs, const uint32_t* __restrict__ qw, int64_t N,
    int64_t pc, const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz, int64_t gsz,
    uint16_t* __restrict__ y, int64_t tiles_m, int64_t tiles_n) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  using ST = typename Elem<SDT>::T;
  constexpr int GM_BM = T::BM, GM_BN = T::BN, GM_LDS_A = T::LDS_A, GM_LDS_B = T::LDS_B;
  constexpr int GM_MFMA_WAVES = T::MFMA_WAVES, GM_XLD = T::XLD, GM_WPT = T::WPT;
  constexpr int GM_NA = T::NA;
  const int lane = threadIdx.x & 63;
  // k-half of this wave (uniform), its wave and thread index within the half
  const int half = T::KS > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6) / T::HALF_WAVES) : 0;
  const int wave = (int)(threadIdx.x >> 6) - half * T::HALF_WAVES;
  const int tid = (int)threadIdx.x - 64 * T::HALF_WAVES * half;
  uint16_t* const sA0 = smem + half * T::HALF_ELEMS;  // GM_NA x buffers
  uint16_t* const sB0 = sA0 + GM_NA * GM_LDS_A;       // GM_NB W buffers
  // tile coordinates in 32-bit scalar registers: a value the compiler cannot prove uniform
  // would turn every buffer load below into a loop over distinct descriptors
  const int t = __builtin_amdgcn_readfirstlane((int)xcd_tile(blockIdx.x, tiles_m * tiles_n));
  const int tn32 = (int)tiles_n;
  const int64_t m0 = (int64_t)__builtin_amdgcn_readfirstlane((t / tn32) * GM_BM);
  const int64_t n0 = (int64_t)__builtin_amdgcn_readfirstlane((t % tn32) * GM_BN);
  const int nk = (int)(K / GM_BK) / T::KS;  // k-steps of this half (the launcher makes both equal)
  const int kb = half * nk;                  // its first k-step

  if (wave >= GM_MFMA_WAVES) {
    // ---------------- loader waves
    // Buffer loads: a per-lane 32-bit offset plus a uniform one; rows past M or N read as zero
    // (their products only reach rows / columns of C that are not stored).
    const int lw = __builtin_amdgcn_readfirstlane(wave - GM_MFMA_WAVES), lt = tid - 64 * GM_MFMA_WAVES;
    const int64_t rows_x = M - m0 < GM_BM ? M - m0 : GM_BM, rows_w = N - n0 < GM_BN ? N - n0 : GM_BN;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(x + m0 * xs), 0, (int)(rows_x * xs * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(qw + n0 * pc), 0, (int)(rows_w * pc * 4), 0x00020000);
    const int64_t G = (K + gsz - 1) / gsz;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<ST*>(qs + n0), 0, (int)((G * N - n0) * (int64_t)sizeof(ST)), 0x00020000);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(qz + n0), 0, (int)(G * N - n0), 0x00020000);
    // x: load j of this wave fills 8-row block b = 8 lw + j of the tile; lane l writes LDS slot
    // l % 8 of row 8 b + l / 8, which holds chunk (l % 8) ^ (l / 8) of that row
    const uint32_t xo = (uint32_t)((((lane >> 3) * xs) + (((lane & 7) ^ (lane >> 3)) << 3)) * 2);
    // W chunk i of this thread: row lt / 4 + 64 i, 16 k at (lt % 4) * 16 (LDS chunks 2 (lt % 4) and
    // 2 (lt % 4) + 1).  Chunks of rows past the tile (a tile narrower than 64 WPT rows) load
    // from an offset past the buffer (zero) and are not stored.
    uint32_t wo[GM_WPT], so[GM_WPT], zo[GM_WPT];
#pragma unroll
    for (int i = 0; i < GM_WPT; ++i) {
      const bool in_tile = (lt >> 2) + 64 * i < GM_BN;
      wo[i] = in_tile ? (uint32_t)(((lt >> 2) * pc + (lt & 3) * 2) * 4) : GM_OOB;
      so[i] = in_tile ? (uint32_t)((lt >> 2) * sizeof(ST)) : GM_OOB;
      zo[i] = in_tile ? (uint32_t)(lt >> 2) : GM_OOB;
    }
    // group of k-step ks = ks / (gsz / 64) as a multiply-high by ceil(2^32 / (gsz / 64)) (one
    // group per step needs no map): exact while both are below 2^16 (checked by the launcher);
    // a division here would branch and make the loads just issued wait
    const uint32_t spg = (uint32_t)(gsz / GM_BK);
    const uint32_t ginv = spg > 1 ? (uint32_t)(((1ull << 32) + spg - 1) / spg) : 0u;
    // the scale and zero point stay raw until the store: converting them at the load would
    // make the load wait for its data
    struct Stage {
      uint2 w[GM_WPT];
      uint32_t sc[GM_WPT], z[GM_WPT];
    };
    // Every step issues the same loads: the x tile of step ks + 2 and the W words, scales and
    // zero points of step ks + 3 (steps past the end reload the last one into a buffer nobody
    // reads), so a fixed vmcnt names "all but this step's loads".  W is issued a step earlier
    // than x because its dequant must finish within the step before the MFMAs use it.
    auto load_x = [&](int ks, int abuf) {
      ks = ks < nk ? ks : nk - 1;
      uint16_t* dst = sA0 + abuf * GM_LDS_A + lw * (GM_XLD * 8 * GM_BK);
#pragma unroll
      for (int j = 0; j < GM_XLD; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(dst + j * 8 * GM_BK), 16, xo,
                                                 (int)((8 * (GM_XLD * lw + j)) * xs * 2) + (kb + ks) * (GM_BK * 2), 0, 0);
    };
    auto load_w = [&](int ks, Stage& S) {
      ks = (ks < nk ? ks : nk - 1) + kb;
      const int g = spg == 1 ? ks : (int)__umulhi((uint32_t)ks, ginv);
#pragma unroll
      for (int i = 0; i < GM_WPT; ++i) {
        S.w[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                               rw, wo[i], (int)(i * 64 * pc * 4) + ks * (GM_BK / 2), 0));
        if constexpr (sizeof(ST) == 4)
          S.sc[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, so[i], (int)((g * N + 64 * i) * 4), 0);
        else
          S.sc[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, so[i], (int)((g * N + 64 * i) * 2), 0);
        S.z[i] = __builtin_amdgcn_raw_buffer_load_b8(rz, zo[i], (int)(g * N + 64 * i), 0);
      }
    };
    // (q - z) * s as fma(q + o - z, s, -o * s): q + o - z is a byte in [0, 255] (o = 128, or 0
    // for z < -112), so one v_add makes four of them; the fma rounds the exact (q - z) * s once,
    // as the reference's fp32 product does
    auto store = [&](const Stage& S, int bbuf) {
      uint16_t* sB = sB0 + bbuf * GM_LDS_B;
#pragma unroll
      for (int i = 0; i < GM_WPT; ++i) {
        float sc;
        if constexpr (sizeof(ST) == 4) sc = __uint_as_float(S.sc[i]);
        else sc = Elem<SDT>::to_f32((ST)S.sc[i]);
        const int z = (int)(int8_t)S.z[i];
        const int off = z < -112 ? 0 : 128;
        const uint32_t bias = (uint32_t)(off - z) * 0x01010101u;
        const float c = -(float)off * sc;
        const int row = (lt >> 2) + 64 * i;
        if (GM_WPT * 64 > GM_BN && row >= GM_BN) continue;
#pragma unroll
        for (int wi = 0; wi < 2; ++wi) {
          const uint32_t w = wi ? S.w[i].y : S.w[i].x;
          const uint32_t lo = (w & 0x0F0F0F0Fu) + bias, hi = ((w >> 4) & 0x0F0F0F0Fu) + bias;
          u32x4 o;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float a = __builtin_fmaf((float)((lo >> (8 * j)) & 0xFFu), sc, c);  // nibble 2j
            const float b = __builtin_fmaf((float)((hi >> (8 * j)) & 0xFFu), sc, c);  // nibble 2j + 1
            o[j] = pack2<XDT>(a, b);
          }
          *(u32x4*)(sB + swz(row, 2 * (lt & 3) + wi)) = o;
        }
      }
    };
    if constexpr (T::SPB == 1) {
      // prologue: W of steps 0..2 and x of steps 0..1; W of step 0 to LDS; barrier once x of
      // step 0 has landed.  The wait is for every load issued so far: the compiler is free to
      // sink the loads of W 2 below the barrier (their values are first used in the loop), and
      // then a count of "the loads after x 0" (W 1, x 1, W 2) would let x 0 still be in flight
      // while the MFMA waves read it.  (Inside the loop each step's loads stay ahead of its
      // barrier; the cost of waiting for everything here is paid once.)
      Stage S0, S1, S2;
      load_w(0, S0);
      load_x(0, 0);
      load_w(1, S1);
      load_x(1, 1);
      load_w(2, S2);
      store(S0, 0);
      loader_barrier<0>();
      // step ks: W of ks + 3 into the stage that held W of ks, x of ks + 2 into the x buffer read
      // at step ks - 1, dequantize W of ks + 1, barrier once x of ks + 1 has landed
      int a2 = 2, b1 = 1;  // x buffer of step ks + 2, W buffer of step ks + 1
      auto step = [&](int ks, Stage& Sfree, Stage& Snext) {
        load_w(ks + 3, Sfree);
        load_x(ks + 2, a2);
        a2 = a2 == GM_NA - 1 ? 0 : a2 + 1;
        if (ks + 1 < nk) store(Snext, b1);
        b1 ^= 1;
        loader_barrier<T::LOADS_PER_STEP>();
      };
      for (int ks = 0; ks < nk; ks += 3) {
        step(ks, S0, S1);
        if (ks + 1 >= nk) break;
        step(ks + 1, S1, S2);
        if (ks + 2 >= nk) break;
        step(ks + 2, S2, S0);
      }
    } else {
      // Two k-steps per period.  Step k's W lives in register stage k % 4, its x in LDS buffer
      // k % 6, its dequantized W in LDS buffer k % 4.  Period p: W and x of steps 2p+4, 2p+5
      // (two periods ahead), dequantize W of steps 2p+2, 2p+3, barrier once x of steps 2p+2,
      // 2p+3 (issued in the period before) has landed: all but this period's loads.
      Stage S0, S1, S2, S3;
      load_w(0, S0);
      load_w(1, S1);
      load_x(0, 0);
      load_x(1, 1);
      load_w(2, S2);
      load_w(3, S3);
      load_x(2, 2);
      load_x(3, 3);
      store(S0, 0);
      if (1 < nk) store(S1, 1);
      loader_barrier<0>();  // everything issued so far (see the one-step prologue)
      const int np = (nk + 1) / 2;
      auto period = [&](int p, Stage& La, Stage& Lb, const Stage& Sa, const Stage& Sb) {
        const int k = 2 * p;
        load_w(k + 4, La);
        load_w(k + 5, Lb);
        load_x(k + 4, (k + 4) % 6);
        load_x(k + 5, (k + 5) % 6);
        if (k + 2 < nk) store(Sa, (k + 2) % 4);
        if (k + 3 < nk) store(Sb, (k + 3) % 4);
        loader_barrier<2 * T::LOADS_PER_STEP>();
      };
      for (int p = 0; p < np; p += 2) {
        period(p, S0, S1, S2, S3);
        if (p + 1 >= np) break;
        period(p + 1, S2, S3, S0, S1);
      }
    }
    // the last steps' reloads land in buffers nobody reads; drain them before the wave ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if constexpr (T::KS > 1) __syncthreads();  // the MFMA waves' accumulator hand-off barrier
    return;
  }

  // ---------------- MFMA waves: MW (m) x NW (n) grid, wave (wm, wn) owns TM x TN of C
  constexpr int FM = T::FM, FN = T::FN;
  const int r = lane & 15, kq = lane >> 4;
  const int wm = wave / T::NW, wn = wave % T::NW;
  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // lane (r, kq) reads chunk kq + 4 s of rows r + 16 i: rows 16 i + r share r & 7, so the
  // swizzled slot is the same for all i
  const int a_off = (wm * T::TM + r) * GM_BK, b_off = (wn * T::TN + r) * GM_BK;
  const int slot0 = ((kq ^ (r & 7)) << 3), slot1 = (((kq + 4) ^ (r & 7)) << 3);
  auto compute = [&](int abuf, int bbuf) {
    const uint16_t* sA = sA0 + abuf * GM_LDS_A + a_off;
    const uint16_t* sB = sB0 + bbuf * GM_LDS_B + b_off;
#pragma unroll
    for (int s = 0; s < GM_BK / 32; ++s) {
      const int slot = s ? slot1 : slot0;
      // every fragment of the sub-step is read before the first MFMA (left alone, the
      // scheduler reads one A fragment, waits for it and runs its MFMAs, one LDS round trip
      // per fragment with the matrix core idle)
      u32x4 b[FN], av[FM];
#pragma unroll
      for (int j = 0; j < FN; ++j) b[j] = *(const u32x4*)(sB + j * 16 * GM_BK + slot);
#pragma unroll
      for (int i = 0; i < FM; ++i) av[i] = *(const u32x4*)(sA + i * 16 * GM_BK + slot);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16<XDT>(av[i], b[j], acc[i][j]);
    }
  };
  __syncthreads();  // step 0 (both steps of period 0) is in LDS
  if constexpr (T::SPB == 1) {
    int ab = 0;
    for (int ks = 0; ks < nk; ++ks) {
      compute(ab, ks & 1);
      ab = ab == GM_NA - 1 ? 0 : ab + 1;
      __syncthreads();
    }
  } else {
    const int np = (nk + 1) / 2;
    for (int p = 0; p < np; ++p) {
      const int k = 2 * p;
      compute(k % 6, k % 4);
      if (k + 1 < nk) compute((k + 1) % 6, (k + 1) % 4);
      __syncthreads();
    }
  }
  if constexpr (T::KS > 1) {
    // the second half's accumulators to the first through LDS (every MFMA read of the loop is
    // done: its last barrier has passed; the loader waves have drained and meet this barrier)
    float* const s_c = (float*)smem;  // [MFMA wave][fragment element][lane]
    constexpr int NE = FM * FN * 4;
    static_assert((size_t)T::MFMA_WAVES * NE * 64 * 4 <= T::HALF_ELEMS * 2, "accumulator hand-off exceeds LDS");
    if (half == 1) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) s_c[(wave * NE + (i * FN + j) * 4 + e) * 64 + lane] = acc[i][j][e];
    }
    __syncthreads();
    if (half == 1) return;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j][e] += s_c[(wave * NE + (i * FN + j) * 4 + e) * 64 + lane];
  }
  // C layout: lane holds rows 4 kq + e of column r of each 16 x 16 block
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t n = n0 + wn * T::TN + j * 16 + r;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm * T::TM + i * 16 + 4 * kq + e;
        if (m < M) y[m * N + n] = Elem<XDT>::cvt(acc[i][j][e]);
      }
  }
}

// ------------------------------------------------------------------ skinny GEMM (small M)
//
// For a few dozen rows of x the tiled kernel's tiles are too few and too thin to keep the chip
// busy, and splitting K over workgroups would write fp32 partials as large as the weights.  Here
// a workgroup of SK_WAVES waves owns SK_MROWS = 32 rows of x against SK_RB = 48 rows of W over
// all of K; the waves split K (128-k blocks) and meet once, in LDS, at the end.
//   - W: each wave copies its rows x k-slice straight into its own LDS region, whole 128-byte
//     lines per row per load (a load of 16 rows x 64 B, the shape an MFMA operand has in
//     registers, ran at half the rate from HBM), and reads one dword per MFMA fragment back;
//   - x: read from L2 into registers in MFMA layout (lane (r, kq) of load s: row r, k 32 s + 8 kq
//     .. + 8 of the block), two blocks ahead;
//   - W enters the MFMA as exact "off + q" fragments (one AND-OR per pair) shared by the two
//     16-row halves of x, and the zero point and scale are applied per 128-k group as
//     s * (sum x (off + q) - (off + z) sum x), the row sums of x coming from an MFMA against an
//     all-ones operand in the same C layout.
// The m-blocks of one W row block run on one XCD (workgroup w runs on XCD w % 8), so W comes from
// HBM once and the other m-blocks read it from that XCD's L2.  A CU pulls ~130 GB/s from L2,
// which is what bounds the x rows per workgroup (32 x K x 2 B) from above; the VALU work per
// MFMA (the nibble conversion) bounds them from below.
constexpr int SK_WAVES = 8, SK_PBMAX = 4, SK_NF = 3, SK_NC = 2;  // waves; blocks per pass; fragments
constexpr int SK_RB = 16 * SK_NF, SK_MROWS = 16 * SK_NC;           // W rows, x rows per workgroup
constexpr int SK_WREGION = SK_RB * 64 * SK_PBMAX;                  // LDS bytes per wave (12 KB)
constexpr int SK_LDS = SK_WAVES * SK_WREGION;

__device__ __forceinline__ void sk_copy_lds(__amdgpu_buffer_rsrc_t r, unsigned char* dst, uint32_t vo, int so) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, vo, so, 0, 0);
}

// PB: 128-k blocks per pass (1, 2 or 4: the launcher takes the fewest that cover a wave's share
// in one pass, up to 4).  Every block a pass loads is used, those past the wave's share (clamped
// reloads) with a zero factor: a load whose value is used only under a condition is sunk into
// that branch by the compiler, below the counted wait for W, which then no longer covers W.
template <int XDT, int SDT, int PB>
__global__ __launch_bounds__(64 * SK_WAVES) void int4_gemm_skinny_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t xs, const uint32_t* __restrict__ qw, int64_t N,
    int64_t pc, const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz,
    uint16_t* __restrict__ y, int row_blocks, int m_blocks) {
  extern __shared__ __attribute__((aligned(16))) unsigned char sk_lds[];  // SK_LDS bytes
  using ST = typename Elem<SDT>::T;
  constexpr float OFF = XDT == ANNA_MI_BF16 ? 128.0f : 1024.0f;
  constexpr uint32_t ONES = XDT == ANNA_MI_BF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr int NF = SK_NF, NC = SK_NC;
  // W in LDS: a pass is copied in halves of up to two blocks (128 B of each row: whole lines),
  // so that the first two blocks' compute need not wait for the rest of the pass.  A half's row
  // span is UNITS 16-byte units (64 B per block); unit c of row R sits at slot c ^ ((R >> RSH) %
  // UNITS), so that the 16 rows x 4 dwords of one fragment read fall on 64 distinct banks.
  constexpr int HB = PB < 2 ? PB : 2, HALVES = PB / HB;  // blocks per half, halves per pass
  constexpr int UNITS = 4 * HB, ROWB = 16 * UNITS, RSH = HB == 2 ? 1 : 2;
  constexpr int RPL = 1024 / ROWB, WLOADS = SK_RB / RPL;  // rows per 1 KB copy, copies per half
  constexpr int HBYTES = SK_RB * ROWB;                     // LDS bytes of one half
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int r = lane & 15, kq = lane >> 4;
  // item -> (row block, m-block); with whole octets of row blocks, the m-blocks of row block rb
  // are workgroups 8 (m_blocks (rb / 8) + mb) + rb % 8: one XCD, launched together
  const int b = (int)blockIdx.x;
  int rb, mb;
  if (row_blocks % NUM_XCD == 0) {
    const int slot = b / NUM_XCD;
    mb = slot % m_blocks;
    rb = (slot / m_blocks) * NUM_XCD + b % NUM_XCD;
  } else {
    rb = b / m_blocks;
    mb = b % m_blocks;
  }
  rb = __builtin_amdgcn_readfirstlane(rb);
  mb = __builtin_amdgcn_readfirstlane(mb);
  const int64_t n0 = (int64_t)rb * SK_RB, m0 = (int64_t)mb * SK_MROWS;
  const int rows_w = (int)(N - n0 < SK_RB ? N - n0 : SK_RB);
  const int rows_x = (int)(M - m0 < SK_MROWS ? M - m0 : SK_MROWS);
  // buffer resources over this workgroup's rows: W rows past N and x rows past M read as zero
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x + m0 * xs), 0, (int)(((rows_x - 1) * xs + K) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(qw + n0 * pc), 0, (int)(rows_w * pc * 4), 0x00020000);
  const int nblk = (int)(K / 128);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<ST*>(qs), 0, (int)((int64_t)nblk * N * (int64_t)sizeof(ST)), 0x00020000);
  const __amdgpu_buffer_rsrc_t rz =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(qz), 0, (int)((int64_t)nblk * N), 0x00020000);
  const int b_lo = wave * nblk / SK_WAVES, b_hi = (wave + 1) * nblk / SK_WAVES;
  unsigned char* const wl = sk_lds + wave * SK_WREGION;
  // W copy i: rows RPL i + lane / UNITS; the lane's slot lane % UNITS holds unit slot ^ key(row)
  const int wrow0 = lane / UNITS, wslot = lane % UNITS;
  auto w_voff = [&](int i) {
    const int row = RPL * i + wrow0;
    return (uint32_t)(row * pc * 4 + ((wslot ^ ((row >> RSH) & (UNITS - 1))) * 16));
  };
  // fragment read of (row 16 f + r, unit u of half h, dword kq)
  auto w_read = [&](int h, int f, int u) -> uint32_t {
    const int row = 16 * f + r;
    return *(const uint32_t*)(wl + h * HBYTES + row * ROWB + ((u ^ ((row >> RSH) & (UNITS - 1))) * 16) + kq * 4);
  };
  // x of c-block c (rows 16 c + r): 16 bytes at k 32 s + 8 kq of a block
  uint32_t xoff[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
    xoff[c] = 16 * c + r < rows_x ? (uint32_t)(((16 * c + r) * xs + kq * 8) * 2) : GM_OOB;
  const u32x4 ones = {ONES, ONES, ONES, ONES};
  f32x4 out[NF][NC];
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int c = 0; c < NC; ++c) out[f][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int p0 = b_lo; p0 < b_hi; p0 += PB) {
    const int nb = b_hi - p0 < PB ? b_hi - p0 : PB;
    // W of the whole pass first (a pass past the wave's share re-copies its own rows' units; the
    // region is the wave's alone, and its reads of the previous pass are done)
#pragma unroll
    for (int h = 0; h < HALVES; ++h)
#pragma unroll
      for (int i = 0; i < WLOADS; ++i) sk_copy_lds(rw, wl + h * HBYTES + i * 1024, w_voff(i), (p0 + h * HB) * 64);
    __builtin_amdgcn_sched_barrier(0);
    // scale and zero point of group p0 + kq (lane (r, kq), row 16 f + r); block j's are taken
    // from lane r + 16 j when it is used
    uint32_t sraw[NF], zraw[NF];
    const int gq = p0 + (kq < nb ? kq : nb - 1);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint32_t gi = (uint32_t)(gq * N + n0 + 16 * f + r);
      if constexpr (sizeof(ST) == 4)
        sraw[f] = __builtin_amdgcn_raw_buffer_load_b32(rs, gi * 4, 0, 0);
      else
        sraw[f] = __builtin_amdgcn_raw_buffer_load_b16(rs, gi * 2, 0, 0);
      zraw[f] = __builtin_amdgcn_raw_buffer_load_b8(rz, gi, 0, 0);
    }
    u32x4 xv[PB][NC][4];
    auto load_x = [&](int j) {
      const int blk = p0 + (j < nb ? j : nb - 1);
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          xv[j][c][s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xoff[c], (blk * 128 + s * 32) * 2, 0));
    };
    load_x(0);
    if constexpr (PB > 1) load_x(1);
    __builtin_amdgcn_sched_barrier(0);
    // the first half of W is in LDS
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((HALVES - 1) * WLOADS + 2 * NF + (PB > 1 ? 2 : 1) * NC * 4) : "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      if (j == HB) {
        // the second half of W: all but the x loads issued since (blocks 2 and 3)
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NC * 4) : "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
      if (j + 2 < PB) load_x(j + 2);
      f32x4 acc[NF][NC], sx[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        sx[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[f][c] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        u32x4 wf[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) wf[f] = nibbles_to_frag<XDT>(w_read(j / HB, f, 4 * (j % HB) + s));
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const u32x4 xa = interleave_x(xv[j][c][s]);
          sx[c] = mfma16<XDT>(xa, ones, sx[c]);
#pragma unroll
          for (int f = 0; f < NF; ++f) acc[f][c] = mfma16<XDT>(xa, wf[f], acc[f][c]);
        }
      }
      const int src = (r + 16 * j) * 4;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const uint32_t sv = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)sraw[f]);
        const int zv = (int)(int8_t)(uint8_t)__builtin_amdgcn_ds_bpermute(src, (int)zraw[f]);
        float sc;
        if constexpr (sizeof(ST) == 4) sc = __uint_as_float(sv);
        else sc = Elem<SDT>::to_f32((ST)sv);
        if (j >= nb) sc = 0.f;  // a clamped reload of the wave's last block
        const float zc = OFF + (float)zv;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) out[f][c][i] = fmaf(sc, fmaf(-zc, sx[c][i], acc[f][c][i]), out[f][c][i]);
      }
    }
  }
  // the waves' partial sums through LDS (every wave's W reads are done after the barrier); wave
  // w < NF NC sums fragment w % NF of c-block w / NF.  C layout: lane (r, kq) element i is x row
  // m0 + 16 c + 4 kq + i, W row n0 + 16 f + r.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped copies of the last pass
  __syncthreads();
  float* const red = (float*)sk_lds;  // [wave][fragment][c-block][element][lane]
  static_assert(SK_WAVES * NF * NC * 4 * 64 * 4 <= SK_LDS, "reduction fits the W regions");
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(((wave * NF + f) * NC + c) * 4 + i) * 64 + lane] = out[f][c][i];
  __syncthreads();
  if (wave >= NF * NC) return;
  const int f = wave % NF, c = wave / NF;
  if (16 * f + r >= rows_w) return;
  const int64_t n = n0 + 16 * f + r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < SK_WAVES; ++w) v += red[(((w * NF + f) * NC + c) * 4 + i) * 64 + lane];
    const int m = 16 * c + 4 * kq + i;
    if (m < rows_x) y[(m0 + m) * N + n] = Elem<XDT>::cvt(v);
  }
}

}  // namespace

bool int4_gemm_tiled_supported(int x_dtype, int64_t M, int64_t N, int64_t K, int64_t xs, const void* x, const void* qweight,
                               int64_t pc, const void* qscale, const void* qzeros, int64_t gsz) {
  (void)qscale;
  (void)qzeros;
  // buffer loads address each workgroup's slice with 32-bit offsets, and the k-step -> group map
  // is a multiply-high that is exact below 2^16 steps
  const int64_t G = gsz > 0 ? (K + gsz - 1) / gsz : 0;
  const bool fits = (int64_t)TileL::BM * xs * 2 < (1ll << 31) && (int64_t)TileL::BN * pc * 4 < (1ll << 31) &&
                    G * N * 4 < (1ll << 31) && K / GM_BK < (1 << 16) && gsz / GM_BK < (1 << 16);
  // (M < 64 works too, rows past M reading as zero: the dispatcher sends 16 < M < 64 here when K
  // is too long for the row-group GEMV)
  return (x_dtype == ANNA_MI_BF16 || x_dtype == ANNA_MI_F16) && M > 16 && K % GM_BK == 0 && gsz % GM_BK == 0 &&
         xs % 8 == 0 && pc % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)qweight % 16 == 0 && fits;
}

int int4_gemm_tiled_launch(const void* x, int x_dtype, int64_t M, int64_t K, int64_t xs, const int32_t* qweight,
                           int64_t N, int64_t pc, const void* qscale, int scale_dtype, const int8_t* qzeros, int64_t gsz,
                           void* y, hipStream_t st) {
  // the largest tile that still gives (about) every compute unit a workgroup (256 of them)
  auto tiles = [&](auto t) {
    using TT = decltype(t);
    return ((M + TT::BM - 1) / TT::BM) * ((N + TT::BN - 1) / TT::BN);
  };
  // The large tile also wins from 192 tiles, or 128 whose m-tiles are all full (N = 12288,
  // K = 4096: M = 768 99 against 125 us with the middle tile; M = 1024, N = 6144: 84 against
  // 87 us; M = 384 (128 tiles, the last half empty) 85 against 74 us).
  const int64_t tl = tiles(TileL{});
  int shape = (tl >= 192 || (tl >= 128 && M % TileL::BM == 0)) ? 0 : tiles(TileM{}) >= 256 ? 1 : 2;
  // the small tile splits K over two halves of the workgroup when its tiles fit one round of
  // workgroups (the 16-wave, 144 KB workgroup takes a whole compute unit: with more tiles, two
  // plain ones per unit are faster) and both halves get the same number of two-step periods
  // (their barriers must pair up).  M = 64, K = 4096: N = 12288 24.1 -> 21.9 us, N = 6144
  // 22.5 -> 19.0 us; M = 256, N = 6144 (512 tiles) split 39.3 against 35 us.
  const bool split = tiles(TileS{}) <= 256 && (K / GM_BK) % (2 * TileS2::SPB) == 0;
  // likewise the middle tile at exactly one round (M = 256, N = 12288: 52.4 -> 46.4 us; M = 192:
  // 51.3 -> 43.9 us), whose one-step periods need an even step count
  const bool msplit = tiles(TileM{}) <= 256 && (K / GM_BK) % (2 * TileM2::SPB) == 0;
  // ANNA_MI_INT4_GEMM_TILE = L / M / S forces a tile shape (read on every call; the tests run
  // every shape on shapes small enough for the CPU oracle)
  if (const char* f = getenv("ANNA_MI_INT4_GEMM_TILE"); f && *f) shape = f[0] == 'L' ? 0 : f[0] == 'M' ? 1 : 2;
  ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
    auto go = [&](auto xdt_tag, auto tile_tag) {
      constexpr int XDT = decltype(xdt_tag)::value;
      using TT = decltype(tile_tag);
      const int64_t tm = (M + TT::BM - 1) / TT::BM, tn = (N + TT::BN - 1) / TT::BN;
      auto kern = int4_gemm_tiled_kernel<XDT, SDT, TT>;
      static bool attr_set = false;
      if (!attr_set) {
        ANNA_CHECK(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)TT::LDS_BYTES) == hipSuccess,
                   "int4 GEMM: cannot raise the LDS limit");
        attr_set = true;
      }
      hipLaunchKernelGGL(kern, dim3((unsigned)(tm * tn)), dim3(TT::THREADS), TT::LDS_BYTES, st, (const uint16_t*)x, M,
                         K, xs, (const uint32_t*)qweight, N, pc, (const typename Elem<SDT>::T*)qscale, qzeros, gsz,
                         (uint16_t*)y, tm, tn);
      return ANNA_MI_OK;
    };
    auto go_x = [&](auto tile_tag) {
      return x_dtype == ANNA_MI_BF16 ? go(std::integral_constant<int, ANNA_MI_BF16>{}, tile_tag)
                                     : go(std::integral_constant<int, ANNA_MI_F16>{}, tile_tag);
    };
    const int rc = shape == 0 ? go_x(TileL{}) : shape == 1 ? (msplit ? go_x(TileM2{}) : go_x(TileM{})) : split ? go_x(TileS2{}) : go_x(TileS{});
    if (rc != ANNA_MI_OK) return rc;
  });
  ANNA_LAUNCH_CHECK("int4_gemm_tiled_kernel");
  return ANNA_MI_OK;
}

int64_t int4_gemm_skinny_workgroups(int64_t M, int64_t N) {
  return ((M + SK_MROWS - 1) / SK_MROWS) * ((N + SK_RB - 1) / SK_RB);
}

bool int4_gemm_skinny_supported(int x_dtype, int64_t M, int64_t N, int64_t K, int64_t xs, const void* x,
                                const void* qweight, int64_t pc, int64_t gsz) {
  // 32-bit buffer offsets: 32 x rows, 48 W rows, the scale / zero-point arrays
  const bool fits = (SK_MROWS * xs + K) * 2 < (1ll << 31) && SK_RB * pc * 4 < (1ll << 31) && (K / 128) * N * 4 < (1ll << 31);
  return (x_dtype == ANNA_MI_BF16 || x_dtype == ANNA_MI_F16) && M > 0 && gsz == 128 && K % 128 == 0 &&
         K / 128 >= SK_WAVES && xs % 8 == 0 && pc % 4 == 0 && (uintptr_t)x % 16 == 0 &&
         (uintptr_t)qweight % 16 == 0 && fits;
}

int int4_gemm_skinny_launch(const void* x, int x_dtype, int64_t M, int64_t K, int64_t xs, const int32_t* qweight,
                            int64_t N, int64_t pc, const void* qscale, int scale_dtype, const int8_t* qzeros,
                            void* y, hipStream_t st) {
  // 48 W rows x 32 x rows per workgroup: N = 6144 gives 128 row blocks, 256 workgroups at M = 64
  const int64_t m_blocks = (M + SK_MROWS - 1) / SK_MROWS, row_blocks = (N + SK_RB - 1) / SK_RB;
  const int64_t per_wave = (K / 128 + SK_WAVES - 1) / SK_WAVES;  // the largest share of blocks
  const int pb = per_wave <= 1 ? 1 : per_wave <= 2 ? 2 : 4;
  ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
    auto go = [&](auto xdt_tag, auto pb_tag) {
      constexpr int XDT = decltype(xdt_tag)::value, PB = decltype(pb_tag)::value;
      auto kern = int4_gemm_skinny_kernel<XDT, SDT, PB>;
      static bool attr_set = false;
      if (!attr_set) {
        ANNA_CHECK(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, SK_LDS) ==
                       hipSuccess,
                   "int4 skinny GEMM: cannot raise the LDS limit");
        attr_set = true;
      }
      hipLaunchKernelGGL(kern, dim3((unsigned)(row_blocks * m_blocks)), dim3(64 * SK_WAVES), SK_LDS, st,
                         (const uint16_t*)x, M, K, xs, (const uint32_t*)qweight, N, pc,
                         (const typename Elem<SDT>::T*)qscale, qzeros, (uint16_t*)y, (int)row_blocks, (int)m_blocks);
      return ANNA_MI_OK;
    };
    auto go_pb = [&](auto xdt_tag) {
      return pb == 1 ? go(xdt_tag, std::integral_constant<int, 1>{})
             : pb == 2 ? go(xdt_tag, std::integral_constant<int, 2>{})
                       : go(xdt_tag, std::integral_constant<int, 4>{});
    };
    const int rc = x_dtype == ANNA_MI_BF16 ? go_pb(std::integral_constant<int, ANNA_MI_BF16>{})
                                           : go_pb(std::integral_constant<int, ANNA_MI_F16>{});
    if (rc != ANNA_MI_OK) return rc;
  });
  ANNA_LAUNCH_CHECK("int4_gemm_skinny_kernel");
  return ANNA_MI_OK;
}

}  // namespace anna
