// W4A16 GEMM for M >= 64 on gfx950: y[M, N] = x[M, K] . dequant(W)[N, K]^T.
//
// Tile 256 (m) x 192 (n) x 64 (k) per workgroup of 12 waves with two roles:
//   8 MFMA waves   a 2 x 4 grid, each owning 128 x 48 of C as 8 x 3 v_mfma_f32_16x16x32
//                  accumulators; they only read LDS;
//   4 loader waves (one per SIMD) load x (256 x 64, 16-bit) and the int4 words of W (192 rows
//                  x 64 k) two k-steps ahead, dequantize W to (q - z) * s in fp32 rounded to the
//                  activation dtype (the reference's dequant numerics, quantization.py:626-648)
//                  and write both to the LDS buffer of the next step.
// The two roles run between the same barriers (one per k-step, double-buffered LDS, 126 KB), so
// each SIMD issues the loaders' VALU work while its MFMA waves keep the matrix core busy.  The
// tile -> workgroup map is XCD-aware and m-major: the n-tiles of one m-tile share one XCD, so
// that XCD's L2 holds the m-tile's slice of x (256 x K, 2 MB at K = 4096) and only the small
// int4 W streams in; M = 2048 with N = 12288 gives 512 tiles (two rounds on 256 CUs).
#include <type_traits>

#include "common.hpp"
#include "int4_frag.hpp"
#include "int4_gemm.hpp"

namespace anna {
namespace {

constexpr int GM_BM = 256, GM_BN = 192, GM_BK = 64;
constexpr int GM_PITCH = GM_BK + 8;  // LDS row pitch (16-bit elements): rows land 4 banks apart
constexpr int GM_MFMA_WAVES = 8, GM_LOAD_WAVES = 4;
constexpr int GM_THREADS = 64 * (GM_MFMA_WAVES + GM_LOAD_WAVES);
constexpr int GM_LT = 64 * GM_LOAD_WAVES;  // loader threads
constexpr int GM_LDS_A = GM_BM * GM_PITCH, GM_LDS_B = GM_BN * GM_PITCH;  // elements per stage
constexpr size_t GM_LDS_BYTES = (size_t)2 * (GM_LDS_A + GM_LDS_B) * 2;
constexpr int GM_XPT = GM_BM * GM_BK / 8 / GM_LT;        // x chunks (16 B) per loader thread: 8
constexpr int GM_WPT = GM_BN * (GM_BK / 16) / GM_LT;     // W chunks (8 B = 16 nibbles) per loader thread: 3

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

template <int XDT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (XDT == ANNA_MI_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){lo, hi}, bf16x2v));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){lo, hi}, f16x2v));
  }
}

template <int XDT, int SDT>
__global__ __launch_bounds__(GM_THREADS) void int4_gemm_tiled_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t xs, const uint32_t* __restrict__ qw, int64_t N,
    int64_t pc, const typename Elem<SDT>::T* __restrict__ qs, const int8_t* __restrict__ qz, int64_t gsz,
    uint16_t* __restrict__ y, int64_t tiles_m, int64_t tiles_n) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  using ST = typename Elem<SDT>::T;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // tile coordinates in 32-bit scalar registers: a value the compiler cannot prove uniform
  // would turn every buffer load below into a loop over distinct descriptors
  const int t = __builtin_amdgcn_readfirstlane((int)xcd_tile(blockIdx.x, tiles_m * tiles_n));
  const int tn32 = (int)tiles_n;
  const int64_t m0 = (int64_t)__builtin_amdgcn_readfirstlane((t / tn32) * GM_BM);
  const int64_t n0 = (int64_t)__builtin_amdgcn_readfirstlane((t % tn32) * GM_BN);
  const int64_t nk = K / GM_BK;

  if (wave >= GM_MFMA_WAVES) {
    // ---------------- loader waves: global -> registers (two steps ahead) -> dequant -> LDS
    // Buffer loads: a per-lane 32-bit offset plus a uniform one, and rows past M or N read as
    // zero (their products only reach rows / columns of C that are not stored).
    const int lt = tid - 64 * GM_MFMA_WAVES;
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
    // x chunk i of this thread: row lt / 8 + 32 i, 8 k at (lt % 8) * 8; W chunk i: row
    // lt / 4 + 64 i, 16 k at (lt % 4) * 16
    const uint32_t xo = (uint32_t)(((lt >> 3) * xs + (lt & 7) * 8) * 2);
    const uint32_t wo = (uint32_t)(((lt >> 2) * pc + (lt & 3) * 2) * 4);
    const uint32_t so = (uint32_t)((lt >> 2) * sizeof(ST)), zo = (uint32_t)(lt >> 2);
    // the scale and zero point stay raw until the store: converting them at the load would
    // make the load wait for its data
    struct Stage {
      u32x4 x[GM_XPT];
      uint2 w[GM_WPT];
      uint32_t sc[GM_WPT], z[GM_WPT];
    };
    // group of k-step ks = ks / (gsz / 64) as a multiply-high by ceil(2^32 / (gsz / 64)) (one
    // group per step needs no map): exact while both are below 2^16 (checked by the launcher);
    // a division here would branch and make the loads just issued wait
    const uint32_t spg = (uint32_t)(gsz / GM_BK);
    const uint32_t ginv = spg > 1 ? (uint32_t)(((1ull << 32) + spg - 1) / spg) : 0u;
    const int nk32 = (int)nk;
    auto load = [&](int ks, Stage& S) {
      ks = ks < nk32 ? ks : nk32 - 1;
#pragma unroll
      for (int i = 0; i < GM_XPT; ++i)
        S.x[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rx, xo, (int)(i * 32 * xs * 2) + ks * (GM_BK * 2), 0));
      const int g = spg == 1 ? ks : (int)__umulhi((uint32_t)ks, ginv);
#pragma unroll
      for (int i = 0; i < GM_WPT; ++i) {
        S.w[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                               rw, wo, (int)(i * 64 * pc * 4) + ks * (GM_BK / 2), 0));
        if constexpr (sizeof(ST) == 4)
          S.sc[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, so, (int)((g * N + 64 * i) * 4), 0);
        else
          S.sc[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, so, (int)((g * N + 64 * i) * 2), 0);
        S.z[i] = __builtin_amdgcn_raw_buffer_load_b8(rz, zo, (int)(g * N + 64 * i), 0);
      }
    };
    auto store = [&](const Stage& S, int buf) {
      uint16_t* sA = smem + buf * GM_LDS_A;
      uint16_t* sB = smem + 2 * GM_LDS_A + buf * GM_LDS_B;
#pragma unroll
      for (int i = 0; i < GM_XPT; ++i)
        *(u32x4*)(sA + ((lt >> 3) + 32 * i) * GM_PITCH + (lt & 7) * 8) = S.x[i];
#pragma unroll
      for (int i = 0; i < GM_WPT; ++i) {
        float sc;
        if constexpr (sizeof(ST) == 4) sc = __uint_as_float(S.sc[i]);
        else sc = Elem<SDT>::to_f32((ST)S.sc[i]);
        const float z = (float)(int8_t)S.z[i];
        uint16_t* dst = sB + ((lt >> 2) + 64 * i) * GM_PITCH + (lt & 3) * 16;
#pragma unroll
        for (int wi = 0; wi < 2; ++wi) {
          const uint32_t w = wi ? S.w[i].y : S.w[i].x;
          const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
          u32x4 o;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float a = ((float)((lo >> (8 * j)) & 0xFFu) - z) * sc;  // nibble 2j
            const float b = ((float)((hi >> (8 * j)) & 0xFFu) - z) * sc;  // nibble 2j + 1
            o[j] = pack2<XDT>(a, b);
          }
          *(u32x4*)(dst + wi * 8) = o;
        }
      }
    };
    Stage S0, S1;
    load(0, S0);
    load(1, S1);
    store(S0, 0);
    __syncthreads();
    for (int ks = 0; ks < nk32; ks += 2) {
      // step ks: MFMA waves read buffer 0; store step ks + 1 into buffer 1
      load(ks + 2, S0);
      if (ks + 1 < nk32) store(S1, 1);
      __syncthreads();
      if (ks + 1 >= nk32) break;
      load(ks + 3, S1);
      if (ks + 2 < nk32) store(S0, 0);
      __syncthreads();
    }
    return;
  }

  // ---------------- MFMA waves: 2 (m) x 4 (n) grid, wave (wm, wn) owns 128 x 48 of C
  const int r = lane & 15, kq = lane >> 4;
  const int wm = wave >> 2, wn = wave & 3;
  f32x4 acc[8][3];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf) {
    const uint16_t* sA = smem + buf * GM_LDS_A + (wm * 128 + r) * GM_PITCH + kq * 8;
    const uint16_t* sB = smem + 2 * GM_LDS_A + buf * GM_LDS_B + (wn * 48 + r) * GM_PITCH + kq * 8;
#pragma unroll
    for (int s = 0; s < GM_BK / 32; ++s) {
      u32x4 b[3];
#pragma unroll
      for (int j = 0; j < 3; ++j) b[j] = *(const u32x4*)(sB + j * 16 * GM_PITCH + s * 32);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u32x4 a = *(const u32x4*)(sA + i * 16 * GM_PITCH + s * 32);
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = mfma16<XDT>(a, b[j], acc[i][j]);
      }
    }
  };
  __syncthreads();  // stage 0 is in LDS
  for (int64_t ks = 0; ks < nk; ++ks) {
    compute((int)(ks & 1));
    __syncthreads();
  }
  // C layout: lane holds rows 4 kq + e of column r of each 16 x 16 block
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int64_t n = n0 + wn * 48 + j * 16 + r;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm * 128 + i * 16 + 4 * kq + e;
        if (m < M) y[m * N + n] = Elem<XDT>::cvt(acc[i][j][e]);
      }
  }
}

}  // namespace

bool int4_gemm_tiled_supported(int x_dtype, int64_t M, int64_t N, int64_t K, int64_t xs, const void* x, const void* qweight,
                               int64_t pc, int64_t gsz) {
  // buffer loads address each workgroup's slice with 32-bit offsets, and the k-step -> group map
  // is a multiply-high that is exact below 2^16 steps
  const int64_t G = gsz > 0 ? (K + gsz - 1) / gsz : 0;
  const bool fits = (int64_t)GM_BM * xs * 2 < (1ll << 31) && (int64_t)GM_BN * pc * 4 < (1ll << 31) &&
                    G * N * 4 < (1ll << 31) && K / GM_BK < (1 << 16) && gsz / GM_BK < (1 << 16);
  return (x_dtype == ANNA_MI_BF16 || x_dtype == ANNA_MI_F16) && M >= 64 && K % GM_BK == 0 && gsz % GM_BK == 0 &&
         xs % 8 == 0 && pc % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)qweight % 16 == 0 && fits;
}

int int4_gemm_tiled_launch(const void* x, int x_dtype, int64_t M, int64_t K, int64_t xs, const int32_t* qweight,
                           int64_t N, int64_t pc, const void* qscale, int scale_dtype, const int8_t* qzeros, int64_t gsz,
                           void* y, hipStream_t st) {
  const int64_t tm = (M + GM_BM - 1) / GM_BM, tn = (N + GM_BN - 1) / GM_BN;
  ANNA_DISPATCH_DTYPE(scale_dtype, SDT, {
    auto go = [&](auto xdt_tag) {
      constexpr int XDT = decltype(xdt_tag)::value;
      auto kern = int4_gemm_tiled_kernel<XDT, SDT>;
      static bool attr_set = false;
      if (!attr_set) {
        ANNA_CHECK(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)GM_LDS_BYTES) == hipSuccess,
                   "int4 GEMM: cannot raise the LDS limit");
        attr_set = true;
      }
      hipLaunchKernelGGL(kern, dim3((unsigned)(tm * tn)), dim3(GM_THREADS), GM_LDS_BYTES, st, (const uint16_t*)x, M, K,
                         xs, (const uint32_t*)qweight, N, pc, (const typename Elem<SDT>::T*)qscale, qzeros, gsz,
                         (uint16_t*)y, tm, tn);
      return ANNA_MI_OK;
    };
    const int rc = x_dtype == ANNA_MI_BF16 ? go(std::integral_constant<int, ANNA_MI_BF16>{})
                                           : go(std::integral_constant<int, ANNA_MI_F16>{});
    if (rc != ANNA_MI_OK) return rc;
  });
  ANNA_LAUNCH_CHECK("int4_gemm_tiled_kernel");
  return ANNA_MI_OK;
}

}  // namespace anna
