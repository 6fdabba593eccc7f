// TurboQuant KV-cache packing and split-KV GQA decode attention on gfx950.
//
// Formats
//   values (reference format, src/anna/model/turboquant.py:157-252): per (head, token,
//     group of G dims) min/max quantization, scale = clamp((max-min)/(2^b-1), 1e-8) and
//     zero = min stored in the value dtype, codes packed 4 per byte (2-bit) or 2 per byte
//     (3/4-bit), element i at bits sb*(i % per_byte).
//   TQ-MSE (this build's definition of the absent `turboquant` package's MSE quantizer,
//     turboquant.py:75-82): y = R x with a seeded rotation R, code_i = number of codebook
//     thresholds t_j with y_i >= t_j * |x|, norm |x| stored as fp16; the reconstruction is
//     |x|_fp16 * R^T c[code].  Codes pack like the values.  R is the randomized Hadamard
//     rotation (1/sqrt(D)) H diag(s) for power-of-two D (tq_hadamard.hpp: an O(D log D)
//     transform in registers), a seeded Haar matrix otherwise.
//
// Numerics of the MSE quantizer are fixed so that the GPU reproduces the CPU oracle bit
// for bit: dense R: |x|^2 and every y_i are fma chains in ascending k; Hadamard R: the order
// of tq_hadamard.hpp; sqrt is correctly rounded.
#include <math.h>
#include <stdlib.h>

#include <type_traits>
#include <vector>

#include "common.hpp"
#include "tq_hadamard.hpp"

namespace anna {
namespace {

__host__ __device__ inline int storage_bits(int bits) { return bits == 2 ? 2 : 4; }

// ------------------------------------------------------------------ host: rotation, codebook


// Power-of-two D: the randomized Hadamard rotation R[i][j] = s_j (-1)^popcount(i & j) / sqrt(D)
// in fp32.  Otherwise a Haar-distributed orthogonal D x D matrix: a seeded standard-normal
// matrix (splitmix64 stream, Box-Muller) whose rows are orthonormalized by modified
// Gram-Schmidt applied twice, in fp64, then rounded to fp32.  Row i of the result is R[i][:],
// y = R x.
void make_rotation(int64_t D, uint64_t seed, float* out) {
  if (tq_is_pow2(D)) {
    std::vector<float> sg((size_t)D);
    tq_hadamard_signs(D, seed, sg.data());
    const float inv = tq_inv_sqrt(D);
    for (int64_t i = 0; i < D; ++i)
      for (int64_t j = 0; j < D; ++j)
        out[i * D + j] = (__builtin_popcountll((unsigned long long)(i & j)) & 1) ? -sg[(size_t)j] * inv : sg[(size_t)j] * inv;
    return;
  }
  std::vector<double> g((size_t)(D * D));
  tq_gaussian(D * D, seed, g.data());
  for (int64_t i = 0; i < D; ++i) {
    double* gi = &g[(size_t)(i * D)];
    for (int pass = 0; pass < 2; ++pass)
      for (int64_t j = 0; j < i; ++j) {
        const double* gj = &g[(size_t)(j * D)];
        double dot = 0.0;
        for (int64_t k = 0; k < D; ++k) dot += gi[k] * gj[k];
        for (int64_t k = 0; k < D; ++k) gi[k] -= dot * gj[k];
      }
    double nrm = 0.0;
    for (int64_t k = 0; k < D; ++k) nrm += gi[k] * gi[k];
    nrm = sqrt(nrm);
    for (int64_t k = 0; k < D; ++k) gi[k] /= nrm;
  }
  for (int64_t i = 0; i < D * D; ++i) out[i] = (float)g[(size_t)i];
}

// Lloyd-Max quantizer of N(0, 1): positive half of the levels (Max 1960), to 17 digits.
const double kLloydMax1[] = {0.79788456080286629};
const double kLloydMax2[] = {0.45278003463649735, 1.5104176084991006};
const double kLloydMax3[] = {0.2450941789442308, 0.75600528120588584, 1.3439092785050075, 2.151945704536995};
const double kLloydMax4[] = {0.12839502985114548, 0.38804829949029002, 0.65675911853246316, 0.94234045648696207,
                             1.2562311973471787,  1.6180463860218879,  2.0690172265313875,  2.732589570995156};

}  // namespace

// 2-bit levels are stored as fp16 magnitudes whose encodings share their low byte
// (0x3C7E = 1.123046875, 0x437E = 3.74609375; ratio 3.335652 vs the Lloyd-Max 3.335686),
// so a 2-bit code becomes an fp16 MFMA operand with one byte permute.
constexpr float TQ2_A16 = 1.123046875f, TQ2_B16 = 3.74609375f;

int tq_codebook(int bits, int64_t D, float* centroids, float* thresholds) {
  const int n = 1 << bits;
  const double* half = bits == 1 ? kLloydMax1 : bits == 2 ? kLloydMax2 : bits == 3 ? kLloydMax3 : kLloydMax4;
  std::vector<double> lv((size_t)n);
  const double inv = 1.0 / sqrt((double)D);
  for (int i = 0; i < n / 2; ++i) {
    double v = half[i];
    if (bits == 2) v = i == 0 ? kLloydMax2[0] : kLloydMax2[0] * ((double)TQ2_B16 / (double)TQ2_A16);
    lv[(size_t)(n / 2 + i)] = v * inv;
    lv[(size_t)(n / 2 - 1 - i)] = -v * inv;
  }
  for (int i = 0; i < n; ++i) centroids[i] = (float)lv[(size_t)i];
  for (int i = 0; i + 1 < n; ++i) thresholds[i] = (float)(0.5 * (lv[(size_t)i] + lv[(size_t)i + 1]));
  return 0;
}

namespace {

// ------------------------------------------------------------------ TQ-MSE quantize / dequant

// Vectors per workgroup (VB): each workgroup re-reads the D x D rotation from L2, so more vectors
// per workgroup mean less of that traffic; 32 up to D = 512, 16 above so the x stage fits in LDS.
constexpr int tq_vectors_per_wg(int64_t D) { return D <= 512 ? 32 : 16; }

// grid: ceil(nvec / VB); block: D threads (D multiple of 64, <= 1024)
template <int XDT, int TQ_VB>
__global__ __launch_bounds__(1024) void tq_mse_quantize_kernel(
    const typename Elem<XDT>::T* __restrict__ x, int64_t nvec, int64_t D, int64_t xs,
    const float* __restrict__ rot_t, const float* __restrict__ thr, int bits,
    uint8_t* __restrict__ codes, uint16_t* __restrict__ norms) {
  extern __shared__ float smem[];  // xs_[VB][D] then codes as bytes [VB][D]
  float* xsm = smem;
  uint8_t* csm = (uint8_t*)(smem + TQ_VB * D);
  __shared__ float nrm[TQ_VB];
  const int i = threadIdx.x;
  const int64_t v0 = (int64_t)blockIdx.x * TQ_VB;
  const int nv = (int)(nvec - v0 < TQ_VB ? nvec - v0 : TQ_VB);
  for (int v = 0; v < TQ_VB; ++v) xsm[v * D + i] = v < nv ? Elem<XDT>::load(x, (v0 + v) * xs + i) : 0.f;
  __syncthreads();
  if (i < TQ_VB) {
    float ss = 0.f;
    for (int64_t k = 0; k < D; ++k) ss = __builtin_fmaf(xsm[i * D + k], xsm[i * D + k], ss);
    nrm[i] = __builtin_sqrtf(ss);
    if (i < nv) norms[v0 + i] = f32_to_f16_bits(nrm[i]);
  }
  // y_i = sum_k R[i][k] x_k as one fma per k in ascending k (the oracle's order), four k per
  // LDS read of x (D is a multiple of 64)
  float acc[TQ_VB];
#pragma unroll
  for (int v = 0; v < TQ_VB; ++v) acc[v] = 0.f;
  for (int64_t k = 0; k < D; k += 4) {
    const float p0 = rot_t[k * D + i], p1 = rot_t[(k + 1) * D + i];
    const float p2 = rot_t[(k + 2) * D + i], p3 = rot_t[(k + 3) * D + i];
#pragma unroll
    for (int v = 0; v < TQ_VB; ++v) {
      const float4 xv = *(const float4*)(xsm + v * D + k);
      acc[v] = __builtin_fmaf(p0, xv.x, acc[v]);
      acc[v] = __builtin_fmaf(p1, xv.y, acc[v]);
      acc[v] = __builtin_fmaf(p2, xv.z, acc[v]);
      acc[v] = __builtin_fmaf(p3, xv.w, acc[v]);
    }
  }
  __syncthreads();
  const int nthr = (1 << bits) - 1;
#pragma unroll
  for (int v = 0; v < TQ_VB; ++v) {
    uint32_t c = 0;
    for (int j = 0; j < nthr; ++j) c += acc[v] >= __fmul_rn(thr[j], nrm[v]) ? 1u : 0u;
    csm[v * D + i] = (uint8_t)c;
  }
  __syncthreads();
  const int sb = storage_bits(bits), per = 8 / sb;
  const int64_t pb = D / per;  // packed bytes per vector
  for (int64_t idx = i; idx < (int64_t)nv * pb; idx += blockDim.x) {
    const int64_t v = idx / pb, b = idx % pb;
    uint32_t byte = 0;
    for (int e = 0; e < per; ++e) byte |= (uint32_t)csm[v * D + b * per + e] << (sb * e);
    codes[(v0 + v) * pb + b] = (uint8_t)byte;
  }
}

// The E codes of every lane of a wave (lane l: elements l*E ..), sb bits each, packed in element
// order into dst (D * sb / 8 bytes).  The whole wave takes part (sub-byte lanes combine by shuffles).
template <int E>
__device__ __forceinline__ void store_codes_wave(const uint32_t (&code)[E], int sb, uint8_t* dst, int lane) {
  const int nbits = E * sb;
  uint64_t pk = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) pk |= (uint64_t)code[e] << (sb * e);
  if (nbits == 8) {
    dst[lane] = (uint8_t)pk;
  } else if (nbits == 16) {
    ((uint16_t*)dst)[lane] = (uint16_t)pk;
  } else if (nbits > 8) {
    for (int k = 0; k < nbits / 8; ++k) dst[lane * (nbits / 8) + k] = (uint8_t)(pk >> (8 * k));
  } else {
    const int per = 8 / nbits;  // lanes per byte
    uint32_t b = (uint32_t)pk << (nbits * (lane % per));
    for (int m = 1; m < per; m <<= 1) b |= (uint32_t)__shfl_xor((int)b, m, 64);
    if (lane % per == 0) dst[lane / per] = (uint8_t)b;
  }
}

// Hadamard TQ-MSE quantizer: each wave takes HNV vectors at once (their shuffle chains are
// independent, so their latencies overlap), 4 waves per 256-thread workgroup; lane l holds
// elements l*E .. l*E + E - 1 of each (E = D / 64).
constexpr int HNV = 4;

template <int XDT, int E>
__global__ __launch_bounds__(256) void tq_hadamard_quantize_kernel(
    const typename Elem<XDT>::T* __restrict__ x, int64_t nvec, int64_t D, int64_t xs,
    const float* __restrict__ signs, const float* __restrict__ thr, int bits, uint8_t* __restrict__ codes,
    uint16_t* __restrict__ norms) {
  const int lane = threadIdx.x & 63;
  const int64_t v0 = ((int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * HNV;
  if (v0 >= nvec) return;  // whole wave
  float xv[HNV][E];
#pragma unroll
  for (int n = 0; n < HNV; ++n) {
    const int64_t v = v0 + n < nvec ? v0 + n : nvec - 1;  // clamped: the tail wave repeats its last vector
#pragma unroll
    for (int e = 0; e < E; ++e) xv[n][e] = Elem<XDT>::load(x, v * xs + lane * E + e);
  }
  uint32_t code[HNV][E];
  float nrm[HNV];
  hadamard_codes_wave_n<HNV, E>(xv, signs, thr, (1 << bits) - 1, tq_inv_sqrt(D), code, nrm);
  const int sb = storage_bits(bits);
  const int64_t pb = D * sb / 8;  // packed bytes per vector
#pragma unroll
  for (int n = 0; n < HNV; ++n) {
    const int64_t v = v0 + n;
    if (v >= nvec) break;
    if (lane == 0) norms[v] = f32_to_f16_bits(nrm[n]);
    store_codes_wave<E>(code[n], sb, codes + v * pb, lane);
  }
}

// out[v][k] = norm_v * sum_i R[i][k] c[code_i]  (fp32 accumulation)
template <int ODT, int TQ_VB>
__global__ __launch_bounds__(1024) void tq_mse_dequant_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms, int64_t nvec, int64_t D,
    const float* __restrict__ rot, const float* __restrict__ cent, int bits,
    typename Elem<ODT>::T* __restrict__ out, int64_t os) {
  extern __shared__ float yv[];  // [VB][D] centroid values
  const int k = threadIdx.x;
  const int64_t v0 = (int64_t)blockIdx.x * TQ_VB;
  const int nv = (int)(nvec - v0 < TQ_VB ? nvec - v0 : TQ_VB);
  const int sb = storage_bits(bits), per = 8 / sb;
  const uint32_t mask = (1u << sb) - 1u;
  const int64_t pb = D / per;
  for (int v = 0; v < TQ_VB; ++v) {
    float c = 0.f;
    if (v < nv) c = cent[(codes[(v0 + v) * pb + k / per] >> (sb * (k % per))) & mask];
    yv[v * D + k] = c;
  }
  __syncthreads();
  float acc[TQ_VB];
#pragma unroll
  for (int v = 0; v < TQ_VB; ++v) acc[v] = 0.f;
  for (int64_t i = 0; i < D; i += 4) {
    const float p0 = rot[i * D + k], p1 = rot[(i + 1) * D + k], p2 = rot[(i + 2) * D + k], p3 = rot[(i + 3) * D + k];
#pragma unroll
    for (int v = 0; v < TQ_VB; ++v) {
      const float4 y4 = *(const float4*)(yv + v * D + i);
      acc[v] = fmaf(p0, y4.x, acc[v]);
      acc[v] = fmaf(p1, y4.y, acc[v]);
      acc[v] = fmaf(p2, y4.z, acc[v]);
      acc[v] = fmaf(p3, y4.w, acc[v]);
    }
  }
  for (int v = 0; v < nv; ++v) out[(v0 + v) * os + k] = Elem<ODT>::cvt(f16_bits_to_f32(norms[v0 + v]) * acc[v]);
}

// ------------------------------------------------------------------ values: min/max groups

// One thread per (row, run of `gpt` groups); rows = H*T with row strides (sh, st).  A run
// always ends on a packed-byte boundary (gpt = 1 when group_size is a multiple of the
// pack width, else the whole row), so no two threads write the same byte.
// Groups g0 .. g0 + gpt - 1 of one vector (`src`, D elements): min/max, scale and zero point
// (rounded to the value dtype), codes packed into `data` (the vector's packed row).  The run
// ends on a packed-byte boundary, so runs of one vector can be done by different threads.
template <int DT>
__device__ void quantize_value_run(const typename Elem<DT>::T* __restrict__ src, int64_t D, int bits, int64_t gsz,
                                   int64_t g0, int64_t gpt, uint8_t* __restrict__ data,
                                   typename Elem<DT>::T* __restrict__ scales, typename Elem<DT>::T* __restrict__ zeros) {
  const float levels = (float)((1 << bits) - 1);
  const int sb = storage_bits(bits), per = 8 / sb;
  uint32_t byte = 0;
  for (int64_t g = g0; g < g0 + gpt; ++g) {
    float vmin = INFINITY, vmax = -INFINITY;
    for (int64_t j = 0; j < gsz; ++j) {
      const float f = Elem<DT>::to_f32(src[g * gsz + j]);
      vmin = fminf(vmin, f);
      vmax = fmaxf(vmax, f);
    }
    float sc = __fdiv_rn(__fsub_rn(vmax, vmin), levels);
    sc = sc < 1e-8f ? 1e-8f : sc;
    const typename Elem<DT>::T sc_s = Elem<DT>::cvt(sc), z_s = Elem<DT>::cvt(vmin);
    scales[g] = sc_s;
    zeros[g] = z_s;
    const float scf = Elem<DT>::to_f32(sc_s), zf = Elem<DT>::to_f32(z_s);
    for (int64_t j = 0; j < gsz; ++j) {
      const int64_t d = g * gsz + j;
      float q = rintf(__fdiv_rn(__fsub_rn(Elem<DT>::to_f32(src[d]), zf), scf));
      q = fminf(fmaxf(q, 0.f), levels);
      byte |= (uint32_t)q << (sb * (d % per));
      if (d % per == per - 1) {
        data[d / per] = (uint8_t)byte;
        byte = 0;
      }
    }
  }
}

// Groups per run: 1 when a group fills whole packed bytes, else the whole vector.
__host__ __device__ inline int64_t value_groups_per_run(int bits, int64_t D, int64_t gsz) {
  return gsz % (8 / storage_bits(bits)) == 0 ? 1 : D / gsz;
}

template <int DT>
__global__ __launch_bounds__(256) void tq_values_quantize_kernel(
    const typename Elem<DT>::T* __restrict__ v, int64_t H, int64_t T, int64_t D, int64_t sh, int64_t st,
    int bits, int64_t gsz, int64_t gpt, uint8_t* __restrict__ data, typename Elem<DT>::T* __restrict__ scales,
    typename Elem<DT>::T* __restrict__ zeros) {
  const int64_t ng = D / gsz;
  const int64_t runs = ng / gpt;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= H * T * runs) return;
  const int64_t row = idx / runs, g0 = (idx % runs) * gpt;
  const int64_t h = row / T, t = row % T;
  const int64_t pb = D * storage_bits(bits) / 8;
  quantize_value_run<DT>(v + h * sh + t * st, D, bits, gsz, g0, gpt, data + row * pb, scales + row * ng, zeros + row * ng);
}

template <int DT, int ODT>
__global__ __launch_bounds__(256) void tq_values_dequant_kernel(
    const uint8_t* __restrict__ data, const typename Elem<DT>::T* __restrict__ scales,
    const typename Elem<DT>::T* __restrict__ zeros, int64_t rows, int64_t D, int bits, int64_t gsz,
    typename Elem<ODT>::T* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * D) return;
  const int64_t row = idx / D, d = idx % D;
  const int sb = storage_bits(bits), per = 8 / sb;
  const uint32_t q = (data[row * (D / per) + d / per] >> (sb * (d % per))) & ((1u << sb) - 1u);
  const int64_t gi = row * (D / gsz) + d / gsz;
  out[idx] = Elem<ODT>::cvt((float)q * Elem<DT>::to_f32(scales[gi]) + Elem<DT>::to_f32(zeros[gi]));
}

// One token per sequence into a cache with one region per (sequence, KV head) -- the general
// form of the batched cache (any head_dim the Hadamard rotation takes, key bits 1..4, value bits
// 2..4): one workgroup per sequence of 2 * min(H, 8) waves; wave w takes the key (w even) or the
// value (w odd) of KV heads w / 2, w / 2 + 8, ...  When the window is full the token leaving it
// (ring slot n % R) is quantized into packed slot n - R -- keys as Hadamard TQ-MSE codes + norm
// (bit-exact with anna_mi_tq_hadamard_quantize), values as min/max groups (bit-exact with
// anna_mi_tq_values_quantize) -- then, after a barrier, the new token takes the slot and the
// length grows by one.  A sequence whose packed region is full is left as it is and raises the
// overflow flag.
template <int XDT, int E>
__global__ __launch_bounds__(1024) void tq_rows_append_kernel(const anna_mi_tq_rows_append_args a) {
  using T = typename Elem<XDT>::T;
  const int lane = threadIdx.x & 63, wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b = blockIdx.x, hstep = blockDim.x >> 7;
  const bool is_v = wave & 1;
  const int64_t H = a.kv_heads, D = a.head_dim, R = a.residual_capacity, C = a.capacity;
  const int n = a.seq_lengths[b];
  const bool evict = n >= R;
  if (evict && (int64_t)n - R >= C) {  // uniform over the workgroup
    if (threadIdx.x == 0) *a.overflow = 1;
    return;
  }
  const int64_t slot = n % R;
  if (evict) {
    const int64_t q = n - R;
    for (int64_t h = wave >> 1; h < H; h += hstep) {
      const int64_t row = b * H + h;
      const T* ring = (const T*)(is_v ? a.residual_value : a.residual_key) + (row * R + slot) * D;
      if (!is_v) {
        float x[E];
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = Elem<XDT>::to_f32(ring[lane * E + e]);
        uint32_t code[E];
        const float nrm =
            hadamard_codes_wave<E>(x, a.signs, a.thresholds, (1 << a.key_bits) - 1, tq_inv_sqrt(D), code);
        const int sb = storage_bits(a.key_bits);
        store_codes_wave<E>(code, sb, a.key_codes + (row * C + q) * (D * sb / 8), lane);
        if (lane == 0) a.key_norms[row * C + q] = f32_to_f16_bits(nrm);
      } else {
        const int64_t gs = a.value_group_size, ng = D / gs;
        const int64_t gpt = value_groups_per_run(a.value_bits, D, gs);
        const int64_t pb = D * storage_bits(a.value_bits) / 8;
        for (int64_t r = lane; r < ng / gpt; r += 64)
          quantize_value_run<XDT>(ring, D, a.value_bits, gs, r * gpt, gpt, a.value_data + (row * C + q) * pb,
                                  (T*)a.value_scales + (row * C + q) * ng, (T*)a.value_zeros + (row * C + q) * ng);
      }
    }
  }
  __syncthreads();  // every read of the leaving token is done before its slot is overwritten
  for (int64_t h = wave >> 1; h < H; h += hstep) {
    const int64_t row = b * H + h;
    T* ring = (T*)(is_v ? a.residual_value : a.residual_key) + (row * R + slot) * D;
    const T* src = (const T*)(is_v ? a.new_value : a.new_key) + row * D;
    for (int64_t i = lane; i < D; i += 64) ring[i] = src[i];
  }
  __syncthreads();
  if (threadIdx.x == 0) a.seq_lengths[b] = n + 1;
}

}  // namespace
}  // namespace anna

using namespace anna;

extern "C" int anna_mi_tq_rotation(int64_t D, uint64_t seed, float* out) {
  ANNA_CHECK(out != nullptr && D > 0 && D <= 4096, "anna_mi_tq_rotation: bad arguments");
  make_rotation(D, seed, out);
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_hadamard_signs(int64_t D, uint64_t seed, float* out) {
  ANNA_CHECK(out != nullptr && D > 0 && D <= 4096, "anna_mi_tq_hadamard_signs: bad arguments");
  tq_hadamard_signs(D, seed, out);
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_hadamard_quantize(const void* x, int x_dtype, int64_t nvec, int64_t D, int64_t x_row_stride,
                                           const float* signs, const float* thresholds, int bits, uint8_t* codes,
                                           uint16_t* norms, void* stream) {
  ANNA_CHECK(x && signs && thresholds && codes && norms, "anna_mi_tq_hadamard_quantize: null pointer");
  ANNA_CHECK(valid_dtype(x_dtype), "anna_mi_tq_hadamard_quantize: bad dtype code");
  ANNA_CHECK(bits >= 1 && bits <= 4, "anna_mi_tq_hadamard_quantize: bits must be 1..4");
  ANNA_CHECK(D == 64 || D == 128 || D == 256 || D == 512 || D == 1024,
             "anna_mi_tq_hadamard_quantize: head_dim must be a power of two in [64, 1024]");
  ANNA_CHECK(x_row_stride >= D, "anna_mi_tq_hadamard_quantize: row stride smaller than head_dim");
  if (nvec <= 0) return ANNA_MI_OK;
  const dim3 grid((unsigned)((nvec + 4 * HNV - 1) / (4 * HNV)));
  ANNA_DISPATCH_DTYPE(x_dtype, XDT, {
    auto go = [&](auto e_tag) {
      constexpr int E = decltype(e_tag)::value;
      hipLaunchKernelGGL((tq_hadamard_quantize_kernel<XDT, E>), grid, dim3(256), 0, as_stream(stream),
                         (const typename Elem<XDT>::T*)x, nvec, D, x_row_stride, signs, thresholds, bits, codes, norms);
    };
    switch (D) {
      case 64: go(std::integral_constant<int, 1>{}); break;
      case 128: go(std::integral_constant<int, 2>{}); break;
      case 256: go(std::integral_constant<int, 4>{}); break;
      case 512: go(std::integral_constant<int, 8>{}); break;
      default: go(std::integral_constant<int, 16>{}); break;
    }
  });
  ANNA_LAUNCH_CHECK("tq_hadamard_quantize_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_codebook(int bits, int64_t D, float* centroids, float* thresholds) {
  ANNA_CHECK(bits >= 1 && bits <= 4, "anna_mi_tq_codebook: bits must be 1..4");
  ANNA_CHECK(centroids && thresholds && D > 0, "anna_mi_tq_codebook: bad arguments");
  return tq_codebook(bits, D, centroids, thresholds);
}

extern "C" int anna_mi_tq_mse_quantize(const void* x, int x_dtype, int64_t nvec, int64_t D, int64_t x_row_stride,
                                       const float* rot_t, const float* thresholds, int bits, uint8_t* codes,
                                       uint16_t* norms, void* stream) {
  ANNA_CHECK(x && rot_t && thresholds && codes && norms, "anna_mi_tq_mse_quantize: null pointer");
  ANNA_CHECK(valid_dtype(x_dtype), "anna_mi_tq_mse_quantize: bad dtype code");
  ANNA_CHECK(bits >= 1 && bits <= 4, "anna_mi_tq_mse_quantize: bits must be 1..4");
  ANNA_CHECK(D >= 64 && D <= 1024 && D % 64 == 0, "anna_mi_tq_mse_quantize: head_dim must be a multiple of 64 in [64, 1024]");
  ANNA_CHECK(x_row_stride >= D, "anna_mi_tq_mse_quantize: row stride smaller than head_dim");
  if (nvec <= 0) return ANNA_MI_OK;
  const int vb = tq_vectors_per_wg(D);
  const size_t lds = (size_t)vb * D * 4 + (size_t)vb * D;
  const dim3 grid((unsigned)((nvec + vb - 1) / vb));
  ANNA_DISPATCH_DTYPE(x_dtype, XDT, {
    if (vb == 32)
      hipLaunchKernelGGL((tq_mse_quantize_kernel<XDT, 32>), grid, dim3((unsigned)D), lds, as_stream(stream),
                         (const typename Elem<XDT>::T*)x, nvec, D, x_row_stride, rot_t, thresholds, bits, codes, norms);
    else
      hipLaunchKernelGGL((tq_mse_quantize_kernel<XDT, 16>), grid, dim3((unsigned)D), lds, as_stream(stream),
                         (const typename Elem<XDT>::T*)x, nvec, D, x_row_stride, rot_t, thresholds, bits, codes, norms);
  });
  ANNA_LAUNCH_CHECK("tq_mse_quantize_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_mse_dequant(const uint8_t* codes, const uint16_t* norms, int64_t nvec, int64_t D,
                                      const float* rot, const float* centroids, int bits, void* out, int out_dtype,
                                      int64_t out_row_stride, void* stream) {
  ANNA_CHECK(codes && norms && rot && centroids && out, "anna_mi_tq_mse_dequant: null pointer");
  ANNA_CHECK(valid_dtype(out_dtype), "anna_mi_tq_mse_dequant: bad dtype code");
  ANNA_CHECK(bits >= 1 && bits <= 4, "anna_mi_tq_mse_dequant: bits must be 1..4");
  ANNA_CHECK(D >= 64 && D <= 1024 && D % 64 == 0, "anna_mi_tq_mse_dequant: head_dim must be a multiple of 64 in [64, 1024]");
  if (nvec <= 0) return ANNA_MI_OK;
  const int vb = tq_vectors_per_wg(D);
  const dim3 grid((unsigned)((nvec + vb - 1) / vb));
  ANNA_DISPATCH_DTYPE(out_dtype, ODT, {
    if (vb == 32)
      hipLaunchKernelGGL((tq_mse_dequant_kernel<ODT, 32>), grid, dim3((unsigned)D), (size_t)vb * D * 4,
                         as_stream(stream), codes, norms, nvec, D, rot, centroids, bits,
                         (typename Elem<ODT>::T*)out, out_row_stride);
    else
      hipLaunchKernelGGL((tq_mse_dequant_kernel<ODT, 16>), grid, dim3((unsigned)D), (size_t)vb * D * 4,
                         as_stream(stream), codes, norms, nvec, D, rot, centroids, bits,
                         (typename Elem<ODT>::T*)out, out_row_stride);
  });
  ANNA_LAUNCH_CHECK("tq_mse_dequant_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_values_quantize(const void* values, int dtype, int64_t H, int64_t T, int64_t D,
                                          int64_t stride_h, int64_t stride_t, int bits, int64_t group_size,
                                          uint8_t* data, void* scales, void* zeros, void* stream) {
  ANNA_CHECK(values && data && scales && zeros, "anna_mi_tq_values_quantize: null pointer");
  ANNA_CHECK(valid_dtype(dtype), "anna_mi_tq_values_quantize: bad dtype code");
  ANNA_CHECK(bits == 2 || bits == 3 || bits == 4, "Unsupported TurboQuant value bit-width: %d. Expected 2, 3, or 4.", bits);
  ANNA_CHECK(group_size > 0 && D % group_size == 0,
             "TurboQuant value group_size=%lld must evenly divide head_dim=%lld.", (long long)group_size, (long long)D);
  ANNA_CHECK(D % (8 / storage_bits(bits)) == 0, "packed TurboQuant values need head_dim divisible by the pack width");
  const int64_t gpt = value_groups_per_run(bits, D, group_size);
  const int64_t n = H * T * (D / group_size / gpt);
  if (n <= 0) return ANNA_MI_OK;
  ANNA_DISPATCH_DTYPE(dtype, DT, {
    hipLaunchKernelGGL((tq_values_quantize_kernel<DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       as_stream(stream), (const typename Elem<DT>::T*)values, H, T, D, stride_h, stride_t, bits,
                       group_size, gpt, data, (typename Elem<DT>::T*)scales, (typename Elem<DT>::T*)zeros);
  });
  ANNA_LAUNCH_CHECK("tq_values_quantize_kernel");
  return ANNA_MI_OK;
}

extern "C" int anna_mi_tq_values_dequant(const uint8_t* data, const void* scales, const void* zeros, int dtype,
                                         int64_t rows, int64_t D, int bits, int64_t group_size, void* out,
                                         int out_dtype, void* stream) {
  ANNA_CHECK(data && scales && zeros && out, "anna_mi_tq_values_dequant: null pointer");
  ANNA_CHECK(valid_dtype(dtype) && valid_dtype(out_dtype), "anna_mi_tq_values_dequant: bad dtype code");
  ANNA_CHECK(bits == 2 || bits == 3 || bits == 4, "anna_mi_tq_values_dequant: bits must be 2, 3 or 4");
  ANNA_CHECK(group_size > 0 && D % group_size == 0, "anna_mi_tq_values_dequant: group_size must divide head_dim");
  const int64_t n = rows * D;
  if (n <= 0) return ANNA_MI_OK;
  ANNA_DISPATCH_DTYPE(dtype, DT, {
    ANNA_DISPATCH_DTYPE(out_dtype, ODT, {
      hipLaunchKernelGGL((tq_values_dequant_kernel<DT, ODT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                         as_stream(stream), data, (const typename Elem<DT>::T*)scales,
                         (const typename Elem<DT>::T*)zeros, rows, D, bits, group_size,
                         (typename Elem<ODT>::T*)out);
    });
  });
  ANNA_LAUNCH_CHECK("tq_values_dequant_kernel");
  return ANNA_MI_OK;
}

extern "C" int64_t anna_mi_sizeof_tq_rows_append_args(void) { return (int64_t)sizeof(anna_mi_tq_rows_append_args); }

extern "C" int anna_mi_tq_rows_append(const anna_mi_tq_rows_append_args* ap, void* stream) {
  ANNA_CHECK(ap != nullptr, "anna_mi_tq_rows_append: null args");
  const anna_mi_tq_rows_append_args& a = *ap;
  ANNA_CHECK(valid_dtype(a.dtype), "anna_mi_tq_rows_append: bad dtype code");
  ANNA_CHECK(a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256 || a.head_dim == 512 || a.head_dim == 1024,
             "anna_mi_tq_rows_append: head_dim must be a power of two in [64, 1024]");
  ANNA_CHECK(a.key_bits >= 1 && a.key_bits <= 4, "anna_mi_tq_rows_append: key bits must be 1..4");
  ANNA_CHECK(a.value_bits >= 2 && a.value_bits <= 4, "anna_mi_tq_rows_append: value bits must be 2..4");
  ANNA_CHECK(a.value_group_size > 0 && a.head_dim % a.value_group_size == 0,
             "anna_mi_tq_rows_append: value_group_size must divide head_dim");
  ANNA_CHECK(a.batch > 0 && a.kv_heads > 0 && a.kv_heads <= 4096, "anna_mi_tq_rows_append: 1..4096 KV heads");
  ANNA_CHECK(a.capacity >= 0 && a.residual_capacity > 0, "anna_mi_tq_rows_append: bad capacities");
  ANNA_CHECK(a.new_key && a.new_value && a.residual_key && a.residual_value && a.seq_lengths && a.overflow && a.signs &&
                 a.thresholds && (a.capacity == 0 || (a.key_codes && a.key_norms && a.value_data && a.value_scales &&
                                                      a.value_zeros)),
             "anna_mi_tq_rows_append: null pointer");
  const dim3 grid((unsigned)a.batch), blk((unsigned)(128 * (a.kv_heads < 8 ? a.kv_heads : 8)));
  ANNA_DISPATCH_DTYPE(a.dtype, XDT, {
    auto go = [&](auto e_tag) {
      constexpr int E = decltype(e_tag)::value;
      hipLaunchKernelGGL((tq_rows_append_kernel<XDT, E>), grid, blk, 0, as_stream(stream), a);
    };
    switch (a.head_dim) {
      case 64: go(std::integral_constant<int, 1>{}); break;
      case 128: go(std::integral_constant<int, 2>{}); break;
      case 256: go(std::integral_constant<int, 4>{}); break;
      case 512: go(std::integral_constant<int, 8>{}); break;
      default: go(std::integral_constant<int, 16>{}); break;
    }
  });
  ANNA_LAUNCH_CHECK("tq_rows_append_kernel");
  return ANNA_MI_OK;
}
