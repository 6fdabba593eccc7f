// Shared helpers for the anna_mi HIP library (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/anna_mi.h"

namespace anna {

// ---------------------------------------------------------------- errors
// Every C-ABI entry point returns 0 on success or a nonzero ANNA_MI_E* code;
// the message of the last failure on the calling thread is kept here.
void set_error(const char* fmt, ...);
int fail_hip(hipError_t e, const char* what);

#define ANNA_CHECK(cond, ...)                       \
  do {                                              \
    if (!(cond)) {                                  \
      ::anna::set_error(__VA_ARGS__);               \
      return ANNA_MI_EINVAL;                        \
    }                                               \
  } while (0)

#define ANNA_LAUNCH_CHECK(what)                                  \
  do {                                                           \
    hipError_t _e = hipGetLastError();                           \
    if (_e != hipSuccess) return ::anna::fail_hip(_e, what);     \
  } while (0)

// ---------------------------------------------------------------- vectors
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- scalars
// Storage types are moved as raw 16-bit patterns; conversions are explicit and
// round to nearest even, the rounding torch's `.to(dtype)` uses.
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const __bf16 v = (__bf16)f;  // v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN
  return __builtin_bit_cast(uint16_t, v);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// dtype codes of anna_mi.h: ANNA_MI_BF16, ANNA_MI_F16, ANNA_MI_F32
template <int DT> struct Elem;
template <> struct Elem<ANNA_MI_BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ T cvt(float f) { return f32_to_bf16_bits(f); }
  static __device__ __forceinline__ float to_f32(T v) { return bf16_bits_to_f32(v); }
};
template <> struct Elem<ANNA_MI_F16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return f16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ T cvt(float f) { return f32_to_f16_bits(f); }
  static __device__ __forceinline__ float to_f32(T v) { return f16_bits_to_f32(v); }
};
template <> struct Elem<ANNA_MI_F32> {
  typedef float T;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ T cvt(float f) { return f; }
  static __device__ __forceinline__ float to_f32(T v) { return v; }
};

inline bool valid_dtype(int dt) { return dt == ANNA_MI_BF16 || dt == ANNA_MI_F16 || dt == ANNA_MI_F32; }

// Dispatch a runtime dtype code to a compile-time template argument.
#define ANNA_DISPATCH_DTYPE(dt, NAME, ...)                                   \
  switch (dt) {                                                              \
    case ANNA_MI_BF16: { constexpr int NAME = ANNA_MI_BF16; __VA_ARGS__; break; } \
    case ANNA_MI_F16:  { constexpr int NAME = ANNA_MI_F16;  __VA_ARGS__; break; } \
    case ANNA_MI_F32:  { constexpr int NAME = ANNA_MI_F32;  __VA_ARGS__; break; } \
    default: ::anna::set_error("unsupported dtype code %d", (int)(dt)); return ANNA_MI_EINVAL; \
  }

// ---------------------------------------------------------------- wave ops
// Value of lane l ^ 16 and of lane l ^ 32 (all 64 lanes active): gfx950's row swaps, one VALU
// instruction and a select instead of a round trip through the LDS pipe.  v_permlane16_swap of
// (v, v) returns {rows 0, 0, 2, 2; rows 1, 1, 3, 3} (16-lane rows), v_permlane32_swap of (v, v)
// {lanes 0-31 twice; lanes 32-63 twice}; a lane takes the copy of the other row.
__device__ __forceinline__ int32_t lane_xor16(int32_t v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (threadIdx.x & 16) ? (int32_t)r[0] : (int32_t)r[1];
}
__device__ __forceinline__ int32_t lane_xor32(int32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? (int32_t)r[0] : (int32_t)r[1];
}
__device__ __forceinline__ float lane_xor16(float v) { return __int_as_float(lane_xor16(__float_as_int(v))); }
__device__ __forceinline__ float lane_xor32(float v) { return __int_as_float(lane_xor32(__float_as_int(v))); }

// Sum over the wave (all 64 lanes active), every lane ending with the total, with no LDS-pipe
// round trip: DPP pairings inside 16-lane rows (quad xor 1, quad xor 2, i <-> 7 - i, i <-> 15 - i)
// then the two row swaps.  Its summation order differs from wave_sum's xor tree.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_rows(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  v += lane_xor16(v);
  return v + lane_xor32(v);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup p runs on XCD p % 8).
// Remapping p to a tile index this way hands each XCD a contiguous range of tiles, so
// tiles that share cache lines (neighbouring rows of scales / zero points) meet in one L2.
constexpr int NUM_XCD = 8;
__device__ __forceinline__ int64_t xcd_tile(int64_t p, int64_t tiles) {
  if (tiles % NUM_XCD != 0) return p;
  return (p % NUM_XCD) * (tiles / NUM_XCD) + p / NUM_XCD;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace anna
