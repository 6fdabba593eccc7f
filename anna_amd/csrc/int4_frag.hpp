// Shared int4 -> MFMA / dot2 fragment helpers (W4A16 kernels of int4_linear.hip, lm_head.hip
// and moe.hip).
#pragma once

#include "common.hpp"

namespace anna {

// Turn 8 nibbles of `w` into 8 exact "off + q" values in the 16-bit float format of
// the MFMA: element 2p is nibble p, element 2p+1 is nibble p+4.
template <int XDT>
__device__ __forceinline__ u32x4 nibbles_to_frag(uint32_t w) {
  // The magic constant is materialized in a VGPR (one VOP1 move, hoisted by the
  // compiler) so that each pair is a single v_and_or_b32 (mask in an SGPR): VOP3 on
  // gfx9 takes no literal operands.
  constexpr uint32_t MAGIC = XDT == ANNA_MI_BF16 ? 0x43004300u : 0x64006400u;
  uint32_t magic;
  asm("v_mov_b32 %0, %1" : "=v"(magic) : "i"(MAGIC));
  u32x4 r;
  r.x = (w & 0x000F000Fu) | magic;
  r.y = ((w >> 4) & 0x000F000Fu) | magic;
  r.z = ((w >> 8) & 0x000F000Fu) | magic;
  r.w = ((w >> 12) & 0x000F000Fu) | magic;
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

// c + a.lo * b.lo + a.hi * b.hi over two packed 16-bit values (bf16 or f16), fp32 accumulation.
template <int XDT>
__device__ __forceinline__ float dot2_acc(uint32_t a, uint32_t b, float c) {
  if constexpr (XDT == ANNA_MI_BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  }
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

}  // namespace anna
