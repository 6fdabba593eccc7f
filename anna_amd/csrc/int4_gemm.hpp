// Internal interface of the tiled W4A16 GEMM (int4_gemm.hip), used by anna_mi_int4_linear.
#pragma once

#include "common.hpp"

namespace anna {

bool int4_gemm_tiled_supported(int x_dtype, int64_t M, int64_t N, int64_t K, int64_t xs, const void* x, const void* qweight,
                               int64_t pc, const void* qscale, const void* qzeros, int64_t gsz);

int int4_gemm_tiled_launch(const void* x, int x_dtype, int64_t M, int64_t K, int64_t xs, const int32_t* qweight,
                           int64_t N, int64_t pc, const void* qscale, int scale_dtype, const int8_t* qzeros, int64_t gsz,
                           void* y, hipStream_t st);

// Skinny form for small M (32 rows of x per workgroup against 48 rows of W over all of K; group 128).
int64_t int4_gemm_skinny_workgroups(int64_t M, int64_t N);
bool int4_gemm_skinny_supported(int x_dtype, int64_t M, int64_t N, int64_t K, int64_t xs, const void* x,
                                const void* qweight, int64_t pc, int64_t gsz);

int int4_gemm_skinny_launch(const void* x, int x_dtype, int64_t M, int64_t K, int64_t xs, const int32_t* qweight,
                            int64_t N, int64_t pc, const void* qscale, int scale_dtype, const int8_t* qzeros,
                            void* y, hipStream_t st);

}  // namespace anna
