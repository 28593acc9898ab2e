// Entry points shared between translation units of libvbhip (not exported).
#pragma once

#include "vb_common.hpp"

namespace vb {

// Rows of a GEMV launch: plain (row r of w), or gathered gate/up pairs of a
// sparse FFN (row r = row gidx[r/2] of w for even r, of w2 for odd r).  zbuf
// / zn: an int buffer the launch clears (counters of a following kernel).
struct RowSrc {
    const void* w2 = nullptr;
    const int32_t* gidx = nullptr;
    int64_t nsrc = 0;  // rows of w / w2; gathered indices are clamped to [0, nsrc)
    int* zbuf = nullptr;
    int zn = 0;
};

int gemv_dispatch(const void* w, const float* x, float* y, int64_t n, int64_t k, int32_t type,
                  hipStream_t st);
int gemv_dispatch_src(const void* w, const RowSrc& src, const float* x, float* y, int64_t n, int64_t k,
                      int32_t type, hipStream_t st);
// Q4_K M=1 GEMV on the int8 matrix cores (gemv_q4k_mfma.hip); arguments
// already validated by gemv_dispatch_src.
int gemv_q4k_mfma(const void* w, const RowSrc& src, const float* x, float* y, int64_t n, int64_t k,
                  hipStream_t st);
// M <= 16 Q4_K GEMM (gemm_skinny.hip); type, M, alignment already validated.
int gemm_q4k_skinny(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K,
                    hipStream_t st);
int gemm_dispatch(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K,
                  int32_t type, int32_t variant, hipStream_t st);

}  // namespace vb
