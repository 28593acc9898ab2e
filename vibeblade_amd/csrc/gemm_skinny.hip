// Skinny dequant-fused GEMM on MFMA, M <= 32:  Y[M, N] = X[M, K] . W[N, K]^T
// (W Q4_K in GGUF layout, X fp16 or fp32 row-major, Y fp32 row-major).
//
// Replaces the reference's per-token gemv_dequant loop for small batches
// (speculative verify, cpp/src/fast_model.cpp:644-669).  At M <= 32 the
// weight stream and its dequantization dominate: every weight byte is read
// and decoded once.  One workgroup per
// skinny::tile (skinny_core.hpp) of up to 64 weight rows; about one
// workgroup per CU, so each activation fragment serves four column groups.
#include "skinny_core.hpp"
#include "vb_internal.hpp"

namespace vb {
namespace {

// MT activation tiles of 16 rows (M <= 16 MT): every dequantized weight
// fragment feeds MT MFMAs.  MT = 2 runs 4-wave workgroups, so a wave may
// hold the two tiles' activation fragments and accumulators (292 / 332
// registers for fp16 / fp32 X, no spills) with 4 super-blocks of K each.
template <int XT, int MT, int NW>
__global__ void __launch_bounds__(64 * NW) gemm_q4k_skinny_kernel(
        const uint8_t* __restrict__ w, const uint8_t* __restrict__ X, float* __restrict__ Y, int M, int N, int K,
        int rb, int rows, int nsb, uint32_t wbytes, uint32_t xbytes) {
    extern __shared__ skinny::u32x4 sk_lds[];
    constexpr uint32_t ES = XT == skinny::X_F16 ? 2u : 4u;
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    skinny::TileArgs<1, MT> ta;
    ta.w[0] = skinny::make_rsrc(w, wbytes);
    ta.x = skinny::make_rsrc(X, xbytes);
    // A rows of this lane: tokens 16 mt + j; tokens >= M read zeros
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int t = 16 * mt + j;
        ta.xoff[mt] = t < M ? (static_cast<uint32_t>(t) * static_cast<uint32_t>(K) + 64u * g) * ES : skinny::X_NONE;
    }
    ta.row0 = static_cast<int>(blockIdx.x) * rows;
    ta.rows = rows;
    ta.nrows = N;
    ta.rb = rb;
    ta.nsb = nsb;
    float4_t s[MT];
    skinny::tile<XT, 1, 2, NW, MT>(ta, reinterpret_cast<uint8_t*>(sk_lds), s);
    if (threadIdx.x < 256) {
        const int q = threadIdx.x >> 6, l = threadIdx.x & 63;
        const int r = 16 * q + (l & 15), n = ta.row0 + r;
        if (r < rows && n < N) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 16 * mt + 4 * (l >> 4) + i;
                    if (t < M) Y[static_cast<int64_t>(t) * N + n] = s[mt][i];
                }
            }
        }
    }
}

}  // namespace

// Caller (gemm_dispatch) has validated type, M <= 32 (M <= 64 with fp16 X),
// alignment (W, X 16 B).
int gemm_q4k_skinny(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K,
                    hipStream_t st) {
    const int64_t nsb = K / 256, rb = nsb * 144;
    const int64_t xbytes = M * K * (x_dtype == skinny::X_F16 ? 2 : 4);
    if (N > INT32_MAX || K > INT32_MAX || N * rb >= (int64_t(1) << 32) || xbytes >= (int64_t(1) << 31)) {
        set_error("vb_gemm: shape too large for the skinny kernel (N=%lld K=%lld)", static_cast<long long>(N),
                  static_cast<long long>(K));
        return E_INVAL;
    }
    // about one workgroup per CU, 16..64 rows each
    int64_t rows = (N + 255) / 256;
    rows = rows < 16 ? 16 : (rows > skinny::ROWS ? skinny::ROWS : rows);
    const dim3 grid(static_cast<uint32_t>((N + rows - 1) / rows)), block(64 * skinny::WAVES);
    const size_t lds = skinny::LDS_BYTES;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const uint8_t* xb = static_cast<const uint8_t*>(X);
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    const int rbi = static_cast<int>(rb), rowsi = static_cast<int>(rows), nsbi = static_cast<int>(nsb);
    const uint32_t wbytes = static_cast<uint32_t>(N * rb), xby = static_cast<uint32_t>(xbytes);
    if (M > 32) {
        // four activation tiles (fp16 X): 4-wave workgroups, one per CU
        if (x_dtype != skinny::X_F16 || M > 64) {
            set_error("vb_gemm: the skinny kernel takes M <= 32 (M <= 64 with fp16 X), got %lld",
                      static_cast<long long>(M));
            return E_INVAL;
        }
        constexpr int NW4 = 4;
        gemm_q4k_skinny_kernel<skinny::X_F16, 4, NW4><<<grid, dim3(64 * NW4), skinny::lds_bytes_mt<NW4, 4, 1>(), st>>>(
            wb, xb, Y, m, n, k, rbi, rowsi, nsbi, wbytes, xby);
    } else if (M > 16) {
        // two activation tiles: 4-wave workgroups (the register file of a
        // SIMD to one wave), one per CU
        constexpr int NW2 = 4;
        const size_t lds2 = skinny::lds_bytes<NW2>();
        if (x_dtype == skinny::X_F16)
            gemm_q4k_skinny_kernel<skinny::X_F16, 2, NW2><<<grid, dim3(64 * NW2), lds2, st>>>(
                wb, xb, Y, m, n, k, rbi, rowsi, nsbi, wbytes, xby);
        else
            gemm_q4k_skinny_kernel<skinny::X_F32, 2, NW2><<<grid, dim3(64 * NW2), lds2, st>>>(
                wb, xb, Y, m, n, k, rbi, rowsi, nsbi, wbytes, xby);
    } else if (x_dtype == skinny::X_F16) {
        gemm_q4k_skinny_kernel<skinny::X_F16, 1, skinny::WAVES><<<grid, block, lds, st>>>(wb, xb, Y, m, n, k, rbi, rowsi,
                                                                                         nsbi, wbytes, xby);
    } else {
        gemm_q4k_skinny_kernel<skinny::X_F32, 1, skinny::WAVES><<<grid, block, lds, st>>>(wb, xb, Y, m, n, k, rbi, rowsi,
                                                                                         nsbi, wbytes, xby);
    }
    return check_launch("vb_gemm");
}

}  // namespace vb
