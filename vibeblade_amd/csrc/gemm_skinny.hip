// Skinny dequant-fused GEMM on MFMA, M <= 16:  Y[M, N] = X[M, K] . W[N, K]^T
// (W Q4_K in GGUF layout, X fp16 or fp32 row-major, Y fp32 row-major).
//
// Replaces the reference's per-token gemv_dequant loop for small batches
// (speculative verify, cpp/src/fast_model.cpp:644-669).  At M <= 16 the
// product is HBM-bound: every weight byte is read once.  One workgroup per
// skinny::tile (skinny_core.hpp) of up to 64 weight rows; about one
// workgroup per CU, so each activation fragment serves four column groups.
#include "skinny_core.hpp"
#include "vb_internal.hpp"

namespace vb {
namespace {

template <int XT>
__global__ void __launch_bounds__(64 * skinny::WAVES) gemm_q4k_skinny_kernel(
        const uint8_t* __restrict__ w, const uint8_t* __restrict__ X, float* __restrict__ Y, int M, int N, int K,
        int rb, int rows, int nsb, uint32_t wbytes, uint32_t xbytes) {
    extern __shared__ skinny::u32x4 sk_lds[];
    constexpr uint32_t ES = XT == skinny::X_F16 ? 2u : 4u;
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    skinny::TileArgs<1> ta;
    ta.w[0] = skinny::make_rsrc(w, wbytes);
    ta.x = skinny::make_rsrc(X, xbytes);
    // A row of this lane: token j; tokens >= M read zeros
    ta.xoff = j < M ? (static_cast<uint32_t>(j) * static_cast<uint32_t>(K) + 64u * g) * ES : skinny::X_NONE;
    ta.row0 = static_cast<int>(blockIdx.x) * rows;
    ta.rows = rows;
    ta.nrows = N;
    ta.rb = rb;
    ta.nsb = nsb;
    float4_t s[1];
    skinny::tile<XT, 1>(ta, reinterpret_cast<uint8_t*>(sk_lds), s);
    if (threadIdx.x < 256) {
        const int q = threadIdx.x >> 6, l = threadIdx.x & 63;
        const int r = 16 * q + (l & 15), n = ta.row0 + r;
        if (r < rows && n < N) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 4 * (l >> 4) + i;
                if (t < M) Y[static_cast<int64_t>(t) * N + n] = s[0][i];
            }
        }
    }
}

}  // namespace

// Caller (gemm_dispatch) has validated type, M <= 16, alignment (W, X 16 B).
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
    if (x_dtype == skinny::X_F16)
        gemm_q4k_skinny_kernel<skinny::X_F16><<<grid, block, lds, st>>>(wb, xb, Y, m, n, k, rbi, rowsi, nsbi, wbytes, xby);
    else
        gemm_q4k_skinny_kernel<skinny::X_F32><<<grid, block, lds, st>>>(wb, xb, Y, m, n, k, rbi, rowsi, nsbi, wbytes, xby);
    return check_launch("vb_gemm");
}

}  // namespace vb
