// Dequant-fused GEMM on MFMA:  Y[M, N] = X[M, K] . W[N, K]^T  (W Q4_K, GGUF
// layout; X fp16 or fp32 row-major; Y fp32 row-major).
//
// The reference runs batched tokens as a per-token loop of gemv_dequant
// (cpp/src/fast_model.cpp:644-669, :905-960), re-streaming every weight once
// per token; cuda::gemm_f32 (cpp/src/cuda_kernels.cu:184-212) needs fp32
// weights.  Here weights are streamed once per M-tile and dequantized to fp16
// in registers, in the B-operand layout of v_mfma_f32_16x16x32_f16
// (mfma_q4k.hpp), accumulating in fp32.
//
// Two kernels:
//  * skinny (M <= 16: speculative verify, MoE expert groups): one 16-row
//    M-fragment; a workgroup owns 16 output columns and splits K over its 4
//    waves (partials meet in LDS).  HBM-bound: the grid has N/16 workgroups.
//  * tiled (M > 16: chunked prefill): 256 x 128 output tile per workgroup,
//    2 x 2 waves of 128 x 64.  X is staged through LDS (double-buffered
//    64-element k-chunks, sigma-permuted, rows padded to 144 B so the
//    fragment reads are bank-conflict free); each wave dequantizes its 64
//    weight rows straight into B fragments.  One barrier per k-chunk.
#include <cstdlib>

#include "mfma_q4k.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int X_F32 = 0;
constexpr int X_F16 = 1;

// A fragment (rows t of X, k0 + 8g .. +8) in sigma order; zeros when !valid.
template <int XT>
__device__ __forceinline__ void load_afrag(const void* X, int64_t ldx, int64_t t, int64_t k, bool valid,
                                           Frag& a) {
    if (!valid) {
        a.u[0] = a.u[1] = a.u[2] = a.u[3] = 0u;
        return;
    }
    if constexpr (XT == X_F16) {
        const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const __half*>(X) + t * ldx + k);
        sigma_permute(v.x, v.y, v.z, v.w, a.u);
    } else {
        const float* p = static_cast<const float*>(X) + t * ldx + k;
        f32x8_to_frag(*reinterpret_cast<const float4*>(p), *reinterpret_cast<const float4*>(p + 4), a.u);
    }
}

// ---- skinny: M <= 16 --------------------------------------------------------

template <int XT>
__global__ void __launch_bounds__(256) gemm_q4k_skinny(const uint8_t* __restrict__ w,
                                                       const void* __restrict__ X, float* __restrict__ Y,
                                                       int M, int64_t N, int64_t K, int64_t rb) {
    __shared__ float4_t red[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    int64_t n = n0 + j;
    n = n < N ? n : N - 1;
    const uint8_t* row = w + n * rb;
    const int nsb = static_cast<int>(K / 256);
    const int sb0 = (wave * nsb) / 4, sb1 = ((wave + 1) * nsb) / 4;
    const bool tvalid = j < M;  // A-fragment row of this lane
    float4_t acc = {0.f, 0.f, 0.f, 0.f};

    uint4 hd;
    uint2 qs[4];
    auto load_w = [&](int sb) {
        const uint8_t* b = row + static_cast<int64_t>(sb) * 144;
        hd = *reinterpret_cast<const uint4*>(b);
#pragma unroll
        for (int c = 0; c < 4; c++) qs[c] = *reinterpret_cast<const uint2*>(b + 16 + 32 * c + 8 * g);
    };
    if (sb0 < sb1) load_w(sb0);
    for (int sb = sb0; sb < sb1; sb++) {
        const uint4 hcur = hd;
        uint2 qcur[4];
#pragma unroll
        for (int c = 0; c < 4; c++) qcur[c] = qs[c];
        if (sb + 1 < sb1) load_w(sb + 1);
        Frag a[8];
#pragma unroll
        for (int sub = 0; sub < 8; sub++)
            load_afrag<XT>(X, K, j, static_cast<int64_t>(sb) * 256 + 32 * sub + 8 * g, tvalid, a[sub]);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            half2_t ds[2], nm[2];
            q4k_chunk_scales(hcur, c, ds, nm);
            Frag lo, hi;
            q4k_bfrags(qcur[c].x, qcur[c].y, ds, nm, lo, hi);
            acc = mfma16x16x32(a[2 * c], lo, acc);
            acc = mfma16x16x32(a[2 * c + 1], hi, acc);
        }
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        const float4_t s = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
        const int64_t col = n0 + j;
        if (col < N) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = 4 * g + r;
                if (t < M) Y[static_cast<int64_t>(t) * N + col] = s[r];
            }
        }
    }
}

// ---- tiled: M > 16 ------------------------------------------------------------

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int XS_STRIDE = BK + 8;  // halves per LDS row (144 bytes)
constexpr int MF = 8, NF = 4;      // fragments per wave (128 x 64)

template <int XT>
__global__ void __launch_bounds__(256) gemm_q4k_tiled(const uint8_t* __restrict__ w,
                                                      const void* __restrict__ X, float* __restrict__ Y,
                                                      int64_t M, int64_t N, int64_t K, int64_t rb) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][BM * XS_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int j = lane & 15, g = lane >> 4;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;
    const int nchunks = static_cast<int>(K / BK);

    // weight rows of this lane's 4 B fragments
    const uint8_t* wrow[NF];
#pragma unroll
    for (int f = 0; f < NF; f++) {
        int64_t n = n0 + wn * 64 + 16 * f + j;
        n = n < N ? n : N - 1;
        wrow[f] = w + n * rb;
    }

    // X staging: thread owns 8 16-byte pieces (row = q/8, part = q%8).
    uint32_t xr[8][4];
    auto load_x = [&](int ch) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int q = tid + 256 * i;
            const int r = q >> 3, part = q & 7;
            const int64_t t = m0 + r;
            Frag f;
            load_afrag<XT>(X, K, t < M ? t : 0, static_cast<int64_t>(ch) * BK + 8 * part, t < M, f);
#pragma unroll
            for (int e = 0; e < 4; e++) xr[i][e] = f.u[e];
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int q = tid + 256 * i;
            const int r = q >> 3, part = q & 7;
            *reinterpret_cast<uint4*>(&xs[buf][r * XS_STRIDE + 8 * part]) =
                make_uint4(xr[i][0], xr[i][1], xr[i][2], xr[i][3]);
        }
    };
    uint4 hd[NF];
    uint2 qv[NF];
    auto load_w = [&](int ch) {
        const int sb = ch >> 2, c = ch & 3;
#pragma unroll
        for (int f = 0; f < NF; f++) {
            const uint8_t* b = wrow[f] + static_cast<int64_t>(sb) * 144;
            if (c == 0) hd[f] = *reinterpret_cast<const uint4*>(b);
            qv[f] = *reinterpret_cast<const uint2*>(b + 16 + 32 * c + 8 * g);
        }
    };

    float4_t acc[MF][NF];
#pragma unroll
    for (int a = 0; a < MF; a++)
#pragma unroll
        for (int b = 0; b < NF; b++) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    load_x(0);
    load_w(0);
    store_x(0);
    for (int ch = 0; ch < nchunks; ch++) {
        const int buf = ch & 1, c = ch & 3;
        // dequantize this chunk's B fragments from the registers loaded last step
        Frag blo[NF], bhi[NF];
#pragma unroll
        for (int f = 0; f < NF; f++) {
            half2_t ds[2], nm[2];
            q4k_chunk_scales(hd[f], c, ds, nm);
            q4k_bfrags(qv[f].x, qv[f].y, ds, nm, blo[f], bhi[f]);
        }
        if (ch + 1 < nchunks) {
            load_x(ch + 1);
            load_w(ch + 1);
        }
        __syncthreads();  // chunk ch of X is in xs[buf]; chunk ch-1 readers are done
        const _Float16* xb = xs[buf];
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
#pragma unroll
            for (int a = 0; a < MF; a++) {
                Frag af;
                const int r = wm * 128 + 16 * a + j;
                const uint4 v = *reinterpret_cast<const uint4*>(&xb[r * XS_STRIDE + 32 * ks + 8 * g]);
                af.u[0] = v.x; af.u[1] = v.y; af.u[2] = v.z; af.u[3] = v.w;
#pragma unroll
                for (int b = 0; b < NF; b++)
                    acc[a][b] = mfma16x16x32(af, ks == 0 ? blo[b] : bhi[b], acc[a][b]);
            }
        }
        if (ch + 1 < nchunks) store_x(buf ^ 1);
    }

#pragma unroll
    for (int a = 0; a < MF; a++) {
#pragma unroll
        for (int b = 0; b < NF; b++) {
            const int64_t col = n0 + wn * 64 + 16 * b + j;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t t = m0 + wm * 128 + 16 * a + 4 * g + r;
                if (t < M) Y[t * N + col] = acc[a][b][r];
            }
        }
    }
}

}  // namespace

int gemm_dispatch(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K,
                  int32_t type, int32_t variant, hipStream_t st) {
    if (type != TYPE_Q4_K) {
        set_error("vb_gemm: weight type %d has no MFMA path yet (Q4_K only)", type);
        return E_UNSUPPORTED;
    }
    const int64_t rb = row_bytes(type, K);
    if (rb < 0 || M < 0 || N < 0 || (x_dtype != X_F32 && x_dtype != X_F16)) {
        set_error("vb_gemm: bad arguments (type=%d K=%lld x_dtype=%d)", type, static_cast<long long>(K), x_dtype);
        return E_INVAL;
    }
    if (M == 0 || N == 0) return OK;
    if (!w || !X || !Y) {
        set_error("vb_gemm: null pointer");
        return E_INVAL;
    }
    if (reinterpret_cast<uintptr_t>(w) % 16 || reinterpret_cast<uintptr_t>(X) % 16) {
        set_error("vb_gemm: W and X must be 16-byte aligned");
        return E_INVAL;
    }
    const bool skinny = variant == 1 || (variant == 0 && M <= 16);
    if (skinny) {
        if (M > 16) {
            set_error("vb_gemm: variant 1 (skinny) takes M <= 16, got %lld", static_cast<long long>(M));
            return E_INVAL;
        }
        const dim3 grid(static_cast<uint32_t>((N + 15) / 16));
        if (x_dtype == X_F16)
            gemm_q4k_skinny<X_F16><<<grid, dim3(256), 0, st>>>(static_cast<const uint8_t*>(w), X, Y,
                                                               static_cast<int>(M), N, K, rb);
        else
            gemm_q4k_skinny<X_F32><<<grid, dim3(256), 0, st>>>(static_cast<const uint8_t*>(w), X, Y,
                                                               static_cast<int>(M), N, K, rb);
        return check_launch("vb_gemm");
    }
    if (variant != 0 && variant != 2) {
        set_error("vb_gemm: unknown variant %d", variant);
        return E_INVAL;
    }
    const dim3 grid(static_cast<uint32_t>((N + BN - 1) / BN), static_cast<uint32_t>((M + BM - 1) / BM));
    if (grid.y > 65535) {
        set_error("vb_gemm: M too large");
        return E_INVAL;
    }
    if (x_dtype == X_F16)
        gemm_q4k_tiled<X_F16><<<grid, dim3(256), 0, st>>>(static_cast<const uint8_t*>(w), X, Y, M, N, K, rb);
    else
        gemm_q4k_tiled<X_F32><<<grid, dim3(256), 0, st>>>(static_cast<const uint8_t*>(w), X, Y, M, N, K, rb);
    return check_launch("vb_gemm");
}

}  // namespace vb

extern "C" int vb_gemm(const void* w, const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n,
                       int64_t k, int32_t ggml_type, int32_t variant, void* stream) {
    return vb::gemm_dispatch(w, x, x_dtype, y, m, n, k, ggml_type, variant, vb::as_stream(stream));
}
