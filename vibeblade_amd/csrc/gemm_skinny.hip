// Skinny dequant-fused GEMM on MFMA, M <= 16:  Y[M, N] = X[M, K] . W[N, K]^T
// (W Q4_K in GGUF layout, X fp16 or fp32 row-major, Y fp32 row-major).
//
// Replaces the reference's per-token gemv_dequant loop for small batches
// (speculative verify, cpp/src/fast_model.cpp:644-669).  At M <= 16 the
// product is HBM-bound: every weight byte is read once, so the kernel is
// built around streaming W at full rate.
//
// Work split.  A workgroup owns `rows` (<= 64) consecutive weight rows, i.e.
// four 16-row MFMA column groups, and all of K; its 8 waves split K into
// contiguous super-block ranges, so with about one workgroup per CU every
// activation fragment a wave loads is reused by the four column groups.
//
// Weight loads.  A wave step is one super-block of its rows: rows x 144 bytes
// read as row-contiguous 16-byte pieces (piece p = 64 i + lane, 9 per lane),
// written to a private LDS area in the same order (rows 144 bytes apart) and
// read back in the MFMA B layout.  Loading the B layout straight from HBM
// would touch 16 rows per load instruction, which streams at about two thirds
// of the row-contiguous rate.  Two steps are in flight per wave.
//
// MFMA mapping (v_mfma_f32_16x16x32_f16, mfma_q4k.hpp).  Column j = weight
// row 16 q + j, A row i = token i.  Lane group g always works on chunk g of
// the super-block (sub-blocks 2g, 2g+1: 32 qs bytes): MFMA step s = 0..3
// takes the low nibbles of bytes 8 s .. 8 s + 7 (elements 64 g + 8 s + ..),
// steps 4..7 the high nibbles of the same bytes (elements 64 g + 32 + ..).
// The k order inside an MFMA is free as long as A and B agree, and with the
// weight scales folded into B (w = d sc q - dmin m, rounded once to fp16) the
// four lane groups may sit in different sub-blocks.  Each lane therefore
// decodes only its own two 6-bit scale / min pairs per super-block.
//
// Partial sums of the 8 k-ranges meet in LDS and are added in a fixed order.
#include <type_traits>

#include "mfma_q4k.hpp"
#include "vb_internal.hpp"

namespace vb {
namespace {

constexpr int SK_WAVES = 8;
constexpr int SK_ROWS = 64;                   // max rows per workgroup: 4 column groups
constexpr int SK_PPL = SK_ROWS * 9 / 64;      // 16-byte pieces per lane per step: 9
constexpr int SK_STAGE = SK_ROWS * 144 + 16;  // per-wave LDS bytes (+ one discard slot)
constexpr int SK_X_F32 = 0;
constexpr int SK_X_F16 = 1;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// d * sc and -dmin * m of sub-blocks 2g, 2g+1 as fp16 splats, for a g that
// varies across the wave (get_scale_min_k4, cpp/src/dequant.cpp:258-266):
//   g < 2:  sc = (s03 >> sh) & 0x3F3F,  m = (s47 >> sh) & 0x3F3F
//   g >= 2: sc = ((s8b >> sh) & 0x0F0F) | ((s03 >> (sh + 2)) & 0x3030)
//           m  = ((s8b >> (sh + 4)) & 0x0F0F) | ((s47 >> (sh + 2)) & 0x3030)
// with sh = 16 (g & 1) and s03, s47, s8b = scales[0:4], [4:8], [8:12].
struct LaneScaleSel {
    uint32_t sh, sh2, shm, m1, m2;
    bool hi;
};

__device__ __forceinline__ LaneScaleSel lane_scale_sel(int g) {
    LaneScaleSel q;
    q.hi = g >= 2;
    q.sh = 16u * static_cast<uint32_t>(g & 1);
    q.sh2 = q.sh + 2u;
    q.shm = q.hi ? q.sh + 4u : q.sh;
    q.m1 = q.hi ? 0x0F0Fu : 0x3F3Fu;
    q.m2 = q.hi ? 0x3030u : 0u;
    return q;
}

__device__ __forceinline__ void lane_chunk_scales(const u32x4& hd, const LaneScaleSel& q, half2_t* ds,
                                                  half2_t* nm) {
    const uint32_t s03 = hd.y, s47 = hd.z, s8b = hd.w;
    const uint32_t SC = (((q.hi ? s8b : s03) >> q.sh) & q.m1) | ((s03 >> q.sh2) & q.m2);
    const uint32_t M = (((q.hi ? s8b : s47) >> q.shm) & q.m1) | ((s47 >> q.sh2) & q.m2);
    const float d = f16lo(hd.x), dmin = f16hi(hd.x);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const _Float16 s = static_cast<_Float16>(d * static_cast<float>((SC >> (8 * i)) & 0xFFu));
        const _Float16 m = static_cast<_Float16>(-(dmin * static_cast<float>((M >> (8 * i)) & 0xFFu)));
        ds[i] = half2_t{s, s};
        nm[i] = half2_t{m, m};
    }
}

// Raw activation words of one step: 8 fragments of 8 elements (fp16: one
// 16-byte word each; fp32: two).
template <int XT> struct XWords;
template <> struct XWords<SK_X_F16> { u32x4 v[8]; };
template <> struct XWords<SK_X_F32> { u32x4 v[16]; };

// Buffer loads: a wave-uniform resource (base, size) plus a 32-bit per-lane
// offset and a uniform offset; no 64-bit address arithmetic per lane, and
// offsets past the resource's size read zeros.  Resource word 3 = 0x00020000
// (raw untyped access on gfx9).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}

__device__ __forceinline__ u32x4 buf_ld128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

// Activations of one step for lane (g, token): xoff = the lane's byte offset
// (token row + 64 g elements), soff = the step's first element in bytes.
template <int XT>
__device__ __forceinline__ void load_xwords(__amdgpu_buffer_rsrc_t xr, uint32_t xoff, uint32_t soff, XWords<XT>& xw) {
    constexpr uint32_t ES = XT == SK_X_F16 ? 2u : 4u;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const uint32_t k = 32u * (s >> 2) + 8u * (s & 3);
        if constexpr (XT == SK_X_F16) {
            xw.v[s] = buf_ld128(xr, xoff + ES * k, soff);
        } else {
            xw.v[2 * s] = buf_ld128(xr, xoff + ES * k, soff);
            xw.v[2 * s + 1] = buf_ld128(xr, xoff + ES * k + 16u, soff);
        }
    }
}

// Fragments in natural k order (q4k_bfrags_nat2): fp16 words are used as
// loaded (tokens >= M read zeros).
template <int XT>
__device__ __forceinline__ void xwords_to_frags(const XWords<XT>& xw, Frag* a) {
#pragma unroll
    for (int s = 0; s < 8; s++) {
        if constexpr (XT == SK_X_F16) {
            const u32x4 v = xw.v[s];
            a[s].u[0] = v.x;
            a[s].u[1] = v.y;
            a[s].u[2] = v.z;
            a[s].u[3] = v.w;
        } else {
            const u32x4 lo = xw.v[2 * s], hi = xw.v[2 * s + 1];
            const float4 f0 = make_float4(__uint_as_float(lo.x), __uint_as_float(lo.y), __uint_as_float(lo.z),
                                          __uint_as_float(lo.w));
            const float4 f1 = make_float4(__uint_as_float(hi.x), __uint_as_float(hi.y), __uint_as_float(hi.z),
                                          __uint_as_float(hi.w));
            f32x8_to_frag_nat(f0, f1, a[s].u);
        }
    }
}

template <int XT>
__global__ void __launch_bounds__(64 * SK_WAVES) gemm_q4k_skinny_kernel(
        const uint8_t* __restrict__ w, const uint8_t* __restrict__ X, float* __restrict__ Y, int M, int N,
        int K, int rb, int rows, int nsb, uint32_t wbytes, uint32_t xbytes) {
    extern __shared__ u32x4 sk_lds[];
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row0 = static_cast<int>(blockIdx.x) * rows;
    const int sb0 = __builtin_amdgcn_readfirstlane((wave * nsb) / SK_WAVES);
    const int sb1 = __builtin_amdgcn_readfirstlane(((wave + 1) * nsb) / SK_WAVES);
    const int nsteps = sb1 - sb0;  // 0 when nsb < 8 for some waves
    uint8_t* stage = reinterpret_cast<uint8_t*>(sk_lds) + wave * SK_STAGE;

    // Pieces of this lane: p = 64 i + lane -> row p / 9, word p % 9 of the
    // step's rows x 144-byte block; pieces past the block reload the last
    // one and land in the discard slot.
    const int npieces = rows * 9;
    uint32_t poff[SK_PPL], soff[SK_PPL];
#pragma unroll
    for (int i = 0; i < SK_PPL; i++) {
        const int p = 64 * i + lane;
        const int pc = p < npieces ? p : npieces - 1;
        const int r = pc / 9, wd = pc - 9 * r;
        int row = row0 + r;
        row = row < N ? row : N - 1;
        poff[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(rb) + 16u * static_cast<uint32_t>(wd);
        soff[i] = p < npieces ? 16u * static_cast<uint32_t>(p) : static_cast<uint32_t>(SK_ROWS * 144);
    }
    // A row of this lane: token j; tokens >= M point past the resource and
    // read zeros.
    constexpr uint32_t ES = XT == SK_X_F16 ? 2u : 4u;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, wbytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(X, xbytes);
    const uint32_t xoff = j < M ? (static_cast<uint32_t>(j) * static_cast<uint32_t>(K) + 64u * g) * ES : 0x80000000u;
    const LaneScaleSel sel = lane_scale_sel(g);
    const NatConsts kc = nat_consts();

    // Weights run two steps ahead (ring of two register buffers), the
    // activations (L2-resident) one step: gfx9 loads retire in order, so the
    // step-s activations are issued before the step-(s+2) weights.  fp16
    // activations feed the MFMAs as loaded and need a buffer per slot; fp32
    // ones are converted first, after which their buffer is free again.
    constexpr int XB = XT == SK_X_F16 ? 2 : 1;
    u32x4 pv[2][SK_PPL];
    XWords<XT> xw[XB];
    int itw = 0, itx = 0;
    // Ring slots are compile-time constants so the buffers stay in registers.
    auto issue_w = [&](auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value;
        int sb = sb0 + itw;
        sb = sb < nsb - 1 ? sb : nsb - 1;  // padding steps reload the last super-block
#pragma unroll
        for (int i = 0; i < SK_PPL; i++) pv[slot][i] = buf_ld128(wr, poff[i], static_cast<uint32_t>(sb) * 144u);
        ++itw;
    };
    auto issue_x = [&](auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value % XB;
        int sb = sb0 + itx;
        sb = sb < nsb - 1 ? sb : nsb - 1;
        load_xwords<XT>(xr, xoff, static_cast<uint32_t>(sb) * 256u * ES, xw[slot]);
        ++itx;
    };

    float4_t acc[4];
#pragma unroll
    for (int q = 0; q < 4; q++) acc[q] = float4_t{0.f, 0.f, 0.f, 0.f};
    int ct = 0;
    auto compute = [&](auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value;
        if (ct >= nsteps) return;  // padding step (uniform)
        Frag a[8];
        xwords_to_frags<XT>(xw[slot % XB], a);
        issue_x(std::integral_constant<int, slot ^ 1>{});  // next step's activations, ahead of its weights
#pragma unroll
        for (int i = 0; i < SK_PPL; i++) *reinterpret_cast<u32x4*>(stage + soff[i]) = pv[slot][i];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint8_t* rp = stage + (16 * q + j) * 144;
            const u32x4 hd = *reinterpret_cast<const u32x4*>(rp);
            const u32x4 qa = *reinterpret_cast<const u32x4*>(rp + 16 + 32 * g);
            const u32x4 qb = *reinterpret_cast<const u32x4*>(rp + 32 + 32 * g);
            half2_t ds[2], nm[2];
            lane_chunk_scales(hd, sel, ds, nm);
            const uint32_t qd[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int s = 0; s < 4; s++) {
                Frag lo, hi;
                q4k_bfrags_nat2(qd[2 * s], qd[2 * s + 1], ds, nm, kc, lo, hi);
                acc[q] = mfma16x16x32(a[s], lo, acc[q]);
                acc[q] = mfma16x16x32(a[4 + s], hi, acc[q]);
            }
        }
        ++ct;
    };

    const int nsteps_p = nsteps <= 2 ? 2 : ((nsteps + 1) & ~1);
    issue_w(std::integral_constant<int, 0>{});
    issue_x(std::integral_constant<int, 0>{});
    issue_w(std::integral_constant<int, 1>{});
    for (int s = 0; s + 2 < nsteps_p; s += 2) {
        compute(std::integral_constant<int, 0>{});
        issue_w(std::integral_constant<int, 0>{});
        compute(std::integral_constant<int, 1>{});
        issue_w(std::integral_constant<int, 1>{});
    }
    compute(std::integral_constant<int, 0>{});
    compute(std::integral_constant<int, 1>{});

    // k-range partials meet in LDS (over the staging areas), fixed order.
    __syncthreads();
    float4_t* red = reinterpret_cast<float4_t*>(sk_lds);  // [wave][q][lane]
#pragma unroll
    for (int q = 0; q < 4; q++) red[(wave * 4 + q) * 64 + lane] = acc[q];
    __syncthreads();
    for (int e = threadIdx.x; e < 256; e += blockDim.x) {
        const int q = e >> 6, l = e & 63;
        float4_t s = red[q * 64 + l];
#pragma unroll
        for (int v = 1; v < SK_WAVES; v++) s += red[(v * 4 + q) * 64 + l];
        const int r = 16 * q + (l & 15), n = row0 + r;
        if (r < rows && n < N) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 4 * (l >> 4) + i;
                if (t < M) Y[static_cast<int64_t>(t) * N + n] = s[i];
            }
        }
    }
}

}  // namespace

// Caller (gemm_dispatch) has validated type, M <= 16, alignment (W, X 16 B).
int gemm_q4k_skinny(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K,
                    hipStream_t st) {
    const int64_t nsb = K / 256, rb = nsb * 144;
    const int64_t xbytes = M * K * (x_dtype == SK_X_F16 ? 2 : 4);
    if (N > INT32_MAX || K > INT32_MAX || N * rb >= (int64_t(1) << 32) || xbytes >= (int64_t(1) << 31)) {
        set_error("vb_gemm: shape too large for the skinny kernel (N=%lld K=%lld)", static_cast<long long>(N),
                  static_cast<long long>(K));
        return E_INVAL;
    }
    // about one workgroup per CU, 16..64 rows each
    int64_t rows = (N + 255) / 256;
    rows = rows < 16 ? 16 : (rows > SK_ROWS ? SK_ROWS : rows);
    const dim3 grid(static_cast<uint32_t>((N + rows - 1) / rows)), block(64 * SK_WAVES);
    const size_t lds = static_cast<size_t>(SK_WAVES) * SK_STAGE;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const uint8_t* xb = static_cast<const uint8_t*>(X);
    if (x_dtype == SK_X_F16)
        gemm_q4k_skinny_kernel<SK_X_F16><<<grid, block, lds, st>>>(wb, xb, Y, static_cast<int>(M), static_cast<int>(N),
                                                                   static_cast<int>(K), static_cast<int>(rb),
                                                                   static_cast<int>(rows), static_cast<int>(nsb),
                                                                   static_cast<uint32_t>(N * rb), static_cast<uint32_t>(xbytes));
    else
        gemm_q4k_skinny_kernel<SK_X_F32><<<grid, block, lds, st>>>(wb, xb, Y, static_cast<int>(M), static_cast<int>(N),
                                                                   static_cast<int>(K), static_cast<int>(rb),
                                                                   static_cast<int>(rows), static_cast<int>(nsb),
                                                                   static_cast<uint32_t>(N * rb), static_cast<uint32_t>(xbytes));
    return check_launch("vb_gemm");
}

}  // namespace vb
