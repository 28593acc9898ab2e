// Batched dequant-fused GEMM for Q6_K, Q8_0 and Q5_K weights (and Q4_K at
// some small-M shapes) on MFMA:
//   Y[M, N] = X[M, K] . W[N, K]^T   (W in GGUF layout, X fp16 or fp32
//   row-major, Y fp32 row-major).
//
// Replaces the reference's batched path for these types, a per-token loop of
// gemv_dequant over rows decoded by dequantize_row (cpp/src/fast_model.cpp:
// 905-960, cpp/src/dequant.cpp:407-425): a Q4_K_M file keeps its ffn_down,
// attn_v and output tensors in Q6_K, and Q8_0 files use Q8_0 throughout.
//
// Design.  A workgroup of 8 waves owns a tile of 16 MA activation rows x
// 16 NCG weight rows and splits K between its waves (contiguous ranges of
// 128-element steps).  Every wave keeps both operands in registers:
//  * A: fragment (a, ks) of a step is X[16 a + j][128 s + 32 ks + 8 g, +8)
//    for lane (j, g), loaded from global memory (L2) at the start of the step;
//  * B: for each column group the wave decodes one "unit" per lane (weight
//    row 16 cg + j, the 8 elements 8 g .. of each 32-element k-step of the
//    128-element step) into four fp16 fragments, w rounded to fp16, from raw
//    bytes it loaded RD steps earlier.
// Each weight is therefore decoded once per M-tile and each activation
// loaded once per N-tile, with no LDS staging; the 8 partial tiles meet in
// LDS at the end and are added in a fixed order (deterministic output).
//
// The k order inside an MFMA is free as long as A and B agree; both use the
// natural order: lane (j, g) of k-step ks holds elements 32 ks + 8 g + 0..7
// of the step, and the Q6_K and Q8_0 layouts put exactly those elements in
// 8 consecutive bytes per lane (below).
//
// GGUF rows of these types are only 2-byte aligned (210- and 34-byte
// blocks), so each 8-byte field is read as the three dwords from its
// address rounded down to 4 and realigned with v_alignbyte; the weight
// resource spans the tensor rounded up to whole dwords (the last dword
// holds tensor bytes, so it is mapped memory).
#include <type_traits>

#include "mfma_q4k.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int KQ_WAVES = 8;
constexpr int KQ_STEP = 128;                 // elements per step: four MFMA k-steps
constexpr uint32_t KQ_X_NONE = 0x80000000u;  // lane offset of an absent activation row (reads zeros)
constexpr int KQ_X_F32 = 0;
constexpr int KQ_X_F16 = 1;

struct KqExperts {
    const uint8_t* p[MOE_KQ_MAX_EXPERTS];
};

template <int TYPE> struct Kq;

// Q4_K (cpp/src/dequant.cpp:258-301; header d, dmin, scales[12] @0, qs[128]
// @16, rows 16-byte aligned): a step is half a super-block, chunks c = 2 h
// and 2 h + 1; k-step 2 (c - 2 h) takes the low nibbles of qs bytes
// [32 c + 8 g, +8) (sub-block 2 c), k-step 2 (c - 2 h) + 1 their high
// nibbles (sub-block 2 c + 1).
template <>
struct Kq<TYPE_Q4_K> {
    static constexpr bool kBlockLane = false;
    struct Raw {
        u32x4 hd;
        uint2 q[2];
    };
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, int g,
                                                 Raw& r) {
        const uint32_t base = rowoff + static_cast<uint32_t>(step >> 1) * 144u;
        const uint32_t qo = base + 16u + 64u * static_cast<uint32_t>(step & 1) + 8u * static_cast<uint32_t>(g);
        r.hd = buf_ld128(w, base, 0);
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(w, static_cast<int>(qo + 32u * c), 0, 0);
            r.q[c] = make_uint2(v[0], v[1]);
        }
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t, int step, int, const KqConsts&, Frag* f) {
        const uint4 hd = make_uint4(r.hd.x, r.hd.y, r.hd.z, r.hd.w);
#pragma unroll
        for (int c = 0; c < 2; c++) {
            half2_t ds[2], nm[2];
            q4k_chunk_scales(hd, 2 * (step & 1) + c, ds, nm);
            q4k_bfrags_nat(r.q[c].x, r.q[c].y, ds, nm, f[2 * c], f[2 * c + 1]);
        }
    }
};

// Q5_K (super-block of 256, 176 bytes: the Q4_K header d, dmin, scales[12]
// @0, qh[32] @16, qs[128] @48; rows 16-byte aligned): a step is half a
// super-block, chunks c = 2 h and 2 h + 1, as for Q4_K; lane group g also
// takes qh bytes [8 g, +8), whose bits 2 c, 2 c + 1 are the fifth bits of the
// chunk's two sub-blocks (q5k_frags).
template <>
struct Kq<TYPE_Q5_K> {
    static constexpr bool kBlockLane = false;
    struct Raw {
        u32x4 hd;
        uint2 q[2];
        uint2 h;
    };
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, int g,
                                                 Raw& r) {
        const uint32_t base = rowoff + static_cast<uint32_t>(step >> 1) * 176u;
        const uint32_t g8 = 8u * static_cast<uint32_t>(g);
        const uint32_t qo = base + 48u + 64u * static_cast<uint32_t>(step & 1) + g8;
        r.hd = buf_ld128(w, base, 0);
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(w, static_cast<int>(qo + 32u * c), 0, 0);
            r.q[c] = make_uint2(v[0], v[1]);
        }
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(w, static_cast<int>(base + 16u + g8), 0, 0);
        r.h = make_uint2(v[0], v[1]);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t, int step, int, const KqConsts& kc,
                                                  Frag* f) {
        const uint4 hd = make_uint4(r.hd.x, r.hd.y, r.hd.z, r.hd.w);
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int cc = 2 * (step & 1) + c;
            half2_t ds[2], nm[2];
            q4k_chunk_scales(hd, cc, ds, nm);
            q5k_frags(r.q[c].x, r.q[c].y, r.h.x, r.h.y, static_cast<uint32_t>(cc), ds, nm, kc, f[2 * c],
                      f[2 * c + 1]);
        }
    }
};

// Q6_K in the GGUF layout (the layout of real files and of the known answers
// in tests/test_kquants.py:134-175; cpp/src/dequant.cpp:359-402 gathers the
// elements in another order): super-block of 256 = two halves h of 128
// elements; bytes ql[128] @0, qh[64] @128, int8
// scales[16] @192, fp16 d @208.  In half h, element l + 32 t (l < 32, t < 4)
// is q - 32 with q = (ql[64 h + l + 32 (t & 1)] >> 4 (t >> 1)) & 15 |
// ((qh[32 h + l] >> 2 t) & 3) << 4, scaled by d * scales[8 h + l / 16 + 2 t].
// A step is one half; k-step ks = t, so lane (j, g) needs ql bytes
// [64 h + 8 g, +8) (t = 0, 2) and [64 h + 32 + 8 g, +8) (t = 1, 3), qh bytes
// [32 h + 8 g, +8), the scales 8 h + g / 2 + 2 t and d.
template <>
struct Kq<TYPE_Q6_K> {
    static constexpr bool kBlockLane = false;
    struct Raw {
        u32x3 l0, l1, qh;
        uint32_t sd;  // lane group g: dword g of (scales of the half: 12 bytes from their dword, d's dword)
    };
    // every field offset is a multiple of 4 from the super-block start, so
    // one shift (the start's offset within its dword) serves all of them
    __device__ static __forceinline__ uint32_t shift(uint32_t rowoff, int step) {
        return (rowoff + static_cast<uint32_t>(step >> 1) * 210u) & 3u;
    }
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, int g,
                                                 Raw& r) {
        const uint32_t base = (rowoff + static_cast<uint32_t>(step >> 1) * 210u) & ~3u;
        const uint32_t h = static_cast<uint32_t>(step & 1), g8 = 8u * static_cast<uint32_t>(g);
        r.l0 = ld96(w, base + 64u * h + g8);
        r.l1 = ld96(w, base + 64u * h + 32u + g8);
        r.qh = ld96(w, base + 128u + 32u * h + g8);
        // the four lane groups of a row share its scales and d: one dword each
        r.sd = ld32(w, g < 3 ? base + 192u + 8u * h + 4u * static_cast<uint32_t>(g) : base + 208u);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t rowoff, int step, int g, const KqConsts& kc,
                                                  Frag* f) {
        const uint32_t sh = shift(rowoff, step);
        // scale dwords 0-2 and d's dword from lane groups 0-3: the pair's
        // even / odd 16-lane rows, then the lower / upper halves of the wave
        const auto p16 = __builtin_amdgcn_permlane16_swap(r.sd, r.sd, false, false);
        const auto e32 = __builtin_amdgcn_permlane32_swap(p16[0], p16[0], false, false);
        const auto o32 = __builtin_amdgcn_permlane32_swap(p16[1], p16[1], false, false);
        const u32x3 scw = {e32[0], o32[0], e32[1]};
        uint32_t l0[2], l1[2], qh[2], sc[2];
        realign(r.l0, sh, l0[0], l0[1]);
        realign(r.l1, sh, l1[0], l1[1]);
        realign(r.qh, sh, qh[0], qh[1]);
        realign(scw, sh, sc[0], sc[1]);
        const float d = f16lo(o32[1] >> (8u * sh));
        // scale bytes g / 2 + {0, 2, 4, 6} of the half's eight
        const uint32_t P = __builtin_amdgcn_perm(sc[1], sc[0], g >= 2 ? 0x07050301u : 0x06040200u);
        half2_t dsc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int8_t s = static_cast<int8_t>((P >> (8 * t)) & 0xFFu);
            const _Float16 v = static_cast<_Float16>(d * static_cast<float>(s));
            dsc[t] = half2_t{v, v};
        }
        const half2_t k1056 = half2_t{static_cast<_Float16>(1056.0f), static_cast<_Float16>(1056.0f)};
#pragma unroll
        for (int dw = 0; dw < 2; dw++) {
            // four 6-bit codes per dword: run t takes nibble t / 2 of l0 (t
            // even) or l1 (t odd) and qh bits 2 t, 2 t + 1, moved to bits 4, 5
            // of the same byte
            uint32_t q[4];
            q[0] = ((qh[dw] << 4) & 0x30303030u) | (l0[dw] & 0x0F0F0F0Fu);
            q[1] = ((qh[dw] << 2) & 0x30303030u) | (l1[dw] & 0x0F0F0F0Fu);
            q[2] = (qh[dw] & 0x30303030u) | ((l0[dw] >> 4) & 0x0F0F0F0Fu);
            q[3] = ((qh[dw] >> 2) & 0x30303030u) | ((l1[dw] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                // bytes (0, 1) and (2, 3) into fp16 halves 1024 + q (exact)
                f[t].u[2 * dw] = h2bits((bits2h(__builtin_amdgcn_perm(kc.h64, q[t], 0x07010500u)) - k1056) * dsc[t]);
                f[t].u[2 * dw + 1] =
                    h2bits((bits2h(__builtin_amdgcn_perm(kc.h64, q[t], 0x07030502u)) - k1056) * dsc[t]);
            }
        }
    }
};

// Q8_0 in the GGUF layout (vibeblade/loader.py:129-133,
// cpp/src/cuda_kernels.cu:718-735): blocks of 32 = fp16 d @0, int8 qs[32]
// @2.  A step is four blocks.  Lane group g takes block 4 s + g whole (one
// 34-byte read, one scale) and k-step ks its codes [8 ks, +8): the "block
// per lane group" k order, which the activation fragments follow (kBlockLane).
// Rows are whole dwords (K % 128 == 0: 136-byte steps), so block g starts
// 2 g bytes into a dword modulo 4.
template <>
struct Kq<TYPE_Q8_0> {
    static constexpr bool kBlockLane = true;
    struct Raw {
        u32x3 q[3];  // 36 bytes from the block's dword
    };
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, int g,
                                                 Raw& r) {
        const uint32_t a = (rowoff + static_cast<uint32_t>(step) * 136u + 34u * static_cast<uint32_t>(g)) & ~3u;
#pragma unroll
        for (int i = 0; i < 3; i++) r.q[i] = ld96(w, a + 12u * i);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t rowoff, int, int g, const KqConsts& kc,
                                                  Frag* f) {
        const uint32_t w[9] = {r.q[0].x, r.q[0].y, r.q[0].z, r.q[1].x, r.q[1].y, r.q[1].z, r.q[2].x, r.q[2].y,
                               r.q[2].z};
        const bool odd = ((rowoff + 2u * static_cast<uint32_t>(g)) & 3u) != 0;  // block at byte 2 of its dword
        // d at bytes [0, 2) or [2, 4); codes at byte 2 (realign by 2) or 4 (dword 1)
        const uint32_t d16 = odd ? (w[0] >> 16) : (w[0] & 0xFFFFu);
        const half2_t dd = bits2h(d16 | (d16 << 16));
        const half2_t k1152 = half2_t{static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            uint32_t qs[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int i = 2 * ks + h;
                qs[h] = odd ? w[i + 1] : __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2u);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // bytes (b0, b1) into the two halves; (b ^ 0x80) | 0x6400 is
                // the half 1024 + q + 128 (exact)
                const uint32_t src = __builtin_amdgcn_perm(0u, qs[i >> 1], (i & 1) ? 0x0C030C02u : 0x0C010C00u);
                f[ks].u[i] = h2bits((bits2h(src ^ kc.x80) - k1152) * dd);
            }
        }
    }
};

// Q4_0 / Q4_1 / Q5_0 / Q5_1 (B32 in mfma_q4k.hpp): as Q8_0, a step is four
// blocks, lane group g takes block 4 s + g whole and k-step ks its codes
// [8 ks, +8) (kBlockLane).  The block (18-24 bytes) is read as the six
// dwords from its start rounded down to 4 (rows are multiples of 8 bytes at
// K % 128 == 0, so 18- and 22-byte blocks start 2 (g % 2) bytes into a
// dword) and realigned.
template <int TYPE>
struct KqB32 {
    static constexpr bool kBlockLane = true;
    using B = B32<TYPE>;
    struct Raw {
        u32x3 q[2];
    };
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, int g,
                                                 Raw& r) {
        const uint32_t a = (rowoff + (4u * static_cast<uint32_t>(step) + static_cast<uint32_t>(g)) * B::kBytes) & ~3u;
        r.q[0] = ld96(w, a);
        r.q[1] = ld96(w, a + 12u);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t rowoff, int, int g, const KqConsts& kc,
                                                  Frag* f) {
        const uint32_t w[6] = {r.q[0].x, r.q[0].y, r.q[0].z, r.q[1].x, r.q[1].y, r.q[1].z};
        const uint32_t sh = (rowoff + static_cast<uint32_t>(g) * B::kBytes) & 3u;  // 0 or 2
#pragma unroll
        for (int ks = 0; ks < 4; ks++) b32_block_frag<TYPE>(w, sh, ks, kc, f[ks]);
    }
};
template <> struct Kq<TYPE_Q4_0> : KqB32<TYPE_Q4_0> {};
template <> struct Kq<TYPE_Q4_1> : KqB32<TYPE_Q4_1> {};
template <> struct Kq<TYPE_Q5_0> : KqB32<TYPE_Q5_0> {};
template <> struct Kq<TYPE_Q5_1> : KqB32<TYPE_Q5_1> {};

// X fragments of one step: A[ks][a] for activation rows 16 a + j.
template <int XT, int MA>
struct XFrags {
    u32x4 v[4][MA][XT == KQ_X_F16 ? 1 : 2];
};

template <int TYPE, int XT, int MA, int NCG, int RD>
__global__ void __launch_bounds__(64 * KQ_WAVES) gemm_kq_kernel(const uint8_t* __restrict__ w, uint32_t wbytes,
                                                                const uint8_t* __restrict__ X, uint32_t xbytes,
                                                                float* __restrict__ Y, int M, int N, int K,
                                                                uint32_t rb) {
    using T = Kq<TYPE>;
    extern __shared__ float4_t kq_red[];  // [wave][MA * NCG][lane]
    constexpr uint32_t ES = XT == KQ_X_F16 ? 2u : 4u;
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int n0 = static_cast<int>(blockIdx.x) * 16 * NCG;
    const int m0 = static_cast<int>(blockIdx.y) * 16 * MA;
    const int nsteps = K / KQ_STEP;
    const int s_beg = __builtin_amdgcn_readfirstlane((wave * nsteps) / KQ_WAVES);
    const int s_end = __builtin_amdgcn_readfirstlane(((wave + 1) * nsteps) / KQ_WAVES);

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, wbytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(X, xbytes);
    uint32_t rowoff[NCG];  // weight rows 16 cg + j (rows past N repeat row N - 1; never stored)
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        int n = n0 + 16 * cg + j;
        n = n < N ? n : N - 1;
        rowoff[cg] = static_cast<uint32_t>(n) * rb;
    }
    // k order of a step: natural (lane group g holds elements 32 ks + 8 g ..
    // of k-step ks) or block per lane group (32 g + 8 ks ..)
    constexpr uint32_t GSTR = T::kBlockLane ? 32u : 8u, KSTR = T::kBlockLane ? 8u : 32u;
    uint32_t xoff[MA];  // activation rows 16 a + j (+ the lane group's elements); rows past M read zeros
#pragma unroll
    for (int a = 0; a < MA; a++) {
        const int t = m0 + 16 * a + j;
        xoff[a] = t < M ? (static_cast<uint32_t>(t) * static_cast<uint32_t>(K) + GSTR * static_cast<uint32_t>(g)) * ES
                        : KQ_X_NONE;
    }
    const KqConsts kc = kq_consts();

    float4_t acc[MA][NCG];
#pragma unroll
    for (int a = 0; a < MA; a++)
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) acc[a][cg] = float4_t{0.f, 0.f, 0.f, 0.f};

    typename T::Raw raw[RD][NCG];
    const int last = s_end - 1;
    auto issue = [&](int slot, int step) {
        step = step < last ? step : last;  // past the wave's range: repeats its last step, unused
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) T::issue(wr, rowoff[cg], step, g, raw[slot][cg]);
    };
    if (s_end > s_beg) {
#pragma unroll
        for (int r = 0; r < RD; r++) issue(r, s_beg + r);
        for (int it = s_beg; it < s_end; it += RD) {
#pragma unroll
            for (int r = 0; r < RD; r++) {
                const int step = it + r;
                if (step >= s_end) break;  // uniform
                XFrags<XT, MA> xf;
                const uint32_t so = static_cast<uint32_t>(step) * KQ_STEP * ES;
#pragma unroll
                for (int ks = 0; ks < 4; ks++)
#pragma unroll
                    for (int a = 0; a < MA; a++) {
                        xf.v[ks][a][0] = buf_ld128(xr, xoff[a], so + KSTR * ES * ks);
                        if constexpr (XT == KQ_X_F32) xf.v[ks][a][1] = buf_ld128(xr, xoff[a], so + KSTR * ES * ks + 16u);
                    }
                Frag af[4][MA];
#pragma unroll
                for (int ks = 0; ks < 4; ks++)
#pragma unroll
                    for (int a = 0; a < MA; a++) {
                        if constexpr (XT == KQ_X_F16) {
                            const u32x4 v = xf.v[ks][a][0];
                            af[ks][a].u[0] = v.x; af[ks][a].u[1] = v.y; af[ks][a].u[2] = v.z; af[ks][a].u[3] = v.w;
                        } else {
                            const u32x4 lo = xf.v[ks][a][0], hi = xf.v[ks][a][1];
                            f32x8_to_frag_nat(make_float4(__uint_as_float(lo.x), __uint_as_float(lo.y),
                                                          __uint_as_float(lo.z), __uint_as_float(lo.w)),
                                              make_float4(__uint_as_float(hi.x), __uint_as_float(hi.y),
                                                          __uint_as_float(hi.z), __uint_as_float(hi.w)),
                                              af[ks][a].u);
                        }
                    }
#pragma unroll
                for (int cg = 0; cg < NCG; cg++) {
                    Frag bf[4];
                    T::decode(raw[r][cg], rowoff[cg], step, g, kc, bf);
                    T::issue(wr, rowoff[cg], (step + RD) < last ? step + RD : last, g, raw[r][cg]);
#pragma unroll
                    for (int ks = 0; ks < 4; ks++)
#pragma unroll
                        for (int a = 0; a < MA; a++) acc[a][cg] = mfma16x16x32(af[ks][a], bf[ks], acc[a][cg]);
                }
            }
        }
    }

    // k-range partials meet in LDS and are added in wave order
#pragma unroll
    for (int a = 0; a < MA; a++)
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) kq_red[(wave * MA * NCG + a * NCG + cg) * 64 + lane] = acc[a][cg];
    __syncthreads();
    for (int e = threadIdx.x; e < MA * NCG * 64; e += 64 * KQ_WAVES) {
        float4_t s = kq_red[e];
#pragma unroll
        for (int v = 1; v < KQ_WAVES; v++) s += kq_red[v * MA * NCG * 64 + e];
        const int idx = e >> 6, l = e & 63, a = idx / NCG, cg = idx - a * NCG;
        const int col = n0 + 16 * cg + (l & 15);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = m0 + 16 * a + 4 * (l >> 4) + r;
            if (t < M) Y[static_cast<int64_t>(t) * N + col] = s[r];
        }
    }
}

// Expert-grouped form for the MoE FFN (moe.hip): workgroup (n-tile, expert
// e) walks expert e's routed slots (elist[eoff[e] .. eoff[e + 1])) 16 at a
// time, with the same k split, decoders and fixed-order reduction as
// gemm_kq_kernel.  Activation rows are gathered: slot q reads row q / xdiv of
// X (fp16; xdiv = topk for the tokens' rows, 1 for the hidden rows of the
// slots).  NMAT = 2: gate and up weights over the same rows, written as fp16
// silu(g) * u into hout[slot][n]; NMAT = 1: fp32 into fout[slot][n], or
// with yacc (top-k <= 2) rw[slot] times it added atomically to
// yacc[slot / topk][n], which the caller has zeroed.
template <int TYPE, int NMAT, int NCG, int RD>
__global__ void __launch_bounds__(64 * KQ_WAVES) moe_kq_kernel(KqExperts w0, KqExperts w1, uint32_t wbytes,
                                                               const uint8_t* __restrict__ X, uint32_t xbytes,
                                                               int xdiv, const int32_t* __restrict__ eoff,
                                                               const int32_t* __restrict__ elist, int nslots,
                                                               int N, int K,
                                                               uint32_t rb, _Float16* __restrict__ hout,
                                                               float* __restrict__ fout,
                                                               const float* __restrict__ rw, int topk,
                                                               float* __restrict__ yacc) {
    using T = Kq<TYPE>;
    extern __shared__ float4_t kq_red[];  // [wave][NMAT * NCG][lane]
    const int e = static_cast<int>(blockIdx.y);
    const SlotRange slots = expert_slots(eoff, elist, e, nslots);
    const int cnt = slots.count;
    if (cnt <= 0) return;
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int n0 = static_cast<int>(blockIdx.x) * 16 * NCG;
    const int nsteps = K / KQ_STEP;
    const int s_beg = __builtin_amdgcn_readfirstlane((wave * nsteps) / KQ_WAVES);
    const int s_end = __builtin_amdgcn_readfirstlane(((wave + 1) * nsteps) / KQ_WAVES);
    __amdgpu_buffer_rsrc_t wr[NMAT];
    wr[0] = make_rsrc(w0.p[e], wbytes);
    if constexpr (NMAT == 2) wr[1] = make_rsrc(w1.p[e], wbytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(X, xbytes);
    uint32_t rowoff[NCG];
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        int n = n0 + 16 * cg + j;
        n = n < N ? n : N - 1;
        rowoff[cg] = static_cast<uint32_t>(n) * rb;
    }
    constexpr uint32_t GSTR = T::kBlockLane ? 32u : 8u, KSTR = T::kBlockLane ? 8u : 32u;
    const KqConsts kc = kq_consts();
    const int last = s_end - 1;
    for (int m0 = 0; m0 < cnt; m0 += 16) {
        const int nrow = cnt - m0 < 16 ? cnt - m0 : 16;
        const uint32_t xoff = j < nrow ? (static_cast<uint32_t>(slots[m0 + j] / xdiv) * static_cast<uint32_t>(K) +
                                          GSTR * static_cast<uint32_t>(g)) * 2u
                                       : KQ_X_NONE;
        float4_t acc[NMAT][NCG];
#pragma unroll
        for (int mt = 0; mt < NMAT; mt++)
#pragma unroll
            for (int cg = 0; cg < NCG; cg++) acc[mt][cg] = float4_t{0.f, 0.f, 0.f, 0.f};
        typename T::Raw raw[RD][NMAT][NCG];
        if (s_end > s_beg) {
#pragma unroll
            for (int r = 0; r < RD; r++) {
                const int step = s_beg + r < last ? s_beg + r : last;
#pragma unroll
                for (int mt = 0; mt < NMAT; mt++)
#pragma unroll
                    for (int cg = 0; cg < NCG; cg++) T::issue(wr[mt], rowoff[cg], step, g, raw[r][mt][cg]);
            }
            for (int it = s_beg; it < s_end; it += RD) {
#pragma unroll
                for (int r = 0; r < RD; r++) {
                    const int step = it + r;
                    if (step >= s_end) break;  // uniform
                    const uint32_t so = static_cast<uint32_t>(step) * KQ_STEP * 2u;
                    Frag af[4];
#pragma unroll
                    for (int ks = 0; ks < 4; ks++) {
                        const u32x4 v = buf_ld128(xr, xoff, so + KSTR * 2u * ks);
                        af[ks].u[0] = v.x; af[ks].u[1] = v.y; af[ks].u[2] = v.z; af[ks].u[3] = v.w;
                    }
                    const int nxt = (step + RD) < last ? step + RD : last;
#pragma unroll
                    for (int mt = 0; mt < NMAT; mt++)
#pragma unroll
                        for (int cg = 0; cg < NCG; cg++) {
                            Frag bf[4];
                            T::decode(raw[r][mt][cg], rowoff[cg], step, g, kc, bf);
                            T::issue(wr[mt], rowoff[cg], nxt, g, raw[r][mt][cg]);
#pragma unroll
                            for (int ks = 0; ks < 4; ks++) acc[mt][cg] = mfma16x16x32(af[ks], bf[ks], acc[mt][cg]);
                        }
                }
            }
        }
#pragma unroll
        for (int mt = 0; mt < NMAT; mt++)
#pragma unroll
            for (int cg = 0; cg < NCG; cg++) kq_red[(wave * NMAT * NCG + mt * NCG + cg) * 64 + lane] = acc[mt][cg];
        __syncthreads();
        for (int q = threadIdx.x; q < NCG * 64; q += 64 * KQ_WAVES) {
            const int cg = q >> 6, l = q & 63;
            float4_t s0 = kq_red[cg * 64 + l];
#pragma unroll
            for (int v = 1; v < KQ_WAVES; v++) s0 += kq_red[(v * NMAT * NCG + cg) * 64 + l];
            float4_t s1 = s0;
            if constexpr (NMAT == 2) {
                s1 = kq_red[(NCG + cg) * 64 + l];
#pragma unroll
                for (int v = 1; v < KQ_WAVES; v++) s1 += kq_red[(v * NMAT * NCG + NCG + cg) * 64 + l];
            }
            const int col = n0 + 16 * cg + (l & 15);
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = 4 * (l >> 4) + r;
                if (t >= nrow) continue;
                const int64_t o = static_cast<int64_t>(slots[m0 + t]) * N + col;
                if constexpr (NMAT == 2) {
                    hout[o] = static_cast<_Float16>(s0[r] / (1.0f + __expf(-s0[r])) * s1[r]);
                } else if (yacc) {
                    // the token's weighted sum over its (at most two) slots:
                    // two additions into zero, in either order the same bits
                    const int q = slots[m0 + t];
                    unsafeAtomicAdd(yacc + static_cast<int64_t>(q / topk) * N + col, rw[q] * s0[r]);
                } else {
                    fout[o] = s0[r];
                }
            }
        }
        __syncthreads();  // kq_red is rewritten by the next 16 slots
    }
}

template <int TYPE, int XT, int MA, int NCG, int RD>
void launch_kq(const uint8_t* w, uint32_t wbytes, const uint8_t* X, uint32_t xbytes, float* Y, int M, int N, int K,
               uint32_t rb, hipStream_t st) {
    const dim3 grid(static_cast<uint32_t>((N + 16 * NCG - 1) / (16 * NCG)),
                    static_cast<uint32_t>((M + 16 * MA - 1) / (16 * MA)));
    const size_t lds = static_cast<size_t>(KQ_WAVES) * MA * NCG * 64 * sizeof(float4_t);
    gemm_kq_kernel<TYPE, XT, MA, NCG, RD><<<grid, dim3(64 * KQ_WAVES), lds, st>>>(w, wbytes, X, xbytes, Y, M, N, K,
                                                                                  rb);
}

// Tile by M and N.  M <= 16: 16-row M tiles and 16-64 weight rows per
// workgroup (enough workgroups at N = 4096 to fill the CUs), raw weight bytes
// two or three steps ahead.  M <= 64: one M tile of 16 ceil(M / 16) rows, so
// every weight is decoded once; at N >= 12288 64 weight rows per workgroup
// (X re-read N / 64 times, at least 192 workgroups) with the raw bytes one
// step ahead, below 16 (two steps ahead).  Above: 64 x 64 tiles (fp32 X:
// 32 x 64, its fragments take twice the registers), one step ahead.  Deeper
// rings measured slower on MI355X at every M (Q4_K 14336 x 4096, M = 17:
// 28.6 us at four steps against 21.3 at one).
template <int TYPE, int XT, int MA>
void launch_kq_mid(const uint8_t* w, uint32_t wbytes, const uint8_t* X, uint32_t xbytes, float* Y, int M, int N,
                   int K, uint32_t rb, hipStream_t st) {
    if (N >= 12288)
        launch_kq<TYPE, XT, MA, 4, 1>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
    else
        launch_kq<TYPE, XT, MA, 1, 2>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
}

template <int TYPE, int XT>
void launch_kq_m(const uint8_t* w, uint32_t wbytes, const uint8_t* X, uint32_t xbytes, float* Y, int M, int N, int K,
                 uint32_t rb, hipStream_t st) {
    if (M <= 16) {
        if (N >= 16384)
            launch_kq<TYPE, XT, 1, 4, 2>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
        else if (N >= 8192)
            launch_kq<TYPE, XT, 1, 2, 2>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
        else
            launch_kq<TYPE, XT, 1, 1, 3>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
    } else if (M <= 32) {
        launch_kq_mid<TYPE, XT, 2>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
    } else if (M <= 48) {
        launch_kq_mid<TYPE, XT, 3>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
    } else if (M <= 64) {
        launch_kq_mid<TYPE, XT, 4>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
    } else if constexpr (XT == KQ_X_F16) {
        launch_kq<TYPE, XT, 4, 4, 1>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
    } else {
        launch_kq<TYPE, XT, 2, 4, 1>(w, wbytes, X, xbytes, Y, M, N, K, rb, st);
    }
}

}  // namespace

// Caller (gemm_dispatch) has checked M, N > 0, pointers, X 16-byte alignment
// and x_dtype.
int gemm_kq(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K, int32_t type,
            hipStream_t st) {
    if (K % KQ_STEP != 0) {
        set_error("vb_gemm: the K-split kernel needs K %% 128 == 0 (K=%lld)", static_cast<long long>(K));
        return E_UNSUPPORTED;
    }
    const int64_t rb = row_bytes(type, K);
    const int64_t wbytes = (N * rb + 3) & ~int64_t(3);
    const int64_t xbytes = M * K * (x_dtype == KQ_X_F16 ? 2 : 4);
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || (M + 15) / 16 > 65535 || wbytes >= (int64_t(1) << 32) ||
        xbytes >= (int64_t(1) << 31)) {
        set_error("vb_gemm: shape too large (M=%lld N=%lld K=%lld)", static_cast<long long>(M),
                  static_cast<long long>(N), static_cast<long long>(K));
        return E_INVAL;
    }
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const uint8_t* xb = static_cast<const uint8_t*>(X);
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    const uint32_t wby = static_cast<uint32_t>(wbytes), xby = static_cast<uint32_t>(xbytes),
                   rbu = static_cast<uint32_t>(rb);
    if (type == TYPE_Q4_K) {
        if (x_dtype == KQ_X_F16)
            launch_kq_m<TYPE_Q4_K, KQ_X_F16>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
        else
            launch_kq_m<TYPE_Q4_K, KQ_X_F32>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
    } else if (type == TYPE_Q5_K) {
        if (x_dtype == KQ_X_F16)
            launch_kq_m<TYPE_Q5_K, KQ_X_F16>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
        else
            launch_kq_m<TYPE_Q5_K, KQ_X_F32>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
    } else if (type == TYPE_Q4_0 || type == TYPE_Q4_1 || type == TYPE_Q5_0 || type == TYPE_Q5_1) {
        auto go = [&](auto t_c) {
            constexpr int T = decltype(t_c)::value;
            if (x_dtype == KQ_X_F16)
                launch_kq_m<T, KQ_X_F16>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
            else
                launch_kq_m<T, KQ_X_F32>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
        };
        if (type == TYPE_Q4_0) go(std::integral_constant<int, TYPE_Q4_0>{});
        else if (type == TYPE_Q4_1) go(std::integral_constant<int, TYPE_Q4_1>{});
        else if (type == TYPE_Q5_0) go(std::integral_constant<int, TYPE_Q5_0>{});
        else go(std::integral_constant<int, TYPE_Q5_1>{});
    } else if (type == TYPE_Q6_K) {
        if (x_dtype == KQ_X_F16)
            launch_kq_m<TYPE_Q6_K, KQ_X_F16>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
        else
            launch_kq_m<TYPE_Q6_K, KQ_X_F32>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
    } else {
        if (x_dtype == KQ_X_F16)
            launch_kq_m<TYPE_Q8_0, KQ_X_F16>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
        else
            launch_kq_m<TYPE_Q8_0, KQ_X_F32>(wb, wby, xb, xby, Y, m, n, k, rbu, st);
    }
    return check_launch("vb_gemm");
}

// Expert-grouped products for the MoE FFN (Q6_K, Q8_0, Q5_K, Q4_0, Q4_1,
// Q5_0, Q5_1; Q4_K where the caller sends it here); the caller
// (moe.hip) has validated the shapes (K % 128 == 0, 32-bit offsets) and the
// per-expert pointers.  gate_up: hout = fp16 silu(W0 x) * (W1 x) over
// rows slot / topk of X (N = i, K = h); else fout = W0 x over rows slot of
// X (N = h, K = i).
int moe_kq(int32_t type, bool gate_up, const void* const* w0, const void* const* w1, int n_exp, const void* X,
           int64_t xbytes, int topk, const int32_t* eoff, const int32_t* elist, int nslots, int64_t N, int64_t K,
           _Float16* hout, float* fout, const float* rw, float* yacc, hipStream_t st) {
    if (n_exp > MOE_KQ_MAX_EXPERTS || K % KQ_STEP != 0) return E_UNSUPPORTED;
    KqExperts a{}, b{};
    for (int e = 0; e < n_exp; e++) {
        a.p[e] = static_cast<const uint8_t*>(w0[e]);
        b.p[e] = gate_up ? static_cast<const uint8_t*>(w1[e]) : a.p[e];
    }
    const int64_t rb = row_bytes(type, K);
    const uint32_t wbytes = static_cast<uint32_t>((N * rb + 3) & ~int64_t(3));
    const uint8_t* xb = static_cast<const uint8_t*>(X);
    const int n = static_cast<int>(N), k = static_cast<int>(K);
    const uint32_t xby = static_cast<uint32_t>(xbytes), rbu = static_cast<uint32_t>(rb);
    auto go = [&](auto kernel, int ncg, int nmat) {
        const dim3 grid(static_cast<uint32_t>((N + 16 * ncg - 1) / (16 * ncg)), static_cast<uint32_t>(n_exp));
        const size_t lds = static_cast<size_t>(KQ_WAVES) * nmat * ncg * 64 * sizeof(float4_t);
        kernel<<<grid, dim3(64 * KQ_WAVES), lds, st>>>(a, b, wbytes, xb, xby, gate_up ? topk : 1, eoff, elist, nslots,
                                                       n, k,
                                                       rbu, hout, fout, rw, topk, yacc);
    };
    // gate/up: two matrices, 32-slot tiles; down: one matrix, ring of three
    auto run = [&](auto t_c) {
        constexpr int T = decltype(t_c)::value;
        if (gate_up) go(moe_kq_kernel<T, 2, 2, 2>, 2, 2);
        else go(moe_kq_kernel<T, 1, 1, 3>, 1, 1);
    };
    switch (type) {
        case TYPE_Q6_K: run(std::integral_constant<int, TYPE_Q6_K>{}); break;
        case TYPE_Q8_0: run(std::integral_constant<int, TYPE_Q8_0>{}); break;
        case TYPE_Q5_K: run(std::integral_constant<int, TYPE_Q5_K>{}); break;
        case TYPE_Q4_0: run(std::integral_constant<int, TYPE_Q4_0>{}); break;
        case TYPE_Q4_1: run(std::integral_constant<int, TYPE_Q4_1>{}); break;
        case TYPE_Q5_0: run(std::integral_constant<int, TYPE_Q5_0>{}); break;
        case TYPE_Q5_1: run(std::integral_constant<int, TYPE_Q5_1>{}); break;
        default: run(std::integral_constant<int, TYPE_Q4_K>{}); break;
    }
    return check_launch("vb_moe_grouped_ffn");
}

}  // namespace vb
