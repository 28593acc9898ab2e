// Dequant-fused Q4_K GEMM for large M with the activation fragments loaded
// straight into registers (fp16 X): Y[M, N] = X[M, K] . W[N, K]^T, W in the
// GGUF Q4_K layout, Y fp32 row-major.
//
// Replaces, like gemm.hip, the reference's per-token loop of gemv_dequant
// (cpp/src/fast_model.cpp:644-669, :905-960) for prefill-sized batches.
//
// Why this shape.  A v_mfma_f32_16x16x32_f16 wave tile of m_w x n_w needs
// (m_w + n_w) x 64 bytes of operands per 32-element k-step.  With the 256 x
// 112 workgroup tile of 4 MFMA waves (64 x 112 each) and both operands
// staged through LDS (gemm_split.hip), a CU moves about 150 bytes of LDS
// traffic per clock at full MFMA rate (the X tile written and read, the B
// tile written and read four times), which is what its LDS delivers.  Here
// the MFMA waves load their own 64 X rows straight into A fragments (rows
// are disjoint between waves: nothing is loaded twice and nothing goes
// through LDS), and only the dequantized B tile, which all four share, goes
// through LDS: about 78 bytes per clock at full MFMA rate.
//
// X in fragment order.  An A fragment holds 16 rows x 8 halves per lane
// group; loaded from row-major X every load instruction touches 16 rows (16
// separate 64-byte pieces, no two adjacent lanes contiguous), and on MI355X
// such loads kept the texture addresser busy about 60 cycles each: the X
// stream, not the MFMAs, bounded the kernel (93 us at M = 512, 14336 x
// 4096; 66 us with the same loads made contiguous).  So a pack pass first
// writes X into the workspace in the order the fragments are read: per
// 256-row tile and 64-element step, [ks][wave][a][lane] x 16 bytes, so each
// A-fragment load is one contiguous 1 KB.  The pack pass reads 2 M K bytes
// and writes as many (4 MB at M = 512, K = 4096).
//
// Roles (8 waves, two per SIMD, so the hardware interleaves one wave's
// MFMAs with the other's VALU work):
//  * consumers, waves 0-3: X rows 64 w .. 64 w + 63 of the tile and all 16 NF
//    columns (4 x NF accumulator tiles).  Per 64-element k-step: the step's B
//    fragments from LDS, 8 A-fragment loads two steps ahead (two register
//    slots: the loads of step s + 2 go out as soon as the MFMAs of step s
//    have read slot s % 2), 8 NF MFMAs.  Nothing but MFMAs and their
//    operands: VALU work in the same scheduling region as the MFMAs made
//    the register allocator rotate the accumulators through copies.
//  * producers, waves 4-7: stage the raw Q4_K bytes of the tile's 16 NF rows
//    one super-block at a time into LDS with row-contiguous 16-byte loads
//    (9 lanes per 144-byte block), loaded two super-blocks ahead; and
//    dequantize super-block sb + 1 from there while the consumers multiply
//    super-block sb: its 4 NF (chunk, fragment) items are dealt round robin
//    (item i = p + 4 q: chunk i / NF, fragment i % NF), two per step.
// LDS: the B ring, two super-blocks x 4 steps x {ks = 0, 1} x NF fragments x
// 64 lanes x 16 bytes, in the lane order the MFMA reads (every access one
// contiguous 1 KB per wave instruction), and two raw super-blocks of the
// tile's rows.  One barrier per super-block (all 8 waves) separates the
// writes of super-block sb + 1 into the B ring from its reads, the last
// reads of super-block sb - 1 from the writes of sb + 1 into the same half,
// and the raw writes from their reads in the same way.
//
// A k-step is 64 elements = chunk c of a super-block (Q4_K sub-blocks 2c,
// 2c + 1); lane (j, g) of 16-row block a holds X[64 w + 16 a + j, 64 s + 32
// ks + 8 g .. + 8) (natural k order, as q4k_bfrags_cvt gives the weights).
#include "mfma_q4k.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int XR_CW = 4;              // consumer waves
constexpr int XR_TM = 64 * XR_CW;     // X rows per workgroup
constexpr int XR_THREADS = 2 * 64 * XR_CW;
constexpr int XR_STEP_BYTES = XR_TM * 128;  // packed X per 64-element step and tile (32 KB)

// M-tile t covers X rows [t0, t0 + XR_TM) with t0 = min(XR_TM t, M - XR_TM)
// (M >= XR_TM): a last, partial tile is moved back to end at row M.
__device__ __forceinline__ int xr_tile_row0(int t, int M) {
    const int r = t * XR_TM;
    return r < M - XR_TM ? r : M - XR_TM;
}

// Pack X (M x K fp16, row-major) into fragment order.  Entry [ks][w][a]
// [lane] of step s of M-tile t (16 bytes) is X[t0 + 64 w + 16 a + lane % 16,
// 64 s + 32 ks + 8 (lane / 16) .. + 8).  Workgroup (kb, blk, t) moves the
// 16 x 256 block of rows t0 + 16 blk .. + 16 and elements 256 kb .. + 256:
// row-contiguous 16-byte loads (32 lanes per 512-byte row piece), a
// transpose through LDS (rows padded by 16 bytes: the 16 rows a fragment
// read gathers fall in distinct banks), and 1 KB contiguous stores (one
// fragment per 64 threads).
__global__ void __launch_bounds__(256) xr_pack_kernel(const uint8_t* __restrict__ X, uint4* __restrict__ Xf,
                                                      int M, int K) {
    __shared__ uint4 tl[16 * 33];
    const int kb = static_cast<int>(blockIdx.x), blk = static_cast<int>(blockIdx.y);
    const int t = static_cast<int>(blockIdx.z), tid = static_cast<int>(threadIdx.x);
    const int nsteps = K / 64;
    const int r0 = xr_tile_row0(t, M) + 16 * blk;
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int idx = q * 256 + tid, row = idx >> 5, piece = idx & 31;
        tl[row * 33 + piece] =
            *reinterpret_cast<const uint4*>(X + (static_cast<int64_t>(r0 + row) * K + 256 * kb + 8 * piece) * 2);
    }
    __syncthreads();
    uint4* dst = Xf + static_cast<int64_t>(t) * nsteps * (XR_STEP_BYTES / 16);
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int idx = q * 256 + tid, c = idx >> 6, lane = idx & 63;
        const int s = 4 * kb + (c >> 1), ks = c & 1;
        dst[((s * 2 + ks) * 16 + blk) * 64 + lane] = tl[(lane & 15) * 33 + 8 * (c >> 1) + 4 * ks + (lane >> 4)];
    }
}

// ---- the weight types of the producers.  A super-block (256 elements of a
// row) is staged as a window of kPieces 16-byte pieces, kStride pieces
// apart in LDS (Q6_K padded by one: rows 224 bytes apart put the 16 rows of
// a decode read on 4 banks, 240 bytes on 8).  The window starts on the
// super-block for Q4_K (144 = 9 x 16 bytes), Q5_K (176 = 11 x 16) and Q8_0
// (eight 34-byte blocks, 272 = 17 x 16), whose rows are multiples of 16
// bytes long; a Q6_K
// super-block (210 bytes) starts on any even byte, so its window starts at
// the 16-byte boundary below and spans the 14 pieces that cover it.
// kOneRaw: one raw buffer instead of two (Q6_K / Q8_0: the B ring and two
// raw buffers of 112 rows would pass the 160 KB of LDS), which costs a
// second barrier per super-block.
template <int TYPE> struct XrRaw;
template <> struct XrRaw<TYPE_Q4_K> {
    static constexpr int kPieces = 9, kStride = 9;
    static constexpr uint32_t kBytes = 144;
    static constexpr bool kOneRaw = false;
};
template <> struct XrRaw<TYPE_Q5_K> {
    static constexpr int kPieces = 11, kStride = 11;
    static constexpr uint32_t kBytes = 176;
    static constexpr bool kOneRaw = false;
};
// Q4_0 / Q4_1 / Q5_0 / Q5_1: eight 32-element blocks of 18-24 bytes
template <int TYPE> struct XrRawB32 {
    static constexpr int kPieces = static_cast<int>(B32<TYPE>::kBytes) / 2, kStride = kPieces;
    static constexpr uint32_t kBytes = 8 * B32<TYPE>::kBytes;
    static constexpr bool kOneRaw = false;
};
template <> struct XrRaw<TYPE_Q4_0> : XrRawB32<TYPE_Q4_0> {};
template <> struct XrRaw<TYPE_Q4_1> : XrRawB32<TYPE_Q4_1> {};
template <> struct XrRaw<TYPE_Q5_0> : XrRawB32<TYPE_Q5_0> {};
template <> struct XrRaw<TYPE_Q5_1> : XrRawB32<TYPE_Q5_1> {};
template <> struct XrRaw<TYPE_Q6_K> {
    static constexpr int kPieces = 14, kStride = 15;
    static constexpr uint32_t kBytes = 210;
    static constexpr bool kOneRaw = true;
};
template <> struct XrRaw<TYPE_Q8_0> {
    static constexpr int kPieces = 17, kStride = 17;
    static constexpr uint32_t kBytes = 272;
    static constexpr bool kOneRaw = true;
};

// Decode of one producer item from a staged window: chunk c (elements 64 c
// .. 64 c + 63 of the super-block) of one row, lane group g; lo = elements
// 8 g .. + 8 of the chunk, hi = 32 + 8 g .. + 8 (natural k order, the order
// of the packed X).  rw: the window's first dword at or below the data, s =
// the data's byte offset within it (0 or 2).  Each weight is rounded to fp16
// once, with the arithmetic of the tiled kernel's decoders (gemm.hip), so
// both kernels multiply the same fp16 weights.
//
// Q6_K (ql[128] @0, qh[64] @128, int8 scales[16] @192, fp16 d @208): chunk
// c is half h = c / 2, nibble p = c % 2; lo takes ql[64 h + 8 g ..], qh bits
// 4 p, 4 p + 1 and scale 8 h + 4 p + g / 2; hi ql[64 h + 32 + 8 g ..], qh
// bits 4 p + 2, 4 p + 3 and that scale + 2.
__device__ __forceinline__ void xr_q6k_item(const uint32_t* rw, uint32_t s, int c, int g, const KqConsts& kc,
                                            Frag& lo, Frag& hi) {
    const int h = c >> 1, p = c & 1;
    const uint32_t sb8 = 8u * s;
    auto r8 = [&](int dw, uint32_t& x, uint32_t& y) {
        const uint32_t a = rw[dw], b = rw[dw + 1], e = rw[dw + 2];
        x = __builtin_amdgcn_alignbyte(b, a, s);
        y = __builtin_amdgcn_alignbyte(e, b, s);
    };
    uint32_t l0[2], l1[2], qh[2];
    r8(16 * h + 2 * g, l0[0], l0[1]);
    r8(16 * h + 8 + 2 * g, l1[0], l1[1]);
    r8(32 + 8 * h + 2 * g, qh[0], qh[1]);
    const uint32_t sc = __builtin_amdgcn_alignbyte(rw[48 + 2 * h + p + 1], rw[48 + 2 * h + p], s);
    const float d = f16lo(rw[52] >> sb8);
    const uint32_t sb = 8u * static_cast<uint32_t>(g >> 1);
    const _Float16 v0 = static_cast<_Float16>(d * static_cast<float>(static_cast<int8_t>(sc >> sb)));
    const _Float16 v1 = static_cast<_Float16>(d * static_cast<float>(static_cast<int8_t>(sc >> (sb + 16u))));
    q6k_frags(l0, l1, qh, static_cast<uint32_t>(p), half2_t{v0, v0}, half2_t{v1, v1}, kc, lo, hi);
}

// Q8_0 (blocks of 32: fp16 d @0, int8 qs[32] @2; the window is aligned):
// chunk c is blocks 2 c (lo: codes 8 g .. + 8) and 2 c + 1 (hi).
__device__ __forceinline__ void xr_q8_item(const uint32_t* rw, int c, int g, const KqConsts& kc, Frag& lo,
                                           Frag& hi) {
    const int b0 = 17 * c;  // block 2 c at byte 68 c, block 2 c + 1 at 68 c + 34
    const uint32_t a0 = rw[b0 + 2 * g], a1 = rw[b0 + 2 * g + 1], a2 = rw[b0 + 2 * g + 2];
    const uint32_t qs[4] = {__builtin_amdgcn_alignbyte(a1, a0, 2u), __builtin_amdgcn_alignbyte(a2, a1, 2u),
                            rw[b0 + 9 + 2 * g], rw[b0 + 10 + 2 * g]};
    const uint32_t d0 = rw[b0] & 0xFFFFu, d1 = rw[b0 + 8] >> 16;
    const half2_t dd[2] = {bits2h(d0 | (d0 << 16)), bits2h(d1 | (d1 << 16))};
    const half2_t k1152 = half2_t{static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        Frag& f = ks ? hi : lo;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // bytes (b0, b1) into the two halves; (b ^ 0x80) | 0x6400 is the
            // half 1024 + q + 128 (exact)
            const uint32_t src = __builtin_amdgcn_perm(0u, qs[2 * ks + (i >> 1)], (i & 1) ? 0x0C030C02u : 0x0C010C00u);
            f.u[i] = h2bits((bits2h(src ^ kc.x80) - k1152) * dd[ks]);
        }
    }
}

// 32-element block types (B32): chunk c is blocks 2 c (lo) and 2 c + 1 (hi),
// codes [8 g, +8) of each (b32_frag); 18- and 22-byte blocks start on even
// bytes, so each field is read as dwords realigned by its offset.
template <int TYPE>
__device__ __forceinline__ void xr_b32_item(const uint8_t* rw, int c, int g, const KqConsts& kc, Frag& lo,
                                            Frag& hi) {
    using B = B32<TYPE>;
    const uint32_t* r32 = reinterpret_cast<const uint32_t*>(rw);
    auto rd4 = [&](uint32_t o) -> uint32_t {  // bytes [o, o + 4), o even
        if constexpr (B::kBytes % 4 == 0 && B::kQs % 4 == 0 && B::kQh % 4 == 0) {
            return r32[o >> 2];
        } else {
            const uint32_t i = o >> 2;
            return (o & 3u) ? __builtin_amdgcn_alignbyte(r32[i + 1], r32[i], o & 3u) : r32[i];
        }
    };
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t bo = (2u * static_cast<uint32_t>(c) + h) * B::kBytes;
        half2_t d, nb;
        b32_scales<TYPE>(rd4(bo), d, nb);
        const uint32_t qo = bo + B::kQs + 8u * static_cast<uint32_t>(g & 1);
        const uint32_t qhb = B::kHigh ? (rd4(bo + B::kQh) >> (8 * g)) & 0xFFu : 0u;
        b32_frag<TYPE>(rd4(qo), rd4(qo + 4u), static_cast<uint32_t>(g >> 1), qhb, d, nb, kc, h ? hi : lo);
    }
}

// K split (blockIdx.z = kz of gridDim.z): the workgroup takes super-blocks
// [kz nsb / KS, (kz + 1) nsb / KS) and writes its sums to Y + kz M N (the
// caller's partial buffers when KS > 1; xr_ksum_kernel adds them).
template <int TYPE, int NF>
__global__ void __launch_bounds__(XR_THREADS) gemm_xr_kernel(const uint8_t* __restrict__ w, uint32_t wbytes,
                                                             const uint8_t* __restrict__ Xf, float* __restrict__ Y,
                                                             int M, int N, int K, uint32_t rb) {
    using R = XrRaw<TYPE>;
    constexpr bool ONE = R::kOneRaw;
    constexpr int HS = NF * 64;  // uint4 per (step, ks) half of the B ring
    constexpr int SS = 2 * HS;   // per step
    constexpr int SB = 4 * SS;   // per super-block
    constexpr int RAW = R::kPieces * 16 * NF;     // pieces of one raw super-block (16 NF rows)
    constexpr int RAWS = R::kStride * 16 * NF;    // uint4 of one raw buffer in LDS
    constexpr int RPT = (RAW + 255) / 256;        // raw pieces per producer thread
    __shared__ uint4 bt[2 * SB];
    // one spare piece: a realigned 32-element-block read may touch the dword
    // past a window's last used byte
    __shared__ uint4 raw[(ONE ? 1 : 2) * RAWS + 1];

    const int lane = static_cast<int>(threadIdx.x) & 63, j = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    // workgroups go to the 8 XCDs round robin (linear id % 8): with two
    // M-tiles each XCD takes one of them
    const int nt = static_cast<int>(gridDim.x), mt = static_cast<int>(gridDim.y);
    int tile_n = static_cast<int>(blockIdx.x), tile_m = static_cast<int>(blockIdx.y);
    if (mt == 2 && nt % 4 == 0) {
        const int lin = tile_n + nt * tile_m, xcd = lin & 7, r = lin >> 3;
        tile_m = xcd >> 2;
        tile_n = (xcd & 3) * (nt >> 2) + r;
    }
    // rows of a moved-back last tile that the tile before also covers are
    // computed twice, bit-identically (same fragments, same MFMA order), and
    // written twice with the same values
    const int mt0 = xr_tile_row0(tile_m, M);
    const int n0 = tile_n * 16 * NF;
    const int nsteps = 4 * (K >> 8);  // packed X steps of the whole row
    const int kz = static_cast<int>(blockIdx.z), ks = static_cast<int>(gridDim.z);
    const int sb0 = (kz * (K >> 8)) / ks;
    const int nsb = ((kz + 1) * (K >> 8)) / ks - sb0;  // this workgroup's super-blocks sb0 .. sb0 + nsb - 1
    Y += static_cast<int64_t>(kz) * M * N;

    if (wave < XR_CW) {
        // ---------------- consumer ----------------
        const __amdgpu_buffer_rsrc_t xfs =
            make_rsrc(Xf + static_cast<int64_t>(tile_m) * nsteps * XR_STEP_BYTES,
                      static_cast<uint32_t>(nsteps) * XR_STEP_BYTES);
        const uint32_t xv = 16u * static_cast<uint32_t>(lane);
        Frag areg[2][2][4];  // [slot][ks][a]
        const int s_last = 4 * (sb0 + nsb) - 1;
        auto load_a = [&](int s, int slot, int ks) {
            s = 4 * sb0 + s;  // local step -> step of the row
            s = s < s_last ? s : s_last;
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const uint32_t so = static_cast<uint32_t>(((s * 2 + ks) * 16 + wave * 4 + a) * 1024);
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xfs, static_cast<int>(xv), static_cast<int>(so), 0);
                areg[slot][ks][a].u[0] = v.x;
                areg[slot][ks][a].u[1] = v.y;
                areg[slot][ks][a].u[2] = v.z;
                areg[slot][ks][a].u[3] = v.w;
            }
        };
        auto read_b = [&](int buf, int t, int ks, Frag* b) {
            const uint4* src = bt + buf * SB + t * SS + ks * HS + lane;
#pragma unroll
            for (int f = 0; f < NF; f++) {
                const uint4 v = src[f * 64];
                b[f].u[0] = v.x; b[f].u[1] = v.y; b[f].u[2] = v.z; b[f].u[3] = v.w;
            }
        };
        float4_t acc[4][NF];
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int f = 0; f < NF; f++) acc[a][f] = float4_t{0.f, 0.f, 0.f, 0.f};
        auto mfmas = [&](const Frag* af, const Frag* b) {
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int f = 0; f < NF; f++) acc[a][f] = mfma16x16x32(af[a], b[f], acc[a][f]);
        };

        load_a(0, 0, 0);
        load_a(0, 0, 1);
        load_a(1, 1, 0);
        load_a(1, 1, 1);
        __syncthreads();  // raw super-block 0 (and 1) staged
        __syncthreads();  // ring half 0 (super-block 0) written
        Frag b0[NF], b1[NF];
        read_b(0, 0, 0, b0);
        for (int sb = 0; sb < nsb; sb++) {
            const int cur = sb & 1, nxt = cur ^ 1;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int s = 4 * sb + t;
                const int slot = t & 1;
                __builtin_amdgcn_sched_barrier(0);
                read_b(cur, t, 1, b1);
                __builtin_amdgcn_sched_barrier(0);
                mfmas(areg[slot][0], b0);
                __builtin_amdgcn_sched_barrier(0);
                load_a(s + 2, slot, 0);
                // one raw buffer: the producers' mid-super-block barrier
                // (raw bytes of super-block sb + 1 staged)
                if (t == 3 || (ONE && t == 0)) __syncthreads();
                read_b(t == 3 ? nxt : cur, (t + 1) & 3, 0, b0);
                __builtin_amdgcn_sched_barrier(0);
                mfmas(areg[slot][1], b1);
                __builtin_amdgcn_sched_barrier(0);
                load_a(s + 2, slot, 1);
            }
        }
        __builtin_amdgcn_sched_barrier(0);

#pragma unroll
        for (int a = 0; a < 4; a++) {
#pragma unroll
            for (int f = 0; f < NF; f++) {
                const int col = n0 + 16 * f + j;
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = mt0 + 64 * wave + 16 * a + 4 * g + r;
                    Y[static_cast<int64_t>(t) * N + col] = acc[a][f][r];
                }
            }
        }
    } else {
        // ---------------- producer ----------------
        const int pw = wave - XR_CW;
        const int pt = static_cast<int>(threadIdx.x) - 64 * XR_CW;
        const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w, wbytes);
        // raw piece p = pt + 256 i of a super-block: 16-byte piece p % kPieces
        // of tile row p / kPieces (rows past N repeat row N - 1, never
        // stored; pieces past the tile repeat the last one and are not
        // written)
        uint32_t rowb[RPT], pc16[RPT];
        int lidx[RPT];
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            int p = pt + 256 * i;
            p = p < RAW ? p : RAW - 1;
            const int row = p / R::kPieces, piece = p - R::kPieces * row;
            int n = n0 + row;
            n = n < N ? n : N - 1;
            rowb[i] = static_cast<uint32_t>(n) * rb;
            pc16[i] = 16u * static_cast<uint32_t>(piece);
            lidx[i] = row * R::kStride + piece;
        }
        u32x4 rr[RPT];
        auto load_raw = [&](int sb) {
            sb = sb0 + (sb < nsb ? sb : nsb - 1);  // local -> super-block of the row
#pragma unroll
            for (int i = 0; i < RPT; i++) {
                if constexpr (TYPE == TYPE_Q6_K) {
                    const uint32_t off = ((rowb[i] + static_cast<uint32_t>(sb) * R::kBytes) & ~15u) + pc16[i];
                    rr[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, static_cast<int>(off), 0, 0);
                } else {
                    rr[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, static_cast<int>(rowb[i] + pc16[i]),
                                                                  static_cast<int>(static_cast<uint32_t>(sb) * R::kBytes),
                                                                  0);
                }
            }
        };
        auto store_raw = [&](int buf) {
#pragma unroll
            for (int i = 0; i < RPT; i++) {
                const int p = pt + 256 * i;
                if (i + 1 < RPT || p < RAW) raw[buf * RAWS + lidx[i]] = make_uint4(rr[i].x, rr[i].y, rr[i].z, rr[i].w);
            }
        };
        // the wave's dequant items q = 0 .. NF - 1: chunk ic[q], fragment ifr[q]
        int ic[NF], ifr[NF];
#pragma unroll
        for (int q = 0; q < NF; q++) {
            const int i = pw + 4 * q;
            ic[q] = i / NF;
            ifr[q] = i - NF * ic[q];
        }
        const KqConsts kc = kq_consts();
        // super-block sb (local) of item q from raw buffer rbuf into ring half buf
        auto dequant_item = [&](int q, int sb, int rbuf, int buf) {
            const uint8_t* rw = reinterpret_cast<const uint8_t*>(raw + rbuf * RAWS) + (16 * ifr[q] + j) * 16 * R::kStride;
            Frag lo, hi;
            if constexpr (TYPE == TYPE_Q4_K) {
                (void)sb;
                const uint4 h = *reinterpret_cast<const uint4*>(rw);
                const uint2 qs = *reinterpret_cast<const uint2*>(rw + 16 + 32 * ic[q] + 8 * g);
                half2_t ds[2], nm[2];
                q4k_chunk_scales_sel(h, ic[q], ds, nm);
                q4k_bfrags_cvt(qs.x, qs.y, ds, nm, lo, hi);
            } else if constexpr (TYPE == TYPE_Q5_K) {
                // d, dmin, scales[12] @0 (the Q4_K header), qh[32] @16, qs[128] @48
                (void)sb;
                const uint4 h = *reinterpret_cast<const uint4*>(rw);
                const uint2 qs = *reinterpret_cast<const uint2*>(rw + 48 + 32 * ic[q] + 8 * g);
                const uint2 qh = *reinterpret_cast<const uint2*>(rw + 16 + 8 * g);
                half2_t ds[2], nm[2];
                q4k_chunk_scales_sel(h, ic[q], ds, nm);
                q5k_frags(qs.x, qs.y, qh.x, qh.y, static_cast<uint32_t>(ic[q]), ds, nm, kc, lo, hi);
            } else if constexpr (TYPE == TYPE_Q6_K) {
                // the window starts (row start + 210 sb) % 16 bytes before the data
                int n = n0 + 16 * ifr[q] + j;
                n = n < N ? n : N - 1;
                const uint32_t sh =
                    (static_cast<uint32_t>(n) * rb + static_cast<uint32_t>(sb0 + (sb < nsb ? sb : nsb - 1)) * 210u) & 15u;
                xr_q6k_item(reinterpret_cast<const uint32_t*>(rw + (sh & ~3u)), sh & 3u, ic[q], g, kc, lo, hi);
            } else if constexpr (TYPE == TYPE_Q8_0) {
                (void)sb;
                xr_q8_item(reinterpret_cast<const uint32_t*>(rw), ic[q], g, kc, lo, hi);
            } else {
                (void)sb;
                xr_b32_item<TYPE>(rw, ic[q], g, kc, lo, hi);
            }
            uint4* dst = bt + buf * SB + ic[q] * SS + ifr[q] * 64 + lane;
            dst[0] = make_uint4(lo.u[0], lo.u[1], lo.u[2], lo.u[3]);
            dst[HS] = make_uint4(hi.u[0], hi.u[1], hi.u[2], hi.u[3]);
        };

        if constexpr (ONE) {
            load_raw(0);
            store_raw(0);
            load_raw(1);
            __syncthreads();  // raw super-block 0 staged
#pragma unroll
            for (int q = 0; q < NF; q++) dequant_item(q, 0, 0, 0);
            __syncthreads();  // ring half 0 written, raw buffer free
            for (int sb = 0; sb < nsb; sb++) {
                // stage super-block sb + 1 (loaded during sb - 1) and load sb +
                // 2; the consumers' barrier at step 0 of sb publishes it; then
                // dequantize it into ring half (sb + 1) % 2, which the
                // consumers last read during sb - 1, before their barrier at
                // step 3.  Past the last super-block: clamped loads, a half
                // nobody reads.
                const int nxt = (sb & 1) ^ 1;
                store_raw(0);
                load_raw(sb + 2);
                __syncthreads();
#pragma unroll
                for (int q = 0; q < NF; q++) dequant_item(q, sb + 1, 0, nxt);
                __syncthreads();
            }
        } else {
            load_raw(0);
            store_raw(0);
            load_raw(1);
            store_raw(1);
            __syncthreads();  // raw super-blocks 0 and 1 staged
#pragma unroll
            for (int q = 0; q < NF; q++) dequant_item(q, 0, 0, 0);
            load_raw(2);
            __syncthreads();  // ring half 0 written
            for (int sb = 0; sb < nsb; sb++) {
                // dequantize super-block sb + 1 (raw half (sb + 1) % 2) into ring
                // half (sb + 1) % 2, two items per step; then stage the raw bytes
                // of super-block sb + 2 (loaded during sb - 1) into raw half sb % 2,
                // free since super-block sb was dequantized during sb - 1, and
                // load those of sb + 3.  Past the last super-block: clamped
                // loads, halves nobody reads.
                const int nxt = (sb & 1) ^ 1;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int k2 = 0; k2 < 2; k2++)
                        if (2 * t + k2 < NF) dequant_item(2 * t + k2, sb + 1, nxt, nxt);
                }
                __builtin_amdgcn_sched_barrier(0);
                store_raw(sb & 1);
                load_raw(sb + 3);
                __syncthreads();
            }
        }
    }
}

// Y = sum of the KS partial products in the order kz = 0, 1, ... (fixed,
// deterministic); four outputs per thread.
__global__ void __launch_bounds__(256) xr_ksum_kernel(const float* __restrict__ P, float* __restrict__ Y,
                                                      int64_t total, int ks) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i + 4 <= total) {
        float4 s = *reinterpret_cast<const float4*>(P + i);
        for (int z = 1; z < ks; z++) {
            const float4 v = *reinterpret_cast<const float4*>(P + static_cast<int64_t>(z) * total + i);
            s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
        }
        *reinterpret_cast<float4*>(Y + i) = s;
    } else {
        for (int64_t e = i; e < total; e++) {
            float s = P[e];
            for (int z = 1; z < ks; z++) s += P[static_cast<int64_t>(z) * total + e];
            Y[e] = s;
        }
    }
}

constexpr int XR_NF = 7;

}  // namespace

// K splits: as many as fit the CUs with one workgroup each (a shape with
// fewer output tiles than CUs, such as the FFN down projection 4096 x 14336
// at M = 512: 37 x 2 tiles, 3 splits), at least 8 super-blocks per split.
int gemm_xr_ksplit(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = (N + 16 * XR_NF - 1) / (16 * XR_NF) * ((M + XR_TM - 1) / XR_TM);
    int64_t ks = num_cus() / (tiles > 0 ? tiles : 1);
    const int64_t kmax = (K / 256) / 8;
    ks = ks < kmax ? ks : kmax;
    return static_cast<int>(ks < 1 ? 1 : (ks > 8 ? 8 : ks));
}

int gemm_ksum(const float* P, float* Y, int64_t total, int ks, hipStream_t st) {
    xr_ksum_kernel<<<dim3(static_cast<uint32_t>((total / 4 + 255) / 256 + 1)), dim3(256), 0, st>>>(P, Y, total, ks);
    return check_launch("vb_gemm");
}

int64_t gemm_xr_workspace(int64_t M, int64_t N, int64_t K) {
    const int64_t xf = (M + XR_TM - 1) / XR_TM * XR_TM * K * 2;
    const int ks = gemm_xr_ksplit(M, N, K);
    return xf + (ks > 1 ? static_cast<int64_t>(ks) * M * N * 4 : 0);
}

bool gemm_xr_type(int32_t type) {
    return type == TYPE_Q4_K || type == TYPE_Q5_K || type == TYPE_Q6_K || type == TYPE_Q8_0 || type == TYPE_Q4_0 ||
           type == TYPE_Q4_1 || type == TYPE_Q5_0 || type == TYPE_Q5_1;
}

// Caller (gemm_dispatch) has validated the type (gemm_xr_type), alignment
// (W, X 16 B), the 32-bit offset bounds (N * row bytes rounded up to whole
// dwords, M * K * 2 < 2^32), K % 256 == 0, M >= 256 and the workspace
// (gemm_xr_workspace bytes, 16-byte aligned): the packed X, then, with K
// splits, one fp32 M x N partial product per split.
int gemm_xr(const void* w, const void* X, float* Y, int64_t M, int64_t N, int64_t K, int32_t type, void* ws,
            hipStream_t st) {
    constexpr int NF = XR_NF;
    const int64_t rb = row_bytes(type, K);
    // whole dwords: a Q6_K window's last dword may hold the tensor's last two bytes
    const uint32_t wbytes = static_cast<uint32_t>((N * rb + 3) & ~int64_t(3));
    const uint32_t mtiles = static_cast<uint32_t>((M + XR_TM - 1) / XR_TM);
    const int ks = gemm_xr_ksplit(M, N, K);
    xr_pack_kernel<<<dim3(static_cast<uint32_t>(K / 256), XR_TM / 16, mtiles), dim3(256), 0, st>>>(
        static_cast<const uint8_t*>(X), static_cast<uint4*>(ws), static_cast<int>(M), static_cast<int>(K));
    float* out = Y;
    if (ks > 1) out = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + mtiles * XR_TM * K * 2);
    const dim3 grid(static_cast<uint32_t>((N + 16 * NF - 1) / (16 * NF)), mtiles, static_cast<uint32_t>(ks));
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const uint8_t* xf = static_cast<const uint8_t*>(ws);
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    const uint32_t r = static_cast<uint32_t>(rb);
    if (type == TYPE_Q4_K)
        gemm_xr_kernel<TYPE_Q4_K, NF><<<grid, dim3(XR_THREADS), 0, st>>>(wb, wbytes, xf, out, m, n, k, r);
    else if (type == TYPE_Q5_K)
        gemm_xr_kernel<TYPE_Q5_K, NF><<<grid, dim3(XR_THREADS), 0, st>>>(wb, wbytes, xf, out, m, n, k, r);
    else if (type == TYPE_Q6_K)
        gemm_xr_kernel<TYPE_Q6_K, NF><<<grid, dim3(XR_THREADS), 0, st>>>(wb, wbytes, xf, out, m, n, k, r);
    else if (type == TYPE_Q4_0)
        gemm_xr_kernel<TYPE_Q4_0, NF><<<grid, dim3(XR_THREADS), 0, st>>>(wb, wbytes, xf, out, m, n, k, r);
    else if (type == TYPE_Q4_1)
        gemm_xr_kernel<TYPE_Q4_1, NF><<<grid, dim3(XR_THREADS), 0, st>>>(wb, wbytes, xf, out, m, n, k, r);
    else if (type == TYPE_Q5_0)
        gemm_xr_kernel<TYPE_Q5_0, NF><<<grid, dim3(XR_THREADS), 0, st>>>(wb, wbytes, xf, out, m, n, k, r);
    else if (type == TYPE_Q5_1)
        gemm_xr_kernel<TYPE_Q5_1, NF><<<grid, dim3(XR_THREADS), 0, st>>>(wb, wbytes, xf, out, m, n, k, r);
    else
        gemm_xr_kernel<TYPE_Q8_0, NF><<<grid, dim3(XR_THREADS), 0, st>>>(wb, wbytes, xf, out, m, n, k, r);
    if (ks > 1) {
        if (const int rc = check_launch("vb_gemm"); rc != OK) return rc;
        return gemm_ksum(out, Y, M * N, ks, st);
    }
    return check_launch("vb_gemm");
}

}  // namespace vb
