// Dequant-fused GEMM on MFMA:  Y[M, N] = X[M, K] . W[N, K]^T  (W Q4_K, Q6_K
// or Q8_0 in the GGUF layout; X fp16 or fp32 row-major; Y fp32 row-major).
//
// The reference runs batched tokens as a per-token loop of gemv_dequant
// (cpp/src/fast_model.cpp:644-669, :905-960), re-streaming every weight once
// per token; cuda::gemm_f32 (cpp/src/cuda_kernels.cu:184-212) needs fp32
// weights.  Here weights are streamed once per M-tile and dequantized to fp16
// in registers, in the B-operand layout of v_mfma_f32_16x16x32_f16
// (mfma_q4k.hpp), accumulating in fp32.
//
// Q4_K: M <= 32 goes to the skinny kernel (gemm_skinny.hip); M > 32
// (chunked prefill) runs the tiled kernel below.  Q6_K / Q8_0 run the
// K-split kernel (gemm_kq.hip) at small M and the tiled kernel above.
#include <cstdlib>

#include "mfma_q4k.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int X_F32 = 0;
constexpr int X_F16 = 1;

// ---- tiled: M > 16 ------------------------------------------------------------
//
// Workgroup tile: TB_M = 64 WM rows of X x BN = 16 * NF weight rows (output
// columns), WM x WN waves; wave (wm, wn) owns X rows [64 wm, +64) x fragment
// columns [wn * NF / WN, +NF / WN): 4 x NF / WN accumulator fragments.  Large
// M runs 256-row tiles (WM = 4, WN = 2: two waves per SIMD); small M narrower
// tiles so the grid still covers the CUs (see tiled_cfg).  k advances one
// Q4_K chunk (64 elements) per step, and
// both operands of a step are staged in LDS (double-buffered):
//  * B: the workgroup dequantizes the BN x 64 weight tile once into fp16 B
//    fragments (natural k order); each of the 4 * BN "units" (8 qs bytes of
//    one row -> the same lane of the step's two fragments) belongs to one
//    thread, consecutive threads owning consecutive LDS lane slots.  Raw
//    weight bytes run PD steps ahead in registers (HBM latency).
//  * A: the 256 x 64 X tile is loaded with row-contiguous 16-byte pieces
//    (8 lanes per 128-byte row: 4 x fewer cache-line requests than loading
//    the fragments directly, and no duplicate loads across wave columns) two
//    steps ahead, converted to fp16 and stored in swizzled 128-byte rows (below);
//    the waves read their A fragments with ds_read_b128.
// One barrier per step.  The grid is ceil(N / BN) x ceil(M / TB_M).
constexpr int XS_ROW = 64;  // halves per LDS row of X (swizzled, no padding)
// weight prefetch distance (steps; K / 64 is a multiple of 4)
constexpr int PD = 4;

// X tile in LDS: 128-byte rows (64 halves) whose eight 16-byte pieces are
// XOR-swizzled by (row / 2) % 8, so the ds_read_b128 of the A fragments (16
// rows x one piece per lane group) and the row-contiguous tile stores meet
// no bank conflicts.  Rows padded to 144 bytes instead showed 3.67e6 bank
// conflict cycles per launch (SQ_LDS_BANK_CONFLICT, M = 512) and ran 2-4 %
// slower; the swizzle reads 0.
__device__ __forceinline__ int xswz(int row) { return (row >> 1) & 7; }

// ---- weight steps of the 2-byte-aligned GGUF types.  A step is 64
// elements; dequant unit (row, ug) yields lane (row % 16, ug) of the step's
// two B fragments: elements 8 ug .. +7 (k-half 0) and 32 + 8 ug .. +7
// (k-half 1), the natural k order.  issue() loads the raw bytes (buffer
// loads, 12-byte reads realigned: rows are 2-byte aligned); decode() rounds
// each weight to fp16 once.  g8 = 8 ug.
template <int TYPE> struct TiledW {
    static constexpr bool kPairOrder = false;
    struct Raw {};
};

// Q6_K in the GGUF layout (super-block of 256: ql[128] @0, qh[64] @128, int8
// scales[16] @192, fp16 d @208; known answers in tests/test_kquants.py:
// 134-175).  In half h, element l + 32 t (l < 32, t < 4) is q - 32 with
// q = (ql[64 h + l + 32 (t & 1)] >> 4 (t >> 1)) & 15 |
// ((qh[32 h + l] >> 2 t) & 3) << 4, scaled by d * scales[8 h + l / 16 + 2 t].
// Step 4 sb + 2 h + p covers t = 2 p + ks of half h, so a lane needs the 8
// ql bytes at 64 h + 8 ug (k-half 0) and 64 h + 32 + 8 ug (k-half 1), nibble
// p, the qh bytes at 128 + 32 h + 8 ug (bits 4 p + 2 ks), the scales
// 8 h + 4 p + ug / 2 (+ 2) and d.
template <>
struct TiledW<TYPE_Q6_K> {
    static constexpr bool kPairOrder = false;
    struct Raw {
        u32x3 l0, l1, qh;
        uint32_t sd;  // lane group ug: the step's scale dwords (ug 0, 1) or d's dword (ug 2, 3)
    };
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, uint32_t g8,
                                                 Raw& r) {
        const uint32_t base = (rowoff + static_cast<uint32_t>(step >> 2) * 210u) & ~3u;
        const uint32_t h = (static_cast<uint32_t>(step) >> 1) & 1u, p = static_cast<uint32_t>(step) & 1u;
        r.l0 = ld96(w, base + 64u * h + g8);
        r.l1 = ld96(w, base + 64u * h + 32u + g8);
        r.qh = ld96(w, base + 128u + 32u * h + g8);
        // the four lane groups of a row share its scales and d: one dword each
        const uint32_t ug = g8 >> 3;
        r.sd = ld32(w, ug < 2 ? base + 192u + 8u * h + 4u * p + 4u * ug : base + 208u);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t rowoff, int step, uint32_t g8,
                                                  const KqConsts& kc, Frag& lo, Frag& hi) {
        const uint32_t sh = (rowoff + static_cast<uint32_t>(step >> 2) * 210u) & 3u;
        uint32_t l0[2], l1[2], qh[2];
        realign(r.l0, sh, l0[0], l0[1]);
        realign(r.l1, sh, l1[0], l1[1]);
        realign(r.qh, sh, qh[0], qh[1]);
        // dwords of lane groups 0-2 (the pair's even / odd 16-lane rows, then
        // the lower / upper halves of the wave)
        const auto p16 = __builtin_amdgcn_permlane16_swap(r.sd, r.sd, false, false);
        const auto e32 = __builtin_amdgcn_permlane32_swap(p16[0], p16[0], false, false);
        const auto o32 = __builtin_amdgcn_permlane32_swap(p16[1], p16[1], false, false);
        const uint32_t sc = __builtin_amdgcn_alignbyte(o32[0], e32[0], sh);
        const float d = f16lo(e32[1] >> (8u * sh));
        const uint32_t sb = 8u * (g8 >> 4);  // byte of scale ug / 2 within the four
        const _Float16 v0 = static_cast<_Float16>(d * static_cast<float>(static_cast<int8_t>(sc >> sb)));
        const _Float16 v1 = static_cast<_Float16>(d * static_cast<float>(static_cast<int8_t>(sc >> (sb + 16u))));
        q6k_frags(l0, l1, qh, static_cast<uint32_t>(step) & 1u, half2_t{v0, v0}, half2_t{v1, v1}, kc, lo, hi);
    }
};

// Q8_0 in the GGUF layout (vibeblade/loader.py:129-133): blocks of 32 =
// fp16 d @0, int8 qs[32] @2.  Step s covers blocks 2 s and 2 s + 1 in the
// pair k order (kPairOrder): lane group ug holds the 16 codes
// [16 (ug & 1), +16) of block 2 s + ug / 2, k-half 0 the first 8 and k-half 1
// the next 8, i.e. step elements 16 ug .. 16 ug + 15 (the activation
// fragments read 8-element pieces 2 ug and 2 ug + 1).  One 20-byte code read
// and one scale read per unit, where the natural order took two of each.
template <>
struct TiledW<TYPE_Q8_0> {
    static constexpr bool kPairOrder = true;
    struct Raw {
        u32x4 q;
        uint32_t q4, d;
    };
    // block 2 s + ug / 2 starts at rowoff + 68 s + 34 (ug / 2); its codes
    // [16 (ug & 1), +16) 2 + 16 (ug & 1) bytes further on
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, uint32_t g8,
                                                 Raw& r) {
        const uint32_t ug = g8 >> 3;
        const uint32_t blk = rowoff + static_cast<uint32_t>(step) * 68u + 34u * (ug >> 1);
        const uint32_t c = (blk + 2u + 16u * (ug & 1u)) & ~3u;
        r.q = buf_ld128(w, c, 0);
        r.q4 = ld32(w, c + 16u);
        r.d = ld32(w, blk & ~3u);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t rowoff, int, uint32_t g8, const KqConsts& kc,
                                                  Frag& lo, Frag& hi) {
        const uint32_t ug = g8 >> 3;
        const uint32_t shb = (rowoff + 34u * (ug >> 1)) & 3u;  // block start within its dword
        const uint32_t shc = (shb + 2u) & 3u;                  // codes start (the odd half: +16, same)
        const uint32_t w[5] = {r.q.x, r.q.y, r.q.z, r.q.w, r.q4};
        uint32_t qs[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], shc);
        const uint32_t d16 = (r.d >> (8u * shb)) & 0xFFFFu;
        const half2_t dd = bits2h(d16 | (d16 << 16));
        const half2_t k1152 = half2_t{static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            Frag& f = ks ? hi : lo;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // bytes (b0, b1) into the two halves; (b ^ 0x80) | 0x6400 is
                // the half 1024 + q + 128 (exact)
                const uint32_t src =
                    __builtin_amdgcn_perm(0u, qs[2 * ks + (i >> 1)], (i & 1) ? 0x0C030C02u : 0x0C010C00u);
                f.u[i] = h2bits((bits2h(src ^ kc.x80) - k1152) * dd);
            }
        }
    }
};

// Q5_K in the GGUF layout (super-block of 256, 176 bytes: fp16 d @0, fp16
// dmin @2, scales[12] @4 in the Q4_K 6-bit packing, qh[32] @16, qs[128] @48).
// Element 64 c + l (l < 64) of a super-block has sub-block 2 c + l / 32 and
// code q5 = ((qs[32 c + l % 32] >> 4 (l / 32)) & 15) | ((qh[l % 32] >> (2 c + l
// / 32)) & 1) << 4, weight d sc q5 - dmin m (the vb_dequant_rows formula).
// Step 4 sb + c: a lane needs the header, qs bytes 32 c + 8 ug .. + 8 (low
// nibbles: k-half 0, high: k-half 1) and qh bytes 8 ug .. + 8 (bits 2 c,
// 2 c + 1), decoded by q5k_frags (1024 + q5 in fp16 halves, exact, then
// (h - 1024) d sc - dmin m with one rounding).
template <>
struct TiledW<TYPE_Q5_K> {
    static constexpr bool kPairOrder = false;
    struct Raw {
        u32x4 hd;
        uint32_t q0, q1, h0, h1;
    };
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, uint32_t g8,
                                                 Raw& r) {
        const uint32_t base = rowoff + static_cast<uint32_t>(step >> 2) * 176u;
        const uint32_t c = static_cast<uint32_t>(step) & 3u;
        r.hd = buf_ld128(w, base, 0);
        r.q0 = ld32(w, base + 48u + 32u * c + g8);
        r.q1 = ld32(w, base + 52u + 32u * c + g8);
        r.h0 = ld32(w, base + 16u + g8);
        r.h1 = ld32(w, base + 20u + g8);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t, int step, uint32_t, const KqConsts& kc,
                                                  Frag& lo, Frag& hi) {
        const int c = step & 3;
        half2_t ds[2], nm[2];
        q4k_chunk_scales(make_uint4(r.hd.x, r.hd.y, r.hd.z, r.hd.w), c, ds, nm);
        q5k_frags(r.q0, r.q1, r.h0, r.h1, static_cast<uint32_t>(c), ds, nm, kc, lo, hi);
    }
};

// Q4_0 / Q4_1 / Q5_0 / Q5_1 (B32 in mfma_q4k.hpp): step s is blocks 2 s
// (k-half 0) and 2 s + 1 (k-half 1); unit ug takes codes [8 ug, +8) of each.
// Rows are multiples of 16 bytes (K % 256 == 0), so block 2 s starts on a
// dword and block 2 s + 1 kBytes later (2 bytes into a dword for the 18- and
// 22-byte blocks); each block is read as the six dwords from its start
// rounded down to 4 (the four units of a row read the same bytes).
template <int TYPE>
struct TiledB32 {
    static constexpr bool kPairOrder = false;
    using B = B32<TYPE>;
    struct Raw {
        u32x3 a[2], b[2];
    };
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, uint32_t,
                                                 Raw& r) {
        const uint32_t o0 = rowoff + 2u * static_cast<uint32_t>(step) * B::kBytes;
        const uint32_t o1 = (o0 + B::kBytes) & ~3u;
        r.a[0] = ld96(w, o0);
        r.a[1] = ld96(w, o0 + 12u);
        r.b[0] = ld96(w, o1);
        r.b[1] = ld96(w, o1 + 12u);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t, int, uint32_t g8, const KqConsts& kc,
                                                  Frag& lo, Frag& hi) {
        const uint32_t wa[6] = {r.a[0].x, r.a[0].y, r.a[0].z, r.a[1].x, r.a[1].y, r.a[1].z};
        const uint32_t wb[6] = {r.b[0].x, r.b[0].y, r.b[0].z, r.b[1].x, r.b[1].y, r.b[1].z};
        const int e = static_cast<int>(g8 >> 3);
        b32_block_frag<TYPE>(wa, 0u, e, kc, lo);
        b32_block_frag<TYPE>(wb, B::kBytes & 3u, e, kc, hi);
    }
};
template <> struct TiledW<TYPE_Q4_0> : TiledB32<TYPE_Q4_0> {};
template <> struct TiledW<TYPE_Q4_1> : TiledB32<TYPE_Q4_1> {};
template <> struct TiledW<TYPE_Q5_0> : TiledB32<TYPE_Q5_0> {};
template <> struct TiledW<TYPE_Q5_1> : TiledB32<TYPE_Q5_1> {};

// fp16 weights, row-major (a GGUF F16 tensor, or any other type decoded to
// fp16 first): lane (row, ug) of a step's fragments is elements 8 ug .. +7
// and 32 + 8 ug .. +7 of the step's 64, 16 bytes each, used as loaded.
template <>
struct TiledW<TYPE_F16> {
    static constexpr bool kPairOrder = false;
    struct Raw {
        u32x4 lo, hi;
    };
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t w, uint32_t rowoff, int step, uint32_t g8,
                                                 Raw& r) {
        const uint32_t base = rowoff + static_cast<uint32_t>(step) * 128u + 2u * g8;
        r.lo = buf_ld128(w, base, 0);
        r.hi = buf_ld128(w, base + 64u, 0);
    }
    __device__ static __forceinline__ void decode(const Raw& r, uint32_t, int, uint32_t, const KqConsts&, Frag& lo,
                                                  Frag& hi) {
        lo.u[0] = r.lo.x; lo.u[1] = r.lo.y; lo.u[2] = r.lo.z; lo.u[3] = r.lo.w;
        hi.u[0] = r.hi.x; hi.u[1] = r.hi.y; hi.u[2] = r.hi.z; hi.u[3] = r.hi.w;
    }
};

// KS = 2 splits K in halves between two groups of WM x WN waves, each with
// its own LDS stage (the tiles below); both run the same number of steps, so
// the one barrier per step serves both.  At the end group 1 hands its
// accumulators to group 0 through LDS (fixed order), which stores Y.
// gridDim.z > 1 splits K between workgroups as well: workgroup z takes steps
// [z nsteps / Z, (z + 1) nsteps / Z) and stores to Y + z M N (a partial
// product; gemm_ksum adds them).
template <int TYPE, int XT, int NF, int WM, int WN, int KS>
__global__ void __launch_bounds__(64 * WM * WN * KS) gemm_tiled(const uint8_t* __restrict__ w, uint32_t wbytes,
                                                                const void* __restrict__ X, float* __restrict__ Y,
                                                                int M, int N, int K, int64_t rb) {
    constexpr int TB_M = 64 * WM;           // X rows per workgroup
    constexpr int NT = 64 * WM * WN;        // threads of one K group
    constexpr int NU = 4 * 16 * NF;         // dequant units per step
    constexpr int UPT = (NU + NT - 1) / NT;  // units per thread
    constexpr int NW = NF / WN;             // B fragments per wave
    constexpr uint32_t XE = XT == X_F16 ? 2u : 4u;  // bytes per X element
    constexpr int XPR = 8;                  // 8-element pieces per X row and step
    constexpr int XPT = TB_M * XPR / NT;    // X pieces per thread and step
    constexpr int XR = XT == X_F16 ? 1 : 2;  // uint4 per piece
    static_assert(NF % WN == 0, "NF must split evenly over the wave columns");
    static_assert(TB_M * XPR % NT == 0, "X pieces must split evenly over the threads");
    // Stage of one K group.  bt: [buffer][k half][fragment][lane]; fragment
    // NF takes the stores of threads without a unit (keeps the loop body
    // branch-free).
    struct Stage {
        uint4 bt[2][2][NF + 1][64];
        _Float16 xs[2][TB_M * XS_ROW];
    };
    static_assert(KS == 1 || sizeof(Stage) >= sizeof(float4_t) * 64 * WM * WN * 4 * (NF / WN),
                  "group 1's stage must hold its accumulators");
    __shared__ __attribute__((aligned(16))) Stage stage[KS];

    const int grp = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / NT);
    const int tid = static_cast<int>(threadIdx.x) - grp * NT, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(tid >> 6));
    auto& bt = stage[grp].bt;
    auto& xs = stage[grp].xs;
    const int wm = wave / WN, wn = wave - wm * WN;
    const int j = lane & 15, g = lane >> 4;
    // Tile of this workgroup.  Workgroups are dealt to the 8 XCDs round
    // robin (linear id % 8).  With Q = (M-tiles) x (K splits) = 2, 4 or 8
    // blocks of X (one per M-tile and K range), each block gets 8 / Q XCDs
    // of its own, so each XCD's L2 holds one block (a bijection when nt is a
    // multiple of 8 / Q).  At 4096 x 14336, M = 512, with four K splits:
    // eight 1.8 MB blocks, one per XCD, instead of all 14.7 MB on every XCD.
    const int nt = static_cast<int>(gridDim.x), mt = static_cast<int>(gridDim.y);
    const int zs = static_cast<int>(gridDim.z);
    int tile_n = static_cast<int>(blockIdx.x), tile_m = static_cast<int>(blockIdx.y);
    int kz = static_cast<int>(blockIdx.z);
    const int Q = mt * zs;
    if ((Q == 2 || Q == 4 || Q == 8) && nt % (8 / Q) == 0) {
        const int G = 8 / Q;  // XCDs per X block
        const int lin = tile_n + nt * (tile_m + mt * kz), xcd = lin & 7, r = lin >> 3;
        const int q = xcd / G;
        tile_m = q % mt;
        kz = q / mt;
        tile_n = (xcd % G) * (nt / G) + r;
    }
    const int mt0 = tile_m * TB_M;
    const int n0 = tile_n * 16 * NF;
    const int nsteps = K / 64;
    // this group's steps: [s_base, s_base + nloc); nloc % PD == 0 (host)
    const int nloc = nsteps / (KS * zs), s_base = (kz * KS + grp) * nloc;
    Y += static_cast<int64_t>(kz) * M * N;

    // ---- weights: dequant unit u = tid + NT i is LDS lane slot u: fragment
    // u / 64, lane l = u % 64 -> weight row un = 16 (u / 64) + l % 16, qs part
    // ug = l / 16.  Each wave stores 1 KB contiguous (bank-conflict free).
    uint32_t urow[UPT];  // byte offset of the unit's weight row in W
    uint32_t uq[UPT];    // byte offset of the unit's 8 qs bytes within a chunk's 32
    int uslot[UPT];      // LDS lane slot
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        int u = tid + NT * i;
        const bool live = u < NU;
        u = live ? u : NU - 1;
        const int l = u & 63, un = 16 * (u >> 6) + (l & 15), ug = l >> 4;
        int n = n0 + un;
        n = n < N ? n : N - 1;
        urow[i] = static_cast<uint32_t>(n) * static_cast<uint32_t>(rb);
        // Q4_K: the unit's qs bytes within a chunk's (after the 16-byte
        // header); other types: 8 ug
        uq[i] = (TYPE == TYPE_Q4_K ? 16u : 0u) + 8u * static_cast<uint32_t>(ug);
        uslot[i] = live ? u : NF * 64 + lane;
    }
    [[maybe_unused]] uint4 whd[PD][UPT];
    [[maybe_unused]] uint2 wqs[PD][UPT];
    [[maybe_unused]] typename TiledW<TYPE>::Raw wraw[PD][UPT];
    [[maybe_unused]] const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w, wbytes);
    [[maybe_unused]] KqConsts kc;
    if constexpr (TYPE != TYPE_Q4_K) kc = kq_consts();
    // the lambdas take the group's local step
    auto load_w = [&](int step, int slot) {
        step += s_base;
        step = step < nsteps ? step : nsteps - 1;
        if constexpr (TYPE == TYPE_Q4_K) {
            const uint32_t sbo = static_cast<uint32_t>(step >> 2) * 144u, co = static_cast<uint32_t>(step & 3) * 32u;
#pragma unroll
            for (int i = 0; i < UPT; i++) {
                whd[slot][i] = *reinterpret_cast<const uint4*>(w + (urow[i] + sbo));
                wqs[slot][i] = *reinterpret_cast<const uint2*>(w + (urow[i] + sbo + uq[i] + co));
            }
        } else {
#pragma unroll
            for (int i = 0; i < UPT; i++) TiledW<TYPE>::issue(wrs, urow[i], step, uq[i], wraw[slot][i]);
        }
    };
    auto dequant_store = [&](int step, int slot, int buf) {
        step += s_base;
        uint4* dst = &bt[buf][0][0][0];
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            Frag lo, hi;
            if constexpr (TYPE == TYPE_Q4_K) {
                half2_t ds[2], nm[2];
                q4k_chunk_scales(whd[slot][i], step & 3, ds, nm);
                q4k_bfrags_nat(wqs[slot][i].x, wqs[slot][i].y, ds, nm, lo, hi);
            } else {
                // the slot holds the clamped step (past the end: never read)
                TiledW<TYPE>::decode(wraw[slot][i], urow[i], step < nsteps ? step : nsteps - 1, uq[i], kc, lo, hi);
            }
            dst[uslot[i]] = make_uint4(lo.u[0], lo.u[1], lo.u[2], lo.u[3]);
            dst[(NF + 1) * 64 + uslot[i]] = make_uint4(hi.u[0], hi.u[1], hi.u[2], hi.u[3]);
        }
    };

    // ---- X: piece q = tid + NT i -> row q / 8, elements 8 (q % 8) .. +8 of the step
    const uint8_t* xb = static_cast<const uint8_t*>(X);
    uint32_t xoff[XPT];
    int xlds[XPT];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int q = tid + NT * i, row = q >> 3, part = q & 7;
        int r = mt0 + row;
        r = r < M ? r : M - 1;
        xoff[i] = (static_cast<uint32_t>(r) * static_cast<uint32_t>(K) + 8u * static_cast<uint32_t>(part)) * XE;
        xlds[i] = row * XS_ROW + 8 * (part ^ xswz(row));
    }
    uint4 xr[2][XPT][XR];
    auto load_x = [&](int step, int slot) {
        step += s_base;
        step = step < nsteps ? step : nsteps - 1;
        const uint32_t ko = static_cast<uint32_t>(step) * 64u * XE;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            xr[slot][i][0] = *reinterpret_cast<const uint4*>(xb + (xoff[i] + ko));
            if constexpr (XT == X_F32) xr[slot][i][1] = *reinterpret_cast<const uint4*>(xb + (xoff[i] + ko + 16u));
        }
    };
    auto store_x = [&](int slot, int buf) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            uint4 v;
            if constexpr (XT == X_F16) {
                v = xr[slot][i][0];
            } else {
                uint32_t o[4];
                f32x8_to_frag_nat(*reinterpret_cast<const float4*>(&xr[slot][i][0]),
                                  *reinterpret_cast<const float4*>(&xr[slot][i][1]), o);
                v = make_uint4(o[0], o[1], o[2], o[3]);
            }
            *reinterpret_cast<uint4*>(&xs[buf][xlds[i]]) = v;
        }
    };
    // A fragment of this lane for a = 0: row wm * 64 + j, 16-byte piece 4 ks + g
    // (16 a + wm * 64 does not change the row's swizzle)
    // (pair k order: pieces 2 g and 2 g + 1)
    const int arow = (wm * 64 + j) * XS_ROW;
    constexpr bool PAIR = TiledW<TYPE>::kPairOrder;
    const int pc0 = PAIR ? 2 * g : g, pc1 = PAIR ? 2 * g + 1 : 4 + g;
    const int aoff0 = arow + 8 * (pc0 ^ xswz(j)), aoff1 = arow + 8 * (pc1 ^ xswz(j));

    float4_t acc[4][NW];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int f = 0; f < NW; f++) acc[a][f] = float4_t{0.f, 0.f, 0.f, 0.f};

    // prologue: weights of steps 0..PD-1 and X of steps 0..2 in flight; tiles
    // of step 0 in LDS
#pragma unroll
    for (int r = 0; r < PD; r++) load_w(r, r);
    load_x(0, 0);
    load_x(1, 1);
    dequant_store(0, 0, 0);
    store_x(0, 0);
    load_x(2, 0);
    __syncthreads();

    // Loads complete in issue order (one vmcnt queue): the weights of step
    // s + PD go out at the start of step s and X of step s + 3 at its end
    // (scheduling fences keep that order); X(s + 1) is consumed at the end of
    // step s, two steps after its loads went out.
    for (int s0 = 0; s0 < nloc; s0 += PD) {
#pragma unroll
        for (int r = 0; r < PD; r++) {
            const int step = s0 + r, buf = r & 1;  // PD is even: buffer = step & 1
            load_w(step + PD, r);  // slot r held step `step`, dequantized during the previous step
            __builtin_amdgcn_sched_barrier(0);
            const uint4* bsrc = &bt[buf][0][wn * NW][0];
            const _Float16* asrc0 = &xs[buf][aoff0];
            const _Float16* asrc1 = &xs[buf][aoff1];
            // every fragment of the step is requested before the first MFMA:
            // one LDS latency per step instead of one per MFMA group
            Frag b[2][NW], af[2][4];
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
#pragma unroll
                for (int f = 0; f < NW; f++) {
                    const uint4 v = bsrc[(ks * (NF + 1) + f) * 64 + lane];
                    b[ks][f].u[0] = v.x; b[ks][f].u[1] = v.y; b[ks][f].u[2] = v.z; b[ks][f].u[3] = v.w;
                }
#pragma unroll
                for (int a = 0; a < 4; a++) {
                    const uint4 v = *reinterpret_cast<const uint4*>((ks ? asrc1 : asrc0) + a * 16 * XS_ROW);
                    af[ks][a].u[0] = v.x; af[ks][a].u[1] = v.y; af[ks][a].u[2] = v.z; af[ks][a].u[3] = v.w;
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int a = 0; a < 4; a++)
#pragma unroll
                    for (int f = 0; f < NW; f++) acc[a][f] = mfma16x16x32(af[ks][a], b[ks][f], acc[a][f]);
            // next step's tiles into the other buffers: weights of step + 1
            // (slot (r + 1) % PD), X of step + 1 (register slot (r + 1) % 2),
            // whose registers then take X of step + 3.  Past the last step the
            // (clamped) loads repeat the last step and the results are never
            // read: no branch in the loop body.
            dequant_store(step + 1, (r + 1) % PD, buf ^ 1);
            store_x((r + 1) & 1, buf ^ 1);
            __builtin_amdgcn_sched_barrier(0);
            load_x(step + 3, (r + 1) & 1);
            __syncthreads();
        }
    }

    if constexpr (KS == 2) {
        // group 1's stage is free (the last barrier ended every LDS read)
        float4_t* red = reinterpret_cast<float4_t*>(&stage[1]);
        if (grp == 1) {
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int f = 0; f < NW; f++) red[((a * NW + f) * (WM * WN) + wave) * 64 + lane] = acc[a][f];
        }
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int f = 0; f < NW; f++) acc[a][f] += red[((a * NW + f) * (WM * WN) + wave) * 64 + lane];
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
#pragma unroll
        for (int f = 0; f < NW; f++) {
            const int col = n0 + 16 * (wn * NW + f) + j;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = mt0 + wm * 64 + 16 * a + 4 * g + r;
                if (t < M) Y[static_cast<int64_t>(t) * N + col] = acc[a][f][r];
            }
        }
    }
}

// Tile configuration for M rows (sweeps on MI355X at N = 14336, K = 4096,
// against the 256 x 128 tile alone): M <= 64: 64-row tiles of 64 columns,
// 4 waves (M = 17: 27.0 us against 59.8 us); 64 < M <= 128: 128 x 64, 4
// waves (M = 100: 35.2 us against 60.8); 128 < M <= 256: 128 x 128, 8 waves
// (M = 256: 48.4 against 63.4); above, 256-row tiles of 128 or 96 columns
// (NF 8 / 6, whichever balances the grid over the CUs; M = 512: 70-72 us).  VB_GEMM_NF (6, 8) overrides NF of the large
// tiles; VB_GEMM_TILE="wm,wn,nf" (wm 1, 2, 4; wn 2, 4; nf 4, 6, 8 with wn
// dividing nf) any configuration.
struct TileCfg { int wm, wn, nf, ks; };

// Tiles that run with K halves (KS = 2, 512 threads, so at most 256
// registers a lane): wider ones spill.
constexpr bool ks2_tile(int wm, int wn, int nf) { return (nf == 4 && wm * wn <= 4) || (wm == 1 && wn == 4 && nf == 8); }

// Q6_K / Q8_0 run the tiled kernel from this M on (variant 0)
constexpr int64_t kKqTiledMinM = 65;

int64_t tile_count(const TileCfg& c, int64_t M, int64_t N) {
    return ((N + 16 * c.nf - 1) / (16 * c.nf)) * ((M + 64 * c.wm - 1) / (64 * c.wm));
}

TileCfg tiled_cfg(int type, int x_dtype, int64_t M, int64_t N, int64_t K) {
    const Knobs& kb = knobs();
    // K halves need a whole number of PD-step rounds per half
    const bool halves = (K / 64) % (2 * PD) == 0;
    if (kb.gemm_tile_wm) {
        const bool ks2 = kb.gemm_tile_ks == 2 && ks2_tile(kb.gemm_tile_wm, kb.gemm_tile_wn, kb.gemm_tile_nf) && halves;
        return TileCfg{kb.gemm_tile_wm, kb.gemm_tile_wn, kb.gemm_tile_nf, ks2 ? 2 : 1};
    }
    const int64_t kCUs = num_cus();
    if (type != TYPE_Q4_K) {
        // Q6_K / Q8_0: the largest tile whose grid still covers about the CUs
        // (MI355X: 4096 x 14336 takes 64 x 64 tiles up to M = 256 and
        // 128 x 64 at M = 512; 14336 x 4096 128 x 64 up to M = 128, 128 x 128
        // at 256, 256 x 96 or 128 above).  fp32 X keeps 96 columns on the
        // 256-row tile (128 spill).
        const int nf_big = x_dtype == X_F16 ? 8 : 6;
        const TileCfg order[4] = {{4, 2, nf_big, 1}, {2, 4, 8, 1}, {2, 2, 4, 1}, {1, 4, 4, 1}};
        for (const TileCfg& c : order)
            if (tile_count(c, M, N) * 8 >= kCUs * 7) return c;
        return order[3];
    }
    // Q4_K at N < 8192 (the down and attention shapes): narrow tiles with K
    // halves keep the grid covered (MI355X, 4096 x 14336: M = 128 / 256
    // 77.6 / 77.7 us on 64 x 64, M = 384 / 512 95.3 / 97.4 on 128 x 64,
    // against 96.4 / 142 / 210 / 211 with the wide-N choices; 4096 x 4096:
    // M = 128 / 256 / 512 24.5 / 25.0 / 30.8 against 29.7 / 44.3 / 65.4;
    // M = 1024 on 128 x 128: 153 against 170)
    if (N < 8192) {
        if (M <= 256) return TileCfg{1, 4, 4, halves ? 2 : 1};
        if (M <= 768) return TileCfg{2, 2, 4, halves ? 2 : 1};
        return TileCfg{2, 4, 8, 1};
    }
    // Q4_K, 33 <= M <= 128: K halves (M = 33 / 64 / 100 / 128 at 14336 x
    // 4096: 24.3 / 25.6 / 30.4 / 31.1 us against 26.9 / 27.3 / 35.4 / 35.6)
    if (M <= 64) return TileCfg{1, 4, 4, halves ? 2 : 1};
    if (M <= 128) return TileCfg{2, 2, 4, halves ? 2 : 1};
    if (M <= 256) return TileCfg{2, 4, 8, 1};
    if (kb.gemm_nf) return TileCfg{4, 2, kb.gemm_nf, 1};
    const int64_t mt = (M + 255) / 256;
    int best = 8;
    int64_t best_cost = -1;
    for (int nf = 8; nf >= 6; nf -= 2) {
        const int64_t tiles = mt * ((N + 16 * nf - 1) / (16 * nf));
        const int64_t cost = ((tiles + kCUs - 1) / kCUs) * nf;
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = nf;
        }
    }
    return TileCfg{4, 2, best, 1};
}

template <int TYPE, int XT, int NF, int WM, int WN>
void launch_tiled_cfg(const uint8_t* w, uint32_t wbytes, const void* X, float* Y, int M, int N, int K, int64_t rb,
                      int ks, int zs, hipStream_t st) {
    const dim3 grid(static_cast<uint32_t>((N + 16 * NF - 1) / (16 * NF)),
                    static_cast<uint32_t>((M + 64 * WM - 1) / (64 * WM)), static_cast<uint32_t>(zs));
    if constexpr (ks2_tile(WM, WN, NF)) {
        if (ks == 2) {
            gemm_tiled<TYPE, XT, NF, WM, WN, 2><<<grid, dim3(128 * WM * WN), 0, st>>>(w, wbytes, X, Y, M, N, K, rb);
            return;
        }
    }
    gemm_tiled<TYPE, XT, NF, WM, WN, 1><<<grid, dim3(64 * WM * WN), 0, st>>>(w, wbytes, X, Y, M, N, K, rb);
}

template <int TYPE, int XT>
int launch_tiled(const TileCfg& c, const uint8_t* w, uint32_t wbytes, const void* X, float* Y, int M, int N, int K,
                 int64_t rb, hipStream_t st, int zs = 1) {
#define VB_TILE(WM_, WN_, NF_)                                                              \
    if (c.wm == WM_ && c.wn == WN_ && c.nf == NF_) {                                       \
        launch_tiled_cfg<TYPE, XT, NF_, WM_, WN_>(w, wbytes, X, Y, M, N, K, rb, c.ks, zs, st);  \
        return OK;                                                                          \
    }
    VB_TILE(4, 2, 8)
    VB_TILE(4, 2, 6)
    VB_TILE(4, 2, 4)
    VB_TILE(2, 4, 8)
    VB_TILE(2, 4, 4)
    VB_TILE(2, 2, 8)
    VB_TILE(2, 2, 6)
    VB_TILE(2, 2, 4)
    VB_TILE(1, 4, 8)
    VB_TILE(1, 4, 4)
    VB_TILE(1, 2, 4)
    VB_TILE(1, 2, 6)
#undef VB_TILE
    set_error("vb_gemm: no tiled kernel for wm=%d wn=%d nf=%d", c.wm, c.wn, c.nf);
    return E_INVAL;
}

}  // namespace

// K split between workgroups for Q6_K / Q8_0 with fp16 X at M >= 384 and
// N < 8192 (the FFN down projection, 4096 x 14336): the 256 x 128 tile,
// whose grid alone (32 x 2 tiles at M = 512) leaves most CUs idle, in as
// many K splits as fill the CUs; each split a whole number of PD-step rounds.
// Returns 1 when the shape does not take it.
int tiled_zsplit(int type, int x_dtype, int64_t M, int64_t N, int64_t K) {
    if ((type != TYPE_Q6_K && type != TYPE_Q8_0) || x_dtype != X_F16 || M < 384 || N >= 8192) return 1;
    if (knobs().gemm_tile_wm) {
        // VB_GEMM_TILE with VB_GEMM_ZSPLIT: that tile in that many splits
        const int z = knobs().gemm_zsplit;
        const int64_t nsteps = K / 64;
        return z >= 2 && z <= 8 && nsteps % (z * PD * knobs().gemm_tile_ks) == 0 ? z : 1;
    }
    const int64_t tiles = tile_count(TileCfg{4, 2, 8, 1}, M, N);
    const int64_t nsteps = K / 64;
    for (int64_t z = num_cus() / (tiles > 0 ? tiles : 1); z >= 2; z--)
        if (z <= 8 && nsteps % (z * PD) == 0 && nsteps / z >= 4 * PD) return static_cast<int>(z);
    return 1;
}

// The 32-element block types (Q4_0, Q4_1, Q5_0, Q5_1) have their decoder in
// the K-split, tiled and packed-X kernels.  The types without a fused
// decoder: Q2_K, Q3_K, BF16 and F32 weights are decoded once to fp16 (each
// value rounded once, as the fused decoders round) into the workspace, then
// multiplied on the tiled kernel with fp16 weights; F16 weights are used in
// place.  The workspace,
// n x k x 2 bytes (none for F16), comes from the caller (vb_gemm_ws) or is
// allocated on the stream for the call (hipMallocAsync / hipFreeAsync).
bool gemm_b32_type(int32_t type) {
    return type == TYPE_Q4_0 || type == TYPE_Q4_1 || type == TYPE_Q5_0 || type == TYPE_Q5_1;
}

bool gemm_b32_high(int32_t type) { return type == TYPE_Q5_0 || type == TYPE_Q5_1; }

// Largest M the 32-element types take the K-split kernel at by default.
// MI355X, fp16 X, Q4_0 / Q5_1: 14336 x 4096 at M = 1 / 8 / 64 / 128: 16.6 /
// 19.7 / 31.9 / 55.9 and 17.3 / 19.9 / 34.4 / 59.3 us, against 76-79 us
// through the fp16 decode pass and the tiled kernel; 4096 x 14336 at M = 8 /
// 128: 18.7 / 90.5 and 18.8 / 94.5 against 112-115.  The packed-X kernel at
// M = 512: 61.3 / 66.9 us (14336 x 4096) and 72.2 / 78.0 (4096 x 14336)
// against 114.8-145.2.
// At N < 8192 the K-split kernel stays ahead up to M = 256 (Q4_0 / Q5_1,
// 4096 x 14336, M = 192 / 256: 87.6 / 87.1 and 90.9 / 89.9 us, against
// 114.5-115.1 and 241.7-242.7 on the tiled kernel with TiledB32, about 114
// through the decode pass).
int64_t gemm_b32_kq_max_m(int64_t N) { return N < 8192 ? 256 : 128; }

bool gemm_other_type(int32_t type) {
    return type == TYPE_F32 || type == TYPE_F16 || type == TYPE_BF16 || type == TYPE_Q2_K || type == TYPE_Q3_K;
}

int64_t gemm_other_workspace(int32_t type, int64_t N, int64_t K) { return type == TYPE_F16 ? 0 : N * K * 2; }

int gemm_other(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K, int32_t type,
               int32_t variant, void* ws, size_t ws_bytes, hipStream_t st) {
    if (variant != 0 && variant != 2) {
        set_error("vb_gemm: type %d runs the tiled kernel only (variant 0 or 2, got %d)", type, variant);
        return E_UNSUPPORTED;
    }
    if (K % 256 != 0) {
        set_error("vb_gemm: type %d needs K %% 256 == 0 for M >= 2 or fp16 X (K=%lld)", type,
                  static_cast<long long>(K));
        return E_UNSUPPORTED;
    }
    const int64_t xbytes = M * K * (x_dtype == X_F16 ? 2 : 4);
    const int64_t wbytes = N * K * 2;
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || wbytes >= (int64_t(1) << 32) ||
        xbytes >= (int64_t(1) << 32)) {
        set_error("vb_gemm: shape too large (M=%lld N=%lld K=%lld)", static_cast<long long>(M),
                  static_cast<long long>(N), static_cast<long long>(K));
        return E_INVAL;
    }
    const uint8_t* wf = static_cast<const uint8_t*>(w);
    void* own = nullptr;
    int rc = OK;
    if (type != TYPE_F16) {
        void* buf = ws;
        if (!buf || static_cast<int64_t>(ws_bytes) < wbytes || reinterpret_cast<uintptr_t>(buf) % 16) {
            if (hipMallocAsync(&own, static_cast<size_t>(wbytes), st) != hipSuccess) {
                (void)hipGetLastError();
                set_error("vb_gemm: could not allocate %lld bytes for the fp16 weights", static_cast<long long>(wbytes));
                return E_NOMEM;
            }
            buf = own;
        }
        rc = dequant_rows_f16(w, static_cast<_Float16*>(buf), N, K, type, st);
        wf = static_cast<const uint8_t*>(buf);
    }
    if (rc == OK) {
        const TileCfg cfg = tiled_cfg(TYPE_F16, x_dtype, M, N, K);
        const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_F16, X_F16>(cfg, wf, static_cast<uint32_t>(wbytes), X, Y, m, n, k,
                                                              K * 2, st)
                              : launch_tiled<TYPE_F16, X_F32>(cfg, wf, static_cast<uint32_t>(wbytes), X, Y, m, n, k,
                                                              K * 2, st);
        if (rc == OK) rc = check_launch("vb_gemm");
    }
    if (own && hipFreeAsync(own, st) != hipSuccess && rc == OK) {
        (void)hipGetLastError();
        set_error("vb_gemm: could not free the fp16 weights");
        rc = E_HIP;
    }
    return rc;
}

int gemm_dispatch(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K,
                  int32_t type, int32_t variant, void* ws, size_t ws_bytes, hipStream_t st) {
    if (type != TYPE_Q4_K && type != TYPE_Q6_K && type != TYPE_Q8_0 && type != TYPE_Q5_K && !gemm_b32_type(type) &&
        !gemm_other_type(type)) {
        set_error("vb_gemm: weight type %d has no batched path", type);
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
    // Q8_0: the batched kernels step K by 128; the rule holds at every M, the
    // one row that runs on the GEMV included, so a shape valid at M = 1 is
    // valid at M = 2
    if (type == TYPE_Q8_0 && K % 128 != 0) {
        set_error("vb_gemm: Q8_0 weights need K %% 128 == 0 (K=%lld)", static_cast<long long>(K));
        return E_UNSUPPORTED;
    }
    // one row: the GEMV (the short-row and split-row kernels; rel-L2 near
    // 5e-5, and at 14336 x 4096 on MI355X 7.4 us against 11.8 us for the
    // skinny tile).  fp32 X for every type; fp16 X on the short-row kernels
    // (k <= 4096) and the split-row kernels (4096 < k <= 16384).
    if (variant == 0 && M == 1) {
        if (x_dtype == X_F32) return gemv_dispatch(w, static_cast<const float*>(X), Y, N, K, type, st);
        if (type == TYPE_Q4_K && K <= 4096 && K % 256 == 0 && !knobs().gemv_q4k_general && N <= INT32_MAX &&
            gemv_q4k_rpw(N) > 0)
            return gemv_q4k_short(w, X, Y, N, K, st, true);
        // Q4_K, 4096 < k <= 16384: the split-row kernel
        if (type == TYPE_Q4_K && K > 4096 && K % 256 == 0 && !knobs().gemv_q4k_general &&
            gemv_q4k_split_rpw(N, K) > 0)
            return gemv_q4k_split(w, X, Y, nullptr, N, K, st, true);
        // Q6_K (k = 2048 / 4096) and Q8_0 (k % 256 == 0, k <= 4096) on their
        // short-row kernel, as vb_gemv takes them
        const bool general = type == TYPE_Q6_K ? knobs().gemv_q6k_general : knobs().gemv_q8_general;
        if (type != TYPE_Q4_K && !general && gemv_short_rpw(type, N, K) > 0)
            return gemv_short(type, w, X, Y, N, K, st, true);
        // and 4096 < k <= 16384 on their split-row kernel
        if (type != TYPE_Q4_K && !general && K > 4096 && gemv_split_rpw(type, N, K) > 0)
            return gemv_split(type, w, X, Y, nullptr, N, K, st, true);
    }
    if (gemm_b32_type(type)) {
        // Q4_0 / Q4_1 / Q5_0 / Q5_1: their decoder in the K-split kernel at
        // small M (variant 4) and in the packed-X kernel for M > 256 with a
        // workspace (variant 5); between, the fp16 decode pass and the tiled
        // kernel (variants 0, 2)
        if (variant == 4 || (variant == 0 && M <= gemm_b32_kq_max_m(N)))
            return gemm_kq(w, X, x_dtype, Y, M, N, K, type, st);
        const int64_t xr_need = gemm_xr_workspace(M, N, K);
        const bool xr_ok = x_dtype == X_F16 && M >= 256 && K % 256 == 0 && M <= INT32_MAX && N <= INT32_MAX &&
                           K <= INT32_MAX && ((N * rb + 3) & ~int64_t(3)) < (int64_t(1) << 32) &&
                           M * K * 2 < (int64_t(1) << 32) && ws != nullptr &&
                           static_cast<int64_t>(ws_bytes) >= xr_need && reinterpret_cast<uintptr_t>(ws) % 16 == 0;
        if (variant == 5) {
            if (!xr_ok) {
                set_error("vb_gemm: variant 5 takes fp16 X, m >= 256, k %% 256 == 0 and a 16-byte-aligned workspace "
                          "of %lld bytes", static_cast<long long>(xr_need));
                return E_INVAL;
            }
            return gemm_xr(w, X, Y, M, N, K, type, ws, st);
        }
        if (variant == 0 && xr_ok && M > 256 && (N >= 8192 || gemm_xr_ksplit(M, N, K) > 1))
            return gemm_xr(w, X, Y, M, N, K, type, ws, st);
    }
    bool tiled = false;
    if (gemm_b32_type(type)) {
        // the tiled kernel with its own decoder (TiledB32); by default for
        // the 4-bit types only: the 5-bit ones run the fp16 decode pass
        // there (14336 x 4096, M = 192 / 256: Q4_0 72.0 / 73.1 us tiled,
        // about 80 through the decode pass; Q5_1 106.7 / 105.5 tiled)
        if (variant == 0 && gemm_b32_high(type))
            return gemm_other(w, X, x_dtype, Y, M, N, K, type, variant, ws, ws_bytes, st);
        if (variant != 0 && variant != 2) {
            set_error("vb_gemm: type %d runs the K-split, tiled and packed-X kernels (variant 0, 2, 4 or 5, got %d)",
                      type, variant);
            return E_UNSUPPORTED;
        }
        if (K % 256 != 0) {
            set_error("vb_gemm: the tiled kernel takes K %% 256 == 0 (K=%lld)", static_cast<long long>(K));
            return E_UNSUPPORTED;
        }
        tiled = true;
    } else if (gemm_other_type(type)) {
        return gemm_other(w, X, x_dtype, Y, M, N, K, type, variant, ws, ws_bytes, st);
    }
    if (type == TYPE_Q5_K) {
        // Q5_K: the K-split kernel at small M (every x dtype, M = 1
        // included), the tiled kernel with its fused decoder above, and the
        // packed-X kernel where Q4_K takes it.  MI355X, fp16 X: 14336 x 4096
        // at M = 2 / 8 / 32 / 64: 26.4 / 28.6 / 29.7 / 37.7 us K-split against
        // 36.2-36.9 tiled; 4096 x 14336 at M = 2 / 8 / 64 / 128: 21.7 / 25.5 /
        // 67.3 / 109.1 against 94.2 / 94.3 / 97.6 / 96.0 tiled; M = 512 on the
        // packed-X kernel 65.7 / 77.5 us against 78.1 / 119.4 tiled.
        if (variant != 0 && variant != 2 && variant != 4 && variant != 5) {
            set_error("vb_gemm: Q5_K runs the tiled, K-split and packed-X kernels (variant 0, 2, 4 or 5, got %d)",
                      variant);
            return E_UNSUPPORTED;
        }
        if (variant == 4 || (variant == 0 && M <= (N < 8192 ? 64 : 32)))
            return gemm_kq(w, X, x_dtype, Y, M, N, K, type, st);
        tiled = true;
    } else if (type == TYPE_Q6_K || type == TYPE_Q8_0) {
        // Q6_K / Q8_0: the K-split kernel (gemm_kq.hip) up to M = 64, where
        // it decodes each weight once; above, the tiled kernel, which decodes
        // each weight once per 64-256 rows of M (the K-split kernel once per
        // 64).  The tiled kernel takes K % 256 == 0.
        if (variant != 0 && variant != 2 && variant != 4 && variant != 5) {
            set_error("vb_gemm: variant %d is Q4_K-only (use 0, 2, 4 or 5 for Q6_K / Q8_0)", variant);
            return E_UNSUPPORTED;
        }
        if ((variant == 2 || variant == 5) && K % 256 != 0) {
            set_error("vb_gemm: the tiled and packed-X kernels take K %% 256 == 0 for Q6_K / Q8_0 (K=%lld)",
                      static_cast<long long>(K));
            return E_UNSUPPORTED;
        }
        // At N < 8192 the K-split kernel stays ahead for Q6_K up to M = 256
        // with fp16 X (MI355X, 4096 x 14336, M = 65-256: 88-100 us against
        // 105-112 tiled) and for both types up to M = 128 with fp32 X (Q8_0
        // M = 65 / 128: 100 / 113 against 107 / 121); Q8_0 with fp16 X runs
        // tiled from M = 65 (93-95 us against 95-109)
        const int kq_max = x_dtype == X_F16 ? (type == TYPE_Q6_K ? 256 : 0) : 128;
        const bool kq_narrow = N < 8192 && M <= kq_max;
        tiled = variant == 2 || variant == 5 || (variant == 0 && M >= kKqTiledMinM && K % 256 == 0 && !kq_narrow);
        if (!tiled) return gemm_kq(w, X, x_dtype, Y, M, N, K, type, st);
    } else if (variant == 4) {
        return gemm_kq(w, X, x_dtype, Y, M, N, K, type, st);
    }
    // 17 <= M <= 32: skinny tiles with two activation tiles per wave for fp16
    // X or N >= 12288, else the K-split kernel (gemm_kq.hip).  On MI355X, fp16
    // X: 14.5 / 17.5 us at M = 17 / 32 for N = 14336, K = 4096 (K-split 21.5 /
    // 24.8, tiled 27.0 / 27.1); 11.5 / 13.3 us at 4096 x 4096 (tiled 26.6);
    // fp32 X at N = 4096 the K-split kernel is 5 % ahead.
    if (!tiled && variant == 0 && M >= 17 && M <= 32 && x_dtype != X_F16 && N < 12288)
        return gemm_kq(w, X, x_dtype, Y, M, N, K, type, st);
    // 33 <= M <= 64 at N < 8192: the K-split kernel (4096 x 14336, M = 64:
    // 63.5 us against 79.3 tiled); M <= 16 there too when K >= 8192 (M = 2 /
    // 4 / 8 / 9 / 16: 18.1 / 19.5 / 21.8 / 21.9 / 26.6 us against 23.1 / 23.3
    // / 23.8 / 23.9 / 26.7 skinny; at 4096 x 4096 the skinny kernel stays
    // ahead, 9.4 against 9.9 at M = 8)
    if (!tiled && variant == 0 && M >= 33 && M <= 64 && N < 8192)
        return gemm_kq(w, X, x_dtype, Y, M, N, K, type, st);
    if (!tiled && variant == 0 && M >= 2 && M <= 16 && N < 8192 && K >= 8192)
        return gemm_kq(w, X, x_dtype, Y, M, N, K, type, st);
    // 33 <= M <= 64, fp16 X, N >= 8192: four activation tiles per wave
    // (14336 x 4096, M = 33 / 48 / 64: 18.6 / 21.5 / 25.8 us against 24.5 /
    // 25.1 / 25.9 tiled; at N < 8192 the K-split kernel above stays ahead)
    const bool skinny = !tiled && (variant == 1 || (variant == 0 && (M <= 32 || (M <= 64 && x_dtype == X_F16))));
    if (skinny) {
        if (M > (x_dtype == X_F16 ? 64 : 32)) {
            set_error("vb_gemm: variant 1 (skinny) takes M <= 32 (64 with fp16 X), got %lld",
                      static_cast<long long>(M));
            return E_INVAL;
        }
        return gemm_q4k_skinny(w, X, x_dtype, Y, M, N, K, st);
    }
    if (variant < 0 || variant > 5) {
        set_error("vb_gemm: unknown variant %d", variant);
        return E_INVAL;
    }
    if ((variant == 3 || variant == 5) && x_dtype != X_F16) {
        set_error("vb_gemm: variant %d (role-split / X in registers) takes fp16 X", variant);
        return E_INVAL;
    }
    const int64_t xbytes = M * K * (x_dtype == X_F16 ? 2 : 4);
    const int64_t wbytes = (N * rb + 3) & ~int64_t(3);  // whole dwords (buffer resource of Q6_K / Q8_0)
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || (M + 63) / 64 > 65535 ||
        wbytes >= (int64_t(1) << 32) || xbytes >= (int64_t(1) << 32)) {
        set_error("vb_gemm: shape too large (M=%lld N=%lld K=%lld)", static_cast<long long>(M),
                  static_cast<long long>(N), static_cast<long long>(K));
        return E_INVAL;
    }
    // 256 < M <= 768, fp16 X: the role-split kernel (gemm_split.hip; at
    // N = 14336, K = 4096 on MI355X 67.9 / 72.0 us at M = 384 / 512 against
    // 71.0 / 74.8 tiled, behind at M = 256 and 1024)
    const int smin = knobs().gemm_split_min_m >= 0 ? knobs().gemm_split_min_m : 257;
    // (at N >= 8192 only: at 4096 x 14336 it ran 211 us against 97 us tiled)
    const bool split_range = smin > 0 && M >= smin && M <= 768 && N >= 8192;
    // 256 < M, N >= 8192, fp16 X, with a workspace: X packed in fragment
    // order and loaded straight into registers (gemm_xr.hip; at N = 14336,
    // K = 4096 on MI355X, pack pass included: M = 384 / 512 / 1024 at 62.8 /
    // 62.6 / 117.5 us against 68.5 / 70.7 / 139.9 us on the role-split and
    // tiled kernels; behind at M = 256, 50.8 against 48.5)
    // With fewer output tiles than CUs (the down projection 4096 x 14336 at
    // M = 512) the same kernel splits K (gemm_xr_ksplit) and a small
    // launch adds the partial products in a fixed order.  Q6_K and Q8_0 take
    // it at the same shapes (MI355X, M = 512: 14336 x 4096 Q6_K / Q8_0 70.0 /
    // 67.9 us against 84.6 / 81.7 on the tiled kernel; 4096 x 14336 84.1 /
    // 80.1 against 85.9 / 83.2 with its K splits; M = 1024 at 14336 x 4096:
    // 131.3 / 124.9 against 165.0 / 156.7).
    const bool xr_auto = variant == 0 && gemm_xr_type(type) &&
                         (type == TYPE_Q4_K || type == TYPE_Q5_K || knobs().gemm_xr_kq) &&
                         x_dtype == X_F16 && M > 256 && K % 256 == 0 &&
                         (N >= 8192 || gemm_xr_ksplit(M, N, K) > 1) && ws != nullptr &&
                         static_cast<int64_t>(ws_bytes) >= gemm_xr_workspace(M, N, K) &&
                         reinterpret_cast<uintptr_t>(ws) % 16 == 0;
    if (xr_auto) return gemm_xr(w, X, Y, M, N, K, type, ws, st);
    if (variant == 5) {
        if (M < 256) {
            set_error("vb_gemm: variant 5 (X in registers) takes m >= 256, got %lld", static_cast<long long>(M));
            return E_INVAL;
        }
        const int64_t need = gemm_xr_workspace(M, N, K);
        if (!ws || static_cast<int64_t>(ws_bytes) < need || reinterpret_cast<uintptr_t>(ws) % 16) {
            set_error("vb_gemm: variant 5 needs a 16-byte-aligned workspace of %lld bytes (got %zu)",
                      static_cast<long long>(need), ws_bytes);
            return E_INVAL;
        }
        return gemm_xr(w, X, Y, M, N, K, type, ws, st);
    }
    if (type == TYPE_Q4_K && (variant == 3 || (variant == 0 && x_dtype == X_F16 && split_range))) {
        return gemm_q4k_split(w, X, Y, M, N, K, st);
    }
    const TileCfg cfg = tiled_cfg(type, x_dtype, M, N, K);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    const uint32_t wby = static_cast<uint32_t>(wbytes);
    int rc;
    // K split between workgroups (partial products in the workspace)
    const int zs = variant == 0 ? tiled_zsplit(type, x_dtype, M, N, K) : 1;
    if (zs > 1 && ws && static_cast<int64_t>(ws_bytes) >= zs * M * N * 4 && reinterpret_cast<uintptr_t>(ws) % 16 == 0) {
        float* part = static_cast<float*>(ws);
        const TileCfg big = knobs().gemm_tile_wm ? cfg : TileCfg{4, 2, 8, 1};
        rc = type == TYPE_Q6_K ? launch_tiled<TYPE_Q6_K, X_F16>(big, wb, wby, X, part, m, n, k, rb, st, zs)
                               : launch_tiled<TYPE_Q8_0, X_F16>(big, wb, wby, X, part, m, n, k, rb, st, zs);
        if (rc != OK) return rc;
        if ((rc = check_launch("vb_gemm")) != OK) return rc;
        return gemm_ksum(part, Y, M * N, zs, st);
    }
    if (type == TYPE_Q4_K)
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_Q4_K, X_F16>(cfg, wb, wby, X, Y, m, n, k, rb, st)
                              : launch_tiled<TYPE_Q4_K, X_F32>(cfg, wb, wby, X, Y, m, n, k, rb, st);
    else if (type == TYPE_Q6_K)
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_Q6_K, X_F16>(cfg, wb, wby, X, Y, m, n, k, rb, st)
                              : launch_tiled<TYPE_Q6_K, X_F32>(cfg, wb, wby, X, Y, m, n, k, rb, st);
    else if (type == TYPE_Q5_K)
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_Q5_K, X_F16>(cfg, wb, wby, X, Y, m, n, k, rb, st)
                              : launch_tiled<TYPE_Q5_K, X_F32>(cfg, wb, wby, X, Y, m, n, k, rb, st);
    else if (type == TYPE_Q4_0)
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_Q4_0, X_F16>(cfg, wb, wby, X, Y, m, n, k, rb, st)
                              : launch_tiled<TYPE_Q4_0, X_F32>(cfg, wb, wby, X, Y, m, n, k, rb, st);
    else if (type == TYPE_Q4_1)
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_Q4_1, X_F16>(cfg, wb, wby, X, Y, m, n, k, rb, st)
                              : launch_tiled<TYPE_Q4_1, X_F32>(cfg, wb, wby, X, Y, m, n, k, rb, st);
    else if (type == TYPE_Q5_0)
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_Q5_0, X_F16>(cfg, wb, wby, X, Y, m, n, k, rb, st)
                              : launch_tiled<TYPE_Q5_0, X_F32>(cfg, wb, wby, X, Y, m, n, k, rb, st);
    else if (type == TYPE_Q5_1)
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_Q5_1, X_F16>(cfg, wb, wby, X, Y, m, n, k, rb, st)
                              : launch_tiled<TYPE_Q5_1, X_F32>(cfg, wb, wby, X, Y, m, n, k, rb, st);
    else
        rc = x_dtype == X_F16 ? launch_tiled<TYPE_Q8_0, X_F16>(cfg, wb, wby, X, Y, m, n, k, rb, st)
                              : launch_tiled<TYPE_Q8_0, X_F32>(cfg, wb, wby, X, Y, m, n, k, rb, st);
    if (rc != OK) return rc;
    return check_launch("vb_gemm");
}

}  // namespace vb

extern "C" int vb_gemm(const void* w, const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n,
                       int64_t k, int32_t ggml_type, int32_t variant, void* stream) {
    return vb::gemm_dispatch(w, x, x_dtype, y, m, n, k, ggml_type, variant, nullptr, 0, vb::as_stream(stream));
}

extern "C" int64_t vb_gemm_workspace(int64_t m, int64_t n, int64_t k, int32_t ggml_type, int32_t x_dtype,
                                     int32_t variant) {
    if (k <= 0 || k % 256 != 0 || m <= 0 || n <= 0) return 0;
    // the 32-element types: none on the K-split kernel, the packed X (and
    // partial products) on the packed-X kernel
    if (vb::gemm_b32_type(ggml_type)) {
        if ((variant == 0 && m <= vb::gemm_b32_kq_max_m(n)) || variant == 4) return 0;
        if ((variant == 5 && m >= 256 && x_dtype == 1) ||
            (variant == 0 && x_dtype == 1 && m > 256 && (n >= 8192 || vb::gemm_xr_ksplit(m, n, k) > 1)))
            return vb::gemm_xr_workspace(m, n, k);
        // the tiled kernel (variant 2; variant 0 for Q4_0 / Q4_1), or the
        // fp16 decode pass (variant 0, Q5_0 / Q5_1)
        return variant == 0 && vb::gemm_b32_high(ggml_type) ? n * k * 2 : 0;
    }
    // the other types: their fp16 decode (none where the call runs the GEMV)
    if (vb::gemm_other_type(ggml_type))
        return m == 1 && x_dtype == 0 && variant == 0 ? 0 : vb::gemm_other_workspace(ggml_type, n, k);
    if (x_dtype != 1) return 0;
    if (!vb::gemm_xr_type(ggml_type)) return 0;
    // the shapes gemm_dispatch sends to the packed-X kernel
    const bool xr_on = ggml_type == vb::TYPE_Q4_K || ggml_type == vb::TYPE_Q5_K || vb::knobs().gemm_xr_kq;
    if ((variant == 5 && m >= 256) ||
        (variant == 0 && xr_on && m > 256 && (n >= 8192 || vb::gemm_xr_ksplit(m, n, k) > 1)))
        return vb::gemm_xr_workspace(m, n, k);
    if (ggml_type == vb::TYPE_Q6_K || ggml_type == vb::TYPE_Q8_0) {
        // the tiled kernel's K splits: one fp32 partial product each
        const int zs = variant == 0 ? vb::tiled_zsplit(ggml_type, x_dtype, m, n, k) : 1;
        return zs > 1 ? static_cast<int64_t>(zs) * m * n * 4 : 0;
    }
    return 0;
}

extern "C" int vb_gemm_ws(const void* w, const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n, int64_t k,
                          int32_t ggml_type, int32_t variant, void* workspace, size_t workspace_bytes, void* stream) {
    return vb::gemm_dispatch(w, x, x_dtype, y, m, n, k, ggml_type, variant, workspace, workspace_bytes,
                             vb::as_stream(stream));
}
