// Role-split dequant-fused GEMM for large M (fp16 X): Y[M, N] = X[M, K] .
// W[N, K]^T with W Q4_K (GGUF layout), Y fp32 row-major.
//
// Replaces, like gemm.hip, the reference's per-token loop of gemv_dequant
// (cpp/src/fast_model.cpp:644-669, :905-960) for prefill-sized batches.
//
// Why a second large-M kernel: in gemm_tiled (gemm.hip) every wave of a workgroup
// loads, dequantizes, stages and multiplies in lockstep behind one barrier
// per k-step, so those costs add up instead of overlapping (at M = 512 each
// of them removed alone saves 8-16 us of ~72 us).  Here the eight waves of
// a workgroup take two roles, one of each on every SIMD:
//  * producers (waves 4-7) stream the raw Q4_K bytes of the workgroup's
//    BN = 16 NF weight rows PD steps ahead (a super-block's header once per
//    four steps), dequantize each 64-element chunk into fp16 B fragments
//    (natural k order, mfma_q4k.hpp), and stage the workgroup's X tile
//    (256 rows x 64 fp16 per step, whole 128-byte rows, loaded two steps
//    ahead into registers); both go into rings of three LDS buffers, two
//    k-steps ahead of the consumers;
//  * consumers (waves 0-3) own 64 X rows each: they read the A and B
//    fragments of a step from LDS (the ks = 1 half under the ks = 0 MFMAs,
//    the next step's ks = 0 half under the ks = 1 MFMAs) and issue 4 x NF
//    MFMAs per 32-element half step.
// One barrier per step orders the rings: the buffer written during step s
// (that of step s + 2) was last read during steps s - 2 and s - 1, before
// the barrier that ends step s - 1, and is read from step s + 1 on, after
// the barrier that ends step s.
//
// Tile: 256 X rows x 112 weight rows (NF = 7): at N = 14336 that is 128
// column tiles, so M = 512 runs exactly 256 workgroups, one per CU.
#include "mfma_q4k.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int CW = 4;            // consumer waves (one per SIMD), 64 X rows each
constexpr int TM = 64 * CW;      // X rows per workgroup
constexpr int PT = 64 * CW;      // producer threads
constexpr int NTHR = 2 * 64 * CW;
constexpr int PD = 4;            // raw weight prefetch distance (steps)

template <int NF>
__global__ void __launch_bounds__(NTHR) gemm_q4k_split_kernel(const uint8_t* __restrict__ w,
                                                              const uint8_t* __restrict__ X,
                                                              float* __restrict__ Y, int M, int N, int K,
                                                              int64_t rb) {
    constexpr int NU = 64 * NF;                // dequant units per step (8 qs bytes of one row each)
    constexpr int UPT = (NU + PT - 1) / PT;    // units per producer thread
    constexpr int BUF = 2 * (NF + 1) * 64;     // uint4 per ring buffer: [ks][fragment][lane]
    // fragment NF of each half takes the stores of producer threads without
    // a unit (keeps their code branch-free)
    constexpr int XBUF = TM * 128;            // bytes of one X ring buffer (256 rows x 64 fp16)
    __shared__ uint4 bt[3 * BUF];
    __shared__ uint4 xring[3 * XBUF / 16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(tid >> 6));
    // Workgroups are dealt to the 8 XCDs round robin (linear id % 8); with
    // two M-tiles each XCD works on one of them, so its L2 holds one M-tile
    // of X (1 MB at K = 4096).
    const int nt = static_cast<int>(gridDim.x), mt = static_cast<int>(gridDim.y);
    int tile_n = static_cast<int>(blockIdx.x), tile_m = static_cast<int>(blockIdx.y);
    if (mt == 2 && nt % 4 == 0) {
        const int lin = tile_n + nt * tile_m, xcd = lin & 7, r = lin >> 3;
        tile_m = xcd >> 2;
        tile_n = (xcd & 3) * (nt >> 2) + r;
    }
    const int mt0 = tile_m * TM;
    const int n0 = tile_n * 16 * NF;
    const int nsteps = K / 64;  // a multiple of 4

    if (wave < CW) {
        // ---- consumer: X rows mt0 + 64 wave + [0, 64) of the X ring ----
        const int j = lane & 15, g = lane >> 4;
        const uint8_t* const xs = reinterpret_cast<const uint8_t*>(xring) + wave * (64 * 128);
        // A fragment (a, ks): row 16 a + j, piece 4 ks + g; (16 a + j) / 2 % 8
        // does not depend on a
        const int aoff[2] = {16 * (j * 8 + (g ^ ((j >> 1) & 7))), 16 * (j * 8 + ((4 + g) ^ ((j >> 1) & 7)))};
        auto read_a = [&](int buf, int ks, Frag* af) {
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const uint4 v = *reinterpret_cast<const uint4*>(xs + buf * XBUF + aoff[ks] + a * 16 * 128);
                af[a].u[0] = v.x; af[a].u[1] = v.y; af[a].u[2] = v.z; af[a].u[3] = v.w;
            }
        };
        auto read_b = [&](int buf, int ks, Frag* b) {
            const uint4* src = bt + buf * BUF + ks * (NF + 1) * 64 + lane;
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

        __syncthreads();  // ring buffers 0 and 1 (steps 0, 1) written
        Frag b0[NF], a0[4];
        read_b(0, 0, b0);
        read_a(0, 0, a0);
        int bc = 0, bn = 1;  // ring buffers of steps s, s + 1
        for (int step = 0; step < nsteps; step++) {
            // fences keep each group of reads ahead of the MFMAs it is meant
            // to overlap (the scheduler would sink them) and the MFMAs ahead
            // of the barrier (it would hoist them past)
            Frag b1[NF], a1[4];
            read_b(bc, 1, b1);
            read_a(bc, 1, a1);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(a0, b0);
            __builtin_amdgcn_sched_barrier(0);
            read_b(bn, 0, b0);  // after the last step: unused
            read_a(bn, 0, a0);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(a1, b1);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            bc = bn;
            bn = bn == 2 ? 0 : bn + 1;
        }

#pragma unroll
        for (int a = 0; a < 4; a++) {
#pragma unroll
            for (int f = 0; f < NF; f++) {
                const int col = n0 + 16 * f + j;
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = mt0 + 64 * wave + 16 * a + 4 * g + r;
                    if (t < M) Y[static_cast<int64_t>(t) * N + col] = acc[a][f][r];
                }
            }
        }
    } else {
        // ---- producer: dequant unit u = ptid + PT i is LDS lane slot u of a
        // half: fragment u / 64, lane l = u % 64 -> weight row 16 (u / 64) +
        // l % 16, qs part l / 16; each wave stores 1 KB contiguous.  A
        // super-block's 16-byte header (d, dmin, scales) serves its four
        // steps: it is loaded once, four steps ahead, into one of two slots
        // (super-blocks alternate); the 8 qs bytes of a step PD steps ahead.
        const int ptid = tid - 64 * CW;
        const int nsb = nsteps >> 2;
        uint32_t urow[UPT], uq[UPT];
        int uslot[UPT];
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            int u = ptid + PT * i;
            const bool live = u < NU;
            u = live ? u : NU - 1;
            const int l = u & 63, un = 16 * (u >> 6) + (l & 15), ug = l >> 4;
            int n = n0 + un;
            n = n < N ? n : N - 1;  // rows past N repeat row N - 1; never stored
            urow[i] = static_cast<uint32_t>(n) * static_cast<uint32_t>(rb);
            uq[i] = 16u + 8u * static_cast<uint32_t>(ug);
            uslot[i] = live ? u : NF * 64 + lane;
        }
        uint4 hd[2][UPT];   // headers of super-blocks sb0 (slot 0) and sb0 + 1 (slot 1)
        uint2 wqs[PD][UPT];
        auto load_hd = [&](int sb, int slot) {
            sb = sb < nsb ? sb : nsb - 1;
#pragma unroll
            for (int i = 0; i < UPT; i++)
                hd[slot][i] = *reinterpret_cast<const uint4*>(w + (urow[i] + static_cast<uint32_t>(sb) * 144u));
        };
        auto load_qs = [&](int step, int slot) {
            step = step < nsteps ? step : nsteps - 1;
            const uint32_t o = static_cast<uint32_t>(step >> 2) * 144u + static_cast<uint32_t>(step & 3) * 32u;
#pragma unroll
            for (int i = 0; i < UPT; i++) wqs[slot][i] = *reinterpret_cast<const uint2*>(w + (urow[i] + o + uq[i]));
        };
        auto dequant_store = [&](int c, int hslot, int slot, int buf) {
            uint4* dst = bt + buf * BUF;
#pragma unroll
            for (int i = 0; i < UPT; i++) {
                half2_t ds[2], nm[2];
                q4k_chunk_scales(hd[hslot][i], c, ds, nm);
                Frag lo, hi;
                q4k_bfrags_nat(wqs[slot][i].x, wqs[slot][i].y, ds, nm, lo, hi);
                dst[uslot[i]] = make_uint4(lo.u[0], lo.u[1], lo.u[2], lo.u[3]);
                dst[(NF + 1) * 64 + uslot[i]] = make_uint4(hi.u[0], hi.u[1], hi.u[2], hi.u[3]);
            }
        };
        // X tile pieces q = ptid + PT i (i < 8): row q / 8 = ptid / 8 + 32 i,
        // 16-byte piece q % 8; rows past M read zeros (the resource ends at
        // row M).  Ring layout: 128-byte rows, pieces XOR-swizzled by
        // (row / 2) % 8 = (ptid / 16) % 8 for every i.
        const int xrows = M - mt0 < TM ? M - mt0 : TM;
        const __amdgpu_buffer_rsrc_t xrs =
            make_rsrc(X + static_cast<uint32_t>(mt0) * static_cast<uint32_t>(K) * 2u,
                      static_cast<uint32_t>(xrows) * static_cast<uint32_t>(K) * 2u);
        const int xp = ptid & 7;
        const uint32_t xv = (static_cast<uint32_t>(ptid >> 3) * static_cast<uint32_t>(K) + 8u * static_cast<uint32_t>(xp)) * 2u;
        const int xst = (ptid >> 3) * 128 + 16 * (xp ^ ((ptid >> 4) & 7));
        u32x4 xr[2][8];
        auto load_x = [&](int step, int slot) {
            step = step < nsteps ? step : nsteps - 1;
            const uint32_t ko = static_cast<uint32_t>(step) * 128u;
#pragma unroll
            for (int i = 0; i < 8; i++)
                xr[slot][i] = buf_ld128(xrs, xv, ko + static_cast<uint32_t>(i) * 64u * static_cast<uint32_t>(K));
        };
        auto store_x = [&](int slot, int buf) {
            uint8_t* xs = reinterpret_cast<uint8_t*>(xring) + buf * XBUF;
#pragma unroll
            for (int i = 0; i < 8; i++) *reinterpret_cast<u32x4*>(xs + xst + i * 32 * 128) = xr[slot][i];
        };
        load_x(0, 0);
        load_x(1, 1);
        load_hd(0, 0);
        load_hd(1, 1);
#pragma unroll
        for (int r = 0; r < PD; r++) load_qs(r, r);
        store_x(0, 0);
        load_x(2, 0);
        store_x(1, 1);
        load_x(3, 1);
        dequant_store(0, 0, 0, 0);
        load_qs(PD, 0);
        dequant_store(1, 0, 1, 1);
        load_qs(PD + 1, 1);
        __syncthreads();
        int bw = 2;  // ring buffer of step s + 2
        for (int s0 = 0; s0 < nsteps; s0 += 8) {
            // steps s0 + r dequantize step s0 + r + 2 (chunk (r + 2) % 4) of
            // super-block s0 / 4 + (r + 2) / 4; s0 / 4 is even, so its header
            // sits in slot (r + 2) / 4 % 2.  Slot 0 is free after r = 1 and
            // takes super-block s0 / 4 + 2, slot 1 after r = 5 and takes
            // s0 / 4 + 3.
#pragma unroll
            for (int r = 0; r < 8; r++) {
                if (r == 4 && s0 + 4 >= nsteps) break;  // K = 256 (mod 512): half a round
                const int step = s0 + r;
                // past the last step the (clamped) loads repeat it and the
                // buffers written are never read.  The fences keep each
                // step's dequant in its step: hoisted together, the steps'
                // dequant would wait for all the prefetched loads.
                __builtin_amdgcn_sched_barrier(0);
                store_x(r & 1, bw);  // X of step + 2 sits in register slot (step + 2) % 2 = r % 2
                load_x(step + 4, r & 1);
                dequant_store((r + 2) & 3, ((r + 2) >> 2) & 1, (r + 2) % PD, bw);
                load_qs(step + 2 + PD, (r + 2) % PD);
                if (r == 2) load_hd((s0 >> 2) + 2, 0);
                if (r == 6) load_hd((s0 >> 2) + 3, 1);
                __builtin_amdgcn_sched_barrier(0);
                __syncthreads();
                bw = bw == 2 ? 0 : bw + 1;
            }
        }
    }
}

}  // namespace

// Caller (gemm_dispatch) has validated type (Q4_K), alignment (W, X 16 B)
// and the 32-bit offset bounds (N * row bytes, M * K * 2 < 2^32).
int gemm_q4k_split(const void* w, const void* X, float* Y, int64_t M, int64_t N, int64_t K, hipStream_t st) {
    constexpr int NF = 7;
    const int64_t rb = row_bytes(TYPE_Q4_K, K);
    const dim3 grid(static_cast<uint32_t>((N + 16 * NF - 1) / (16 * NF)), static_cast<uint32_t>((M + TM - 1) / TM));
    gemm_q4k_split_kernel<NF><<<grid, dim3(NTHR), 0, st>>>(static_cast<const uint8_t*>(w),
                                                           static_cast<const uint8_t*>(X), Y, static_cast<int>(M),
                                                           static_cast<int>(N), static_cast<int>(K), rb);
    return check_launch("vb_gemm");
}

}  // namespace vb
