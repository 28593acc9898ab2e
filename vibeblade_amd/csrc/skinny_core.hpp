// Skinny Q4_K x activations tile on MFMA (16 activation rows per tile, MT
// tiles), shared by the M <= 32 GEMM (gemm_skinny.hip) and the MoE expert
// kernels (moe.hip).
//
// A workgroup of 8 waves computes, for `rows` (<= 64) consecutive weight rows
// of NMAT matrices with the same shape (MoE gate and up: NMAT = 2), the dot
// products with up to 16 activation rows over all of K.  The waves split K
// into contiguous super-block ranges, so every activation fragment a wave
// loads is reused by the four 16-row column groups.
//
// Weight loads.  A wave "unit" is one super-block of one matrix for the
// workgroup's rows: rows x 144 bytes read as row-contiguous 16-byte pieces
// (piece p = 64 i + lane, 9 per lane) with buffer loads (wave-uniform
// resource, 32-bit lane offsets), written to a private LDS area in the same
// order (rows 144 bytes apart) and read back in the MFMA B layout.  Loading
// the B layout straight from HBM would touch 16 rows per load instruction,
// which streams at about two thirds of the row-contiguous rate.  Units run
// two ahead in a ring of two register buffers.
//
// MFMA mapping (v_mfma_f32_16x16x32_f16, mfma_q4k.hpp).  Column j = weight
// row 16 q + j, A row i = activation row i.  Lane group g always works on
// chunk g of the super-block (sub-blocks 2g, 2g+1: 32 qs bytes): MFMA step
// s = 0..3 takes the low nibbles of bytes 8 s .. 8 s + 7 (elements
// 64 g + 8 s + ..), steps 4..7 the high nibbles of the same bytes (elements
// 64 g + 32 + ..).  The k order inside an MFMA is free as long as A and B
// agree, and with the weight scales folded into B (w = d sc q - dmin m,
// rounded once to fp16) the four lane groups may sit in different sub-blocks:
// each lane decodes only its own two 6-bit scale / min pairs per super-block.
//
// Partial sums of the 8 k-ranges meet in LDS and are added in a fixed order.
#pragma once

#include <type_traits>

#include "mfma_q4k.hpp"

namespace vb {
namespace skinny {

constexpr int WAVES = 8;                   // default waves per workgroup
constexpr int ROWS = 64;                   // max rows per workgroup: 4 column groups
constexpr int PPL = ROWS * 9 / 64;         // 16-byte pieces per lane per unit: 9
constexpr int STAGE = ROWS * 144 + 16;     // per-wave LDS bytes (+ one discard slot)
// Dynamic LDS of a launch with NW waves: the staging areas, which the final
// sums (NMAT x NW x 4 KiB, NMAT <= 2) reuse.
template <int NW = WAVES>
constexpr int lds_bytes() { return NW * STAGE; }
// With MT activation tiles of NMAT matrices the final sums take MT NMAT 4 KB
// per wave, which passes the staging areas from MT NMAT = 3 on.
template <int NW, int MT, int NMAT>
constexpr int lds_bytes_mt() {
    return NW * STAGE > MT * NMAT * NW * 4096 ? NW * STAGE : MT * NMAT * NW * 4096;
}
constexpr int LDS_BYTES = lds_bytes<WAVES>();
constexpr int X_F32 = 0;
constexpr int X_F16 = 1;
constexpr uint32_t X_NONE = 0x80000000u;   // lane offset of an absent activation row (reads zeros)

// buffer-load helpers shared with the GEMV (vb_common.hpp)
using vb::u32x4;
using vb::make_rsrc;
using vb::buf_ld128;

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

// Raw activation words of one super-block for one lane: 8 fragments of 8
// elements (fp16: one 16-byte word each; fp32: two).
template <int XT> struct XWords;
template <> struct XWords<X_F16> { u32x4 v[8]; };
template <> struct XWords<X_F32> { u32x4 v[16]; };

// xoff = the lane's byte offset (activation row + 64 g elements), soff = the
// super-block's first element in bytes.
template <int XT>
__device__ __forceinline__ void load_xwords(__amdgpu_buffer_rsrc_t xr, uint32_t xoff, uint32_t soff, XWords<XT>& xw) {
    constexpr uint32_t ES = XT == X_F16 ? 2u : 4u;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const uint32_t k = 32u * (s >> 2) + 8u * (s & 3);
        if constexpr (XT == X_F16) {
            xw.v[s] = buf_ld128(xr, xoff + ES * k, soff);
        } else {
            xw.v[2 * s] = buf_ld128(xr, xoff + ES * k, soff);
            xw.v[2 * s + 1] = buf_ld128(xr, xoff + ES * k + 16u, soff);
        }
    }
}

// A fragments in natural k order (q4k_bfrags_cvt): fp16 words are used as
// loaded, fp32 ones rounded to fp16.
template <int XT>
__device__ __forceinline__ void xwords_to_frags(const XWords<XT>& xw, Frag* a) {
#pragma unroll
    for (int s = 0; s < 8; s++) {
        if constexpr (XT == X_F16) {
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

template <int NMAT, int MT = 1>
struct TileArgs {
    __amdgpu_buffer_rsrc_t w[NMAT];  // the weight matrices (same shape)
    __amdgpu_buffer_rsrc_t x;        // activations
    uint32_t xoff[MT];               // per 16-row activation tile: this lane's row offset in bytes
                                     // (+ 64 g elements), or X_NONE
    int row0, rows, nrows;           // rows [row0, row0 + rows) of nrows
    int rb, nsb;                     // bytes per weight row, super-blocks per row
};

// Runs the tile with NW waves and returns, in threads 0..255 (q = tid / 64,
// l = tid % 64), the sums of weight row row0 + 16 q + l % 16 with activation
// rows 4 (l / 16) + 0..3 of every matrix and activation tile: out[mt * NMAT
// + m].  MT activation tiles (16 rows each) share every dequantized weight
// fragment.  All threads of the workgroup must call it (it synchronises);
// `lds` = the launch's dynamic LDS (lds_bytes<NW>()).
// PAIRS (fp16 X, one activation tile, a ring of two): super-blocks are taken
// in pairs t, t + 1 (t even) and the pairs dealt round-robin over the waves
// (pair p of wave w: t = 2 (NW p + w)); a wave issues the units of one
// matrix for both super-blocks of its pair back to back (g(t), g(t + 1),
// then u(t), u(t + 1) with two matrices g, u).  A 144-byte super-block slice
// of a row always straddles two 128-byte lines; this way the two slices
// sharing a line are requested together (same wave, or neighbouring waves
// in the same period), and a period of the workgroup spans 2 NW super-blocks
// = 9 NW lines of every row, so no line is shared across periods.  Without
// it a line shared by units issued a period apart is fetched twice (the
// MoE expert kernels read 1.3-1.6x their weight bytes).  The wave keeps no
// weight load in flight while it computes; its workgroup and the other
// workgroup on the CU cover that time.
template <int XT, int NMAT, int RING = 2, int NW = WAVES, int MT = 1, bool PAIRS = false>
__device__ __forceinline__ void tile(const TileArgs<NMAT, MT>& ta, uint8_t* lds, float4_t* out) {
    // the launch gives the workgroup lds_bytes_mt<NW, MT, NMAT>() bytes: the
    // staging areas, or the final sums where those need more
    static_assert(!PAIRS || (RING == 2 && XT == X_F16 && MT == 1), "paired units: a ring of two, fp16 X, one token tile");
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int nsb = ta.nsb;
    const int sb0 = __builtin_amdgcn_readfirstlane((wave * nsb) / NW);
    const int sb1 = __builtin_amdgcn_readfirstlane(((wave + 1) * nsb) / NW);
    const int nsbw = sb1 - sb0;             // the wave's super-blocks (0 when nsb < NW for some waves)
    const int nunits = nsbw * NMAT;
    // PAIRS: periods (one pair per wave); the wave's idx-th super-block
    const int nper = (nsb + 2 * NW - 1) / (2 * NW);
    auto sb_of = [&](int idx) __attribute__((always_inline)) -> int {
        return 2 * (NW * (idx >> 1) + wave) + (idx & 1);
    };
    uint8_t* stage = lds + wave * STAGE;

    // Pieces of this lane: p = 64 i + lane -> row p / 9, word p % 9 of the
    // unit's rows x 144-byte block; pieces past the block reload the last
    // one and land in the discard slot.
    const int npieces = ta.rows * 9;
    uint32_t poff[PPL], soff[PPL];
#pragma unroll
    for (int i = 0; i < PPL; i++) {
        const int p = 64 * i + lane;
        const int pc = p < npieces ? p : npieces - 1;
        const int r = pc / 9, wd = pc - 9 * r;
        int row = ta.row0 + r;
        row = row < ta.nrows ? row : ta.nrows - 1;
        poff[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(ta.rb) + 16u * static_cast<uint32_t>(wd);
        soff[i] = p < npieces ? 16u * static_cast<uint32_t>(p) : static_cast<uint32_t>(ROWS * 144);
    }
    constexpr uint32_t ES = XT == X_F16 ? 2u : 4u;
    const LaneScaleSel sel = lane_scale_sel(g);

    // Weight units run two ahead (ring of two register buffers); the
    // activations (L2-resident) one super-block ahead: gfx9 loads retire in
    // order, so the activations of super-block b + 1 are issued before the
    // weights of its first unit.  fp16 activations feed the MFMAs as loaded
    // and need a buffer per super-block parity; fp32 ones are converted when
    // their super-block starts, after which their buffer is free again.
    constexpr int XB = XT == X_F16 ? 2 : 1;
    constexpr int P = 2 * NMAT;  // units per unrolled period (ring slot and buffer parities repeat)
    u32x4 pv[RING][PPL];
    XWords<XT> xw[MT][XB];
    Frag a[MT][XT == X_F32 ? 8 : 1];  // converted fp32 activations of the current super-block
    int itw = 0, itx = 0;
    // Ring slots are compile-time constants so the buffers stay in registers.
    auto issue_w = [&](auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value;  // ring slot
        int sb = sb0 + itw / NMAT;
        sb = sb < nsb - 1 ? sb : nsb - 1;  // padding units reload the last super-block
        if constexpr (NMAT == 1 || RING == 2) {
            // NMAT = 2 with a ring of two: the slot is the unit parity, i.e. the matrix
#pragma unroll
            for (int i = 0; i < PPL; i++)
                pv[slot][i] = buf_ld128(ta.w[slot % NMAT], poff[i], static_cast<uint32_t>(sb) * 144u);
        } else {
            // one slot for both matrices: pick the resource by the unit's parity
            const __amdgpu_buffer_rsrc_t r = (itw & 1) ? ta.w[NMAT - 1] : ta.w[0];
#pragma unroll
            for (int i = 0; i < PPL; i++) pv[slot][i] = buf_ld128(r, poff[i], static_cast<uint32_t>(sb) * 144u);
        }
        ++itw;
    };
    // PAIRS: unit itw of period p = itw / (2 NMAT) is matrix mat (a constant
    // of the caller) over the wave's super-block 2 p + slot
    auto issue_wp = [&](auto slot_c, auto mat_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value, mat = decltype(mat_c)::value;
        int sb = sb_of(2 * (itw / (2 * NMAT)) + slot);
        sb = sb < nsb - 1 ? sb : nsb - 1;  // padding units reload the last super-block
#pragma unroll
        for (int i = 0; i < PPL; i++)
            pv[slot][i] = buf_ld128(ta.w[mat], poff[i], static_cast<uint32_t>(sb) * 144u);
        ++itw;
    };
    auto issue_x = [&](auto buf_c) __attribute__((always_inline)) {
        constexpr int buf = decltype(buf_c)::value % XB;
        int sb = PAIRS ? sb_of(itx) : sb0 + itx;
        sb = sb < nsb - 1 ? sb : nsb - 1;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            load_xwords<XT>(ta.x, ta.xoff[mt], static_cast<uint32_t>(sb) * 256u * ES, xw[mt][buf]);
        ++itx;
    };

    float4_t acc[MT][NMAT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int q = 0; q < 4; q++) acc[mt][m][q] = float4_t{0.f, 0.f, 0.f, 0.f};
    int ct = 0;
    auto compute = [&](auto u_c) __attribute__((always_inline)) {
        constexpr int u = decltype(u_c)::value;  // position in the period
        constexpr int slot = RING == 1 ? 0 : u % 2;
        constexpr int m = PAIRS ? u / 2 : u % NMAT, xb = PAIRS ? u % 2 : (u / NMAT) % 2;
        if constexpr (PAIRS) {
            // padding units (uniform): super-blocks past the end, in the
            // last period of some waves
            const bool pad = sb_of(2 * (ct / (2 * NMAT)) + (u & 1)) >= nsb;
            if (pad) {
                ++ct;
                return;
            }
        } else if (ct >= nunits) {
            return;  // padding unit (uniform)
        }
        if constexpr (m == 0 && !PAIRS) {
            if constexpr (XT == X_F32) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++) xwords_to_frags<XT>(xw[mt][0], a[mt]);
            }
            issue_x(std::integral_constant<int, xb ^ 1>{});  // next super-block's activations
        }
        // fp16 activations are read in place: no copy lives across units
        auto afrag = [&](int mt, int s) __attribute__((always_inline)) -> Frag {
            if constexpr (XT == X_F16) {
                Frag f;
                const u32x4 v = xw[mt][xb % XB].v[s];
                f.u[0] = v.x;
                f.u[1] = v.y;
                f.u[2] = v.z;
                f.u[3] = v.w;
                return f;
            } else {
                return a[mt][s];
            }
        };
#pragma unroll
        for (int i = 0; i < PPL; i++) *reinterpret_cast<u32x4*>(stage + soff[i]) = pv[slot][i];
        if constexpr (RING == 1) {
            // the unit is in LDS: its registers take the next unit now
            if (ct + 1 < nunits) issue_w(std::integral_constant<int, 0>{});
        }
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
                q4k_bfrags_cvt(qd[2 * s], qd[2 * s + 1], ds, nm, lo, hi);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    acc[mt][m][q] = mfma16x16x32(afrag(mt, s), lo, acc[mt][m][q]);
                    acc[mt][m][q] = mfma16x16x32(afrag(mt, 4 + s), hi, acc[mt][m][q]);
                }
            }
        }
        ++ct;
    };

    // Prologue: units 0, 1 and super-block 0's activations.  Each period
    // computes P units and refills the ring two units ahead; the last period
    // issues nothing past the end.
    const int nunits_p = nunits <= P ? P : ((nunits + P - 1) / P) * P;
    if constexpr (PAIRS) {
        // Period: the activations of t, t + 1 and the first matrix's units
        // of t, t + 1 are in flight; those units are computed, the second
        // matrix's units issued and computed, then the next period's loads
        // issued.
        issue_x(std::integral_constant<int, 0>{});
        issue_x(std::integral_constant<int, 1>{});
        issue_wp(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
        issue_wp(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
        for (int pp = 0; pp < nper; pp++) {
            compute(std::integral_constant<int, 0>{});
            compute(std::integral_constant<int, 1>{});
            if constexpr (NMAT == 2) {
                issue_wp(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
                issue_wp(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
                compute(std::integral_constant<int, 2>{});
                compute(std::integral_constant<int, 3>{});
            }
            if (pp + 1 < nper) {
                issue_x(std::integral_constant<int, 0>{});
                issue_x(std::integral_constant<int, 1>{});
                issue_wp(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
                issue_wp(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
            }
        }
    } else if constexpr (RING == 1) {
        // one unit in flight per wave, refilled as soon as it is staged
        issue_w(std::integral_constant<int, 0>{});
        issue_x(std::integral_constant<int, 0>{});
        for (int u0 = 0; u0 < nunits_p; u0 += P) {
            compute(std::integral_constant<int, 0>{});
            compute(std::integral_constant<int, 1>{});
            if constexpr (NMAT == 2) {
                compute(std::integral_constant<int, 2>{});
                compute(std::integral_constant<int, 3>{});
            }
        }
    } else {
    issue_w(std::integral_constant<int, 0>{});
    issue_x(std::integral_constant<int, 0>{});
    issue_w(std::integral_constant<int, 1>{});
    for (int u0 = 0; u0 + P < nunits_p; u0 += P) {
        compute(std::integral_constant<int, 0>{});
        issue_w(std::integral_constant<int, 0>{});
        compute(std::integral_constant<int, 1>{});
        issue_w(std::integral_constant<int, 1>{});
        if constexpr (NMAT == 2) {
            compute(std::integral_constant<int, 2>{});
            issue_w(std::integral_constant<int, 0>{});
            compute(std::integral_constant<int, 3>{});
            issue_w(std::integral_constant<int, 1>{});
        }
    }
    if constexpr (NMAT == 2) {
        compute(std::integral_constant<int, 0>{});
        issue_w(std::integral_constant<int, 0>{});
        compute(std::integral_constant<int, 1>{});
        issue_w(std::integral_constant<int, 1>{});
        compute(std::integral_constant<int, 2>{});
        compute(std::integral_constant<int, 3>{});
    } else {
        compute(std::integral_constant<int, 0>{});
        compute(std::integral_constant<int, 1>{});
    }
    }

    // k-range partials meet in LDS (over the staging areas), fixed order.
    __syncthreads();
    float4_t* red = reinterpret_cast<float4_t*>(lds);  // [mt * NMAT + m][wave][q][lane]
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                red[(((mt * NMAT + m) * NW + wave) * 4 + q) * 64 + lane] = acc[mt][m][q];
    __syncthreads();
    if (threadIdx.x < 256) {
        const int e = threadIdx.x;
#pragma unroll
        for (int mm = 0; mm < MT * NMAT; mm++) {
            float4_t s = red[(mm * NW * 4) * 64 + e];
#pragma unroll
            for (int v = 1; v < NW; v++) s += red[((mm * NW + v) * 4) * 64 + e];
            out[mm] = s;
        }
    }
    __syncthreads();  // the next tile may overwrite the sums
}

}  // namespace skinny
}  // namespace vb
