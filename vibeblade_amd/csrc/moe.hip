// MoE expert-grouped FFN: route, group tokens per expert, SwiGLU experts,
// weighted combine.
//
// Reference semantics: per token, softmax over the router logits (clamped to
// +-50), top-k, renormalise the k weights (vibeblade/moe.py:184-206,
// cpp/src/fast_model.cpp:534-548), expert FFN down(silu(gate x) * up x)
// (vibeblade/moe_executor.py:331-344, cpp/src/fast_model.cpp:552-572), and
// y_t = sum_k w_tk * FFN_(e_tk)(x_t) (vibeblade/moe.py:457-482).  The
// reference's HotColdExecutor.dispatch routes only the first token of a batch
// (vibeblade/moe_executor.py:210-212); this routes every token.
//
// Four launches, no host round trip:
//   1. prep: routes every token once (routing written for the combine and the
//      caller), lists the slots (token * topk + k) of each expert in slot
//      order, and rounds x to fp16.
//   2. gate/up.  Q4_K experts: grid (i/64, E), skinny tiles (skinny_core.hpp)
//      of 64 gate and 64 up rows per 16 slots, silu(g) * u written as fp16
//      into hbuf.  F32 experts: grid (i/16, E), 16-row tiles on
//      v_mfma_f32_16x16x32_f16, hbuf in fp32.
//   3. down: activations = hbuf rows of the expert's slots, writes the expert
//      output of every slot into obuf.
//   4. combine: y_t = sum_k w_tk * obuf[t*topk + k] in slot order (fixed
//      order, deterministic); also copies the routing to (indices, weights).
// Each expert's weights are streamed once per 16 routed slots.
#include "mfma_q4k.hpp"
#include "skinny_core.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int MOE_MAX_EXPERTS = 64;
constexpr int MOE_MAX_TOPK = 8;
constexpr int MOE_MAX_SLOTS = 1024;  // tokens * topk

struct ExpertPtrs {
    const uint8_t* p[MOE_MAX_EXPERTS];
};

// Butterfly exchanges over a wave without LDS: quad xor 1 and 2, half-row
// and row mirrors (DPP), then the 16- and 32-lane halves swapped
// (v_permlane16 / v_permlane32_swap).  Each step pairs lanes symmetrically,
// so a commutative combine leaves every lane with the same bits.
template <typename C>
__device__ __forceinline__ float wave_allreduce_f(float v, C comb) {
    v = comb(v, dpp_f<0xB1>(v));
    v = comb(v, dpp_f<0x4E>(v));
    v = comb(v, dpp_f<0x141>(v));
    v = comb(v, dpp_f<0x140>(v));
    const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = comb(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return comb(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// (p, id) of the lane that ranks first by (p desc, id asc), a total order,
// on every lane
__device__ __forceinline__ void wave_argmax(float& bp, int& bi) {
    auto take = [&](float op, int oi) {
        if (op > bp || (op == bp && oi < bi)) {
            bp = op;
            bi = oi;
        }
    };
    take(dpp_f<0xB1>(bp), dpp_i<0xB1>(bi));
    take(dpp_f<0x4E>(bp), dpp_i<0x4E>(bi));
    take(dpp_f<0x141>(bp), dpp_i<0x141>(bi));
    take(dpp_f<0x140>(bp), dpp_i<0x140>(bi));
    {
        const auto sp = __builtin_amdgcn_permlane16_swap(__float_as_uint(bp), __float_as_uint(bp), false, false);
        const auto si = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(bi), static_cast<uint32_t>(bi), false,
                                                         false);
        bp = __uint_as_float(sp[0]);
        bi = static_cast<int>(si[0]);
        take(__uint_as_float(sp[1]), static_cast<int>(si[1]));
    }
    {
        const auto sp = __builtin_amdgcn_permlane32_swap(__float_as_uint(bp), __float_as_uint(bp), false, false);
        const auto si = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(bi), static_cast<uint32_t>(bi), false,
                                                         false);
        bp = __uint_as_float(sp[0]);
        bi = static_cast<int>(si[0]);
        take(__uint_as_float(sp[1]), static_cast<int>(si[1]));
    }
}

// Route one token with one wave, lane e = expert e (e_n <= 64): top-k of
// softmax(clamp(logits, -50, 50)), renormalised; ties go to the lower expert
// id.  Max and sum are butterflies (every lane ends with the same bits:
// each step adds the same two values, a + b == b + a); the top k come out
// one per round of a butterfly argmax over (p desc, id asc), a total order,
// so every lane agrees on the winner.  Lanes k < topk write slot k.
// The weight sum runs in rank order.
__device__ __forceinline__ void route_token_wave(const float* __restrict__ logits, int e_n, int topk,
                                                 int32_t* __restrict__ out_idx, float* __restrict__ out_w,
                                                 int* __restrict__ sexp, int32_t* __restrict__ copy_idx = nullptr,
                                                 float* __restrict__ copy_w = nullptr) {
    const int lane = threadIdx.x & 63;
    const bool live = lane < e_n;
    float z = logits[live ? lane : e_n - 1];  // clamped index: the load stays outside any branch
    z = live ? fminf(fmaxf(z, -50.f), 50.f) : -INFINITY;
    const float mx = wave_allreduce_f(z, [](float a, float b) { return fmaxf(a, b); });
    const float ex = live ? __expf(z - mx) : 0.f;
    const float den = wave_allreduce_f(ex, [](float a, float b) { return a + b; });
    float p = live ? ex / den : -1.f;  // absent experts rank below every live one
    float s = 0.f, myw = 0.f;
    int myi = -1;
    for (int k = 0; k < topk; k++) {
        float bp = p;
        int bi = lane;
        wave_argmax(bp, bi);
        s += bp;
        if (lane == k) {
            myw = bp;
            myi = bi;
        }
        if (lane == bi) p = -2.f;  // taken
    }
    s = s < 1e-12f ? 1.f : s;
    if (lane < topk) {
        const float wn = myw / s;
        out_idx[lane] = myi;
        out_w[lane] = wn;
        if (sexp) sexp[lane] = myi;
        if (copy_idx) copy_idx[lane] = myi;  // the caller's routing outputs, from registers
        if (copy_w) copy_w[lane] = wn;
    }
}

// One 16-row tile of F32 expert weights times the gathered fp32 activation
// rows arow[0..nrow) (nrow <= 16), k split over the 4 waves.  NMAT = 1 or 2
// matrices over the same activations.  Returns the per-lane D fragments of
// the full-k sums in red (LDS, [4 waves][64 lanes] per matrix).
template <int NMAT, int WT>
__device__ void tile_mfma(const uint8_t* const* wrow, const float* const* arow, int nrow, int64_t k,
                          float4_t (*red)[4][64]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int nsb = static_cast<int>(k / 256);
    const int sb0 = (wave * nsb) / 4, sb1 = ((wave + 1) * nsb) / 4;
    const bool avalid = j < nrow;
    const float* ap = avalid ? arow[j] : arow[0];
    float4_t acc[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) acc[m] = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int sb = sb0; sb < sb1; sb++) {
        Frag a[8];
#pragma unroll
        for (int sub = 0; sub < 8; sub++) {
            const float* p = ap + static_cast<int64_t>(sb) * 256 + 32 * sub + 8 * g;
            const float4 lo4 = *reinterpret_cast<const float4*>(p);
            const float4 hi4 = *reinterpret_cast<const float4*>(p + 4);
            f32x8_to_frag(avalid ? lo4 : make_float4(0.f, 0.f, 0.f, 0.f),
                          avalid ? hi4 : make_float4(0.f, 0.f, 0.f, 0.f), a[sub].u);
        }
        {  // F32 weights: row n, k = 256 sb + 32 sub + 8 g .. +8, rounded to fp16
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const float* wp = reinterpret_cast<const float*>(wrow[m]) + static_cast<int64_t>(sb) * 256 + 8 * g;
#pragma unroll
                for (int sub = 0; sub < 8; sub++) {
                    Frag b;
                    f32x8_to_frag(*reinterpret_cast<const float4*>(wp + 32 * sub),
                                  *reinterpret_cast<const float4*>(wp + 32 * sub + 4), b.u);
                    acc[m] = mfma16x16x32(a[sub], b, acc[m]);
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++) red[m][wave][lane] = acc[m];
    __syncthreads();
}

template <int WT>
__global__ void __launch_bounds__(256) moe_gate_up_kernel(ExpertPtrs wg, ExpertPtrs wu, const float* __restrict__ x,
                                                          const int32_t* __restrict__ eoff,
                                                          const int32_t* __restrict__ elist, int nslots, int topk,
                                                          int64_t h, int64_t i_dim, int64_t rb,
                                                          float* __restrict__ hbuf) {
    __shared__ float4_t red[2][4][64];
    const int e = blockIdx.y;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    const SlotRange slots = expert_slots(eoff, elist, e, nslots);
    const int cnt = slots.count;
    if (cnt <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    int64_t n = n0 + j;
    n = n < i_dim ? n : i_dim - 1;
    const uint8_t* wrow[2] = {wg.p[e] + n * rb, wu.p[e] + n * rb};
    for (int m0 = 0; m0 < cnt; m0 += 16) {
        const int nrow = cnt - m0 < 16 ? cnt - m0 : 16;
        const float* arow[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int s = slots[m0 + (r < nrow ? r : 0)];
            arow[r] = x + static_cast<int64_t>(s / topk) * h;
        }
        tile_mfma<2, WT>(wrow, arow, nrow, h, red);
        if (wave == 0) {
            const float4_t gs = (red[0][0][lane] + red[0][1][lane]) + (red[0][2][lane] + red[0][3][lane]);
            const float4_t us = (red[1][0][lane] + red[1][1][lane]) + (red[1][2][lane] + red[1][3][lane]);
            const int64_t col = n0 + j;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * g + r;
                if (row < nrow && col < i_dim) {
                    const float gv = gs[r];
                    hbuf[static_cast<int64_t>(slots[m0 + row]) * i_dim + col] = gv / (1.0f + __expf(-gv)) * us[r];
                }
            }
        }
        __syncthreads();
    }
}

template <int WT>
__global__ void __launch_bounds__(256) moe_down_kernel(ExpertPtrs wd, const float* __restrict__ hbuf,
                                                       const int32_t* __restrict__ eoff,
                                                       const int32_t* __restrict__ elist, int nslots, int64_t h,
                                                       int64_t i_dim, int64_t rb, float* __restrict__ obuf) {
    __shared__ float4_t red[1][4][64];
    const int e = blockIdx.y;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    const SlotRange slots = expert_slots(eoff, elist, e, nslots);
    const int cnt = slots.count;
    if (cnt <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    int64_t n = n0 + j;
    n = n < h ? n : h - 1;
    const uint8_t* wrow[1] = {wd.p[e] + n * rb};
    for (int m0 = 0; m0 < cnt; m0 += 16) {
        const int nrow = cnt - m0 < 16 ? cnt - m0 : 16;
        const float* arow[16];
#pragma unroll
        for (int r = 0; r < 16; r++) arow[r] = hbuf + static_cast<int64_t>(slots[m0 + (r < nrow ? r : 0)]) * i_dim;
        tile_mfma<1, WT>(wrow, arow, nrow, i_dim, red);
        if (wave == 0) {
            const float4_t s = (red[0][0][lane] + red[0][1][lane]) + (red[0][2][lane] + red[0][3][lane]);
            const int64_t col = n0 + j;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * g + r;
                if (row < nrow && col < h) obuf[static_cast<int64_t>(slots[m0 + row]) * h + col] = s[r];
            }
        }
        __syncthreads();
    }
}

// ---- Q4_K experts: skinny tiles (skinny_core.hpp) --------------------------
//
// prep: block 0 routes every token once and writes the routing (ridx, rw)
// and the slots of each expert in slot order (elist[eoff[e] .. eoff[e+1]));
// the other blocks round x to fp16 (xh) -- the MFMA path rounds its
// activations to fp16 anyway, and fp16 halves the activation traffic of the
// expert kernels.
constexpr int PREP_THREADS = 1024;

__global__ void __launch_bounds__(PREP_THREADS) moe_prep_kernel(
        const float* __restrict__ x, const float* __restrict__ logits, int t_n, int e_n, int topk, int64_t nx,
        _Float16* __restrict__ xh, int32_t* __restrict__ ridx, float* __restrict__ rw, int32_t* __restrict__ eoff,
        int32_t* __restrict__ elist, float* __restrict__ yzero, int32_t* __restrict__ out_idx,
        float* __restrict__ out_w) {
    if (blockIdx.x > 0) {
        const int64_t i8 = (static_cast<int64_t>(blockIdx.x - 1) * PREP_THREADS + threadIdx.x) * 8;
        if (i8 < nx) {  // nx = t_n * h, a multiple of 256
            const float4 a = *reinterpret_cast<const float4*>(x + i8);
            const float4 b = *reinterpret_cast<const float4*>(x + i8 + 4);
            uint32_t o[4];
            f32x8_to_frag_nat(a, b, o);
            *reinterpret_cast<uint4*>(xh + i8) = make_uint4(o[0], o[1], o[2], o[3]);
            if (yzero) {  // y has x's shape; the down kernels add into it
                *reinterpret_cast<float4*>(yzero + i8) = make_float4(0.f, 0.f, 0.f, 0.f);
                *reinterpret_cast<float4*>(yzero + i8 + 4) = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        return;
    }
    __shared__ int sexp[MOE_MAX_SLOTS];
    __shared__ int scnt[MOE_MAX_EXPERTS + 1];
    const int nslots = t_n * topk;
    // one wave per token
    // with yzero no combine launch follows, and the routing result goes to
    // out_idx / out_w here
    int32_t* const cidx = yzero ? out_idx : nullptr;
    float* const cw = yzero ? out_w : nullptr;
    for (int t = static_cast<int>(threadIdx.x >> 6); t < t_n; t += PREP_THREADS / 64)
        route_token_wave(logits + static_cast<int64_t>(t) * e_n, e_n, topk, ridx + t * topk, rw + t * topk,
                         sexp + t * topk, cidx ? cidx + t * topk : nullptr, cw ? cw + t * topk : nullptr);
    __syncthreads();
    if (nslots <= 64) {
        // one wave: expert e's slots are the lanes whose expert is e; a
        // ballot per expert gives its count, the running total its offset,
        // and the lanes below a slot with the same expert its position
        // (slot order, as the loops below)
        if (threadIdx.x < 64) {
            const int q = static_cast<int>(threadIdx.x);
            const int eq = q < nslots ? sexp[q] : -1;
            const uint64_t below = (uint64_t(1) << q) - 1u;
            int total = 0, my_off = 0, my_pos = -1;
            for (int e = 0; e < e_n; e++) {
                const uint64_t m = __ballot(eq == e);
                if (q == e) my_off = total;
                if (eq == e) my_pos = total + __popcll(m & below);
                total += __popcll(m);
            }
            if (q < e_n) eoff[q] = my_off;
            if (q == 0) eoff[e_n] = total;
            if (my_pos >= 0) elist[my_pos] = q;
        }
        return;
    }
    // counts per expert, then exclusive offsets (slots with no expert -- NaN
    // logits -- are in no list)
    if (threadIdx.x < e_n) {
        int c = 0;
        for (int q = 0; q < nslots; q++) c += sexp[q] == static_cast<int>(threadIdx.x);
        scnt[threadIdx.x + 1] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        scnt[0] = 0;
        for (int e = 0; e < e_n; e++) scnt[e + 1] += scnt[e];
        for (int e = 0; e <= e_n; e++) eoff[e] = scnt[e];
    }
    __syncthreads();
    for (int q = threadIdx.x; q < nslots; q += PREP_THREADS) {
        const int e = sexp[q];
        if (e < 0 || e >= e_n) continue;
        int pos = 0;
        for (int r = 0; r < q; r++) pos += sexp[r] == e;
        elist[scnt[e] + pos] = q;
    }
}

// gate/up: grid (ceil(i / 64), E).  A workgroup streams 64 rows of the
// expert's gate and up matrices once per group of 16 routed slots (the tile
// takes super-blocks in interleaved pairs, the gate units of a pair then its
// up units, which share the activation fragments) and writes silu(g) * u for
// every (slot, row) into hbuf as fp16 -- the down kernel rounds its
// activations to fp16 anyway.
// Four-wave workgroups with at most 256 VGPRs, so two run on each CU: one's
// start-up and reduction overlap the other's weight stream.
constexpr int MOE_WAVES = 4;

template <int NW>
__global__ void __launch_bounds__(64 * NW, NW <= 4 ? 2 : 1) moe_gate_up_q4k(
        ExpertPtrs wg, ExpertPtrs wu, const _Float16* __restrict__ xh, const int32_t* __restrict__ eoff,
        const int32_t* __restrict__ elist, int nslots, int topk, int h, int i_dim, int rb, uint32_t wbytes,
        uint32_t xbytes, _Float16* __restrict__ hbuf) {
    extern __shared__ skinny::u32x4 moe_lds[];
    const int e = blockIdx.y;
    const SlotRange slots = expert_slots(eoff, elist, e, nslots);
    const int cnt = slots.count;
    if (cnt <= 0) return;
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    skinny::TileArgs<2> ta;
    ta.w[0] = skinny::make_rsrc(wg.p[e], wbytes);
    ta.w[1] = skinny::make_rsrc(wu.p[e], wbytes);
    ta.x = skinny::make_rsrc(xh, xbytes);
    ta.row0 = static_cast<int>(blockIdx.x) * skinny::ROWS;
    ta.rows = i_dim - ta.row0 < skinny::ROWS ? i_dim - ta.row0 : skinny::ROWS;
    ta.nrows = i_dim;
    ta.rb = rb;
    ta.nsb = h / 256;
    for (int m0 = 0; m0 < cnt; m0 += 16) {
        const int nrow = cnt - m0 < 16 ? cnt - m0 : 16;
        ta.xoff[0] = j < nrow ? (static_cast<uint32_t>(slots[m0 + j] / topk) * static_cast<uint32_t>(h) + 64u * g) * 2u
                           : skinny::X_NONE;
        float4_t s[2];
        skinny::tile<skinny::X_F16, 2, 2, NW, 1, true>(ta, reinterpret_cast<uint8_t*>(moe_lds), s);
        if (threadIdx.x < 256) {
            const int q = threadIdx.x >> 6, l = threadIdx.x & 63;
            const int r = 16 * q + (l & 15), n = ta.row0 + r;
            if (r < ta.rows) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int t = 4 * (l >> 4) + v;
                    if (t < nrow) {
                        const float gv = s[0][v], uv = s[1][v];
                        hbuf[static_cast<int64_t>(slots[m0 + t]) * i_dim + n] =
                                static_cast<_Float16>(gv / (1.0f + __expf(-gv)) * uv);
                    }
                }
            }
        }
    }
}

// down: grid (ceil(h / 64), E); activations = the fp16 hbuf rows of the
// expert's slots; writes the expert output of every slot into obuf.
template <int NW>
__global__ void __launch_bounds__(64 * NW, NW <= 4 ? 2 : 1) moe_down_q4k(
        ExpertPtrs wd, const _Float16* __restrict__ hbuf, const int32_t* __restrict__ eoff,
        const int32_t* __restrict__ elist, int nslots, int h, int i_dim, int rb, uint32_t wbytes, uint32_t hbytes,
        float* __restrict__ obuf, const float* __restrict__ rw, int topk, float* __restrict__ yacc) {
    extern __shared__ skinny::u32x4 moe_lds[];
    const int e = blockIdx.y;
    const SlotRange slots = expert_slots(eoff, elist, e, nslots);
    const int cnt = slots.count;
    if (cnt <= 0) return;
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    skinny::TileArgs<1> ta;
    ta.w[0] = skinny::make_rsrc(wd.p[e], wbytes);
    ta.x = skinny::make_rsrc(hbuf, hbytes);
    ta.row0 = static_cast<int>(blockIdx.x) * skinny::ROWS;
    ta.rows = h - ta.row0 < skinny::ROWS ? h - ta.row0 : skinny::ROWS;
    ta.nrows = h;
    ta.rb = rb;
    ta.nsb = i_dim / 256;
    for (int m0 = 0; m0 < cnt; m0 += 16) {
        const int nrow = cnt - m0 < 16 ? cnt - m0 : 16;
        ta.xoff[0] = j < nrow ? (static_cast<uint32_t>(slots[m0 + j]) * static_cast<uint32_t>(i_dim) + 64u * g) * 2u
                           : skinny::X_NONE;
        float4_t s[1];
        skinny::tile<skinny::X_F16, 1, 2, NW, 1, true>(ta, reinterpret_cast<uint8_t*>(moe_lds), s);
        if (threadIdx.x < 256) {
            const int q = threadIdx.x >> 6, l = threadIdx.x & 63;
            const int r = 16 * q + (l & 15), n = ta.row0 + r;
            if (r < ta.rows) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int t = 4 * (l >> 4) + v;
                    if (t >= nrow) continue;
                    const int q = slots[m0 + t];
                    if (yacc)  // at most two additions into zero: the same bits in either order
                        unsafeAtomicAdd(yacc + static_cast<int64_t>(q / topk) * h + n, rw[q] * s[0][v]);
                    else
                        obuf[static_cast<int64_t>(q) * h + n] = s[0][v];
                }
            }
        }
    }
}

// combine from the prep kernel's routing: grid (T, ceil(h / 1024)), four
// outputs per thread; y_t = sum_k w_tk * obuf[t*topk + k] in slot order.
__global__ void __launch_bounds__(256) moe_combine_routed(const float* __restrict__ obuf,
                                                          const int32_t* __restrict__ ridx,
                                                          const float* __restrict__ rw, int topk, int64_t h,
                                                          float* __restrict__ y, int32_t* __restrict__ out_idx,
                                                          float* __restrict__ out_w) {
    const int t = blockIdx.x;
    if (blockIdx.y == 0 && static_cast<int>(threadIdx.x) < topk) {
        if (out_idx) out_idx[t * topk + threadIdx.x] = ridx[t * topk + threadIdx.x];
        if (out_w) out_w[t * topk + threadIdx.x] = rw[t * topk + threadIdx.x];
    }
    const int64_t o = (static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x) * 4;
    if (o >= h) return;  // h is a multiple of 256
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < topk; k++) {
        if (ridx[t * topk + k] < 0) continue;
        const float wk = rw[t * topk + k];
        const float4 v = *reinterpret_cast<const float4*>(obuf + (static_cast<int64_t>(t) * topk + k) * h + o);
        s.x += wk * v.x;
        s.y += wk * v.y;
        s.z += wk * v.z;
        s.w += wk * v.w;
    }
    *reinterpret_cast<float4*>(y + static_cast<int64_t>(t) * h + o) = s;
}

// Workspace: hbuf (slots x i, fp32 for F32 experts, fp16 for Q4_K), obuf
// (slots x h fp32); Q4_K only: xh (tokens x h fp16), routing (ridx, rw),
// per-expert slot lists (eoff, elist).
struct MoeWs {
    size_t hbuf, obuf, xh, ridx, rw, eoff, elist, total;
};

MoeWs moe_ws(int64_t t, int32_t topk, int64_t h, int64_t i) {
    MoeWs w;
    auto al = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t slots = static_cast<size_t>(t) * topk;
    w.hbuf = 0;
    w.obuf = al(slots * i * sizeof(float));
    w.xh = w.obuf + al(slots * h * sizeof(float));
    w.ridx = w.xh + al(static_cast<size_t>(t) * h * 2);
    w.rw = w.ridx + al(slots * sizeof(int32_t));
    w.eoff = w.rw + al(slots * sizeof(float));
    w.elist = w.eoff + al((MOE_MAX_EXPERTS + 1) * sizeof(int32_t));
    w.total = w.elist + al(slots * sizeof(int32_t));
    return w;
}

}  // namespace
}  // namespace vb

using namespace vb;

extern "C" int64_t vb_moe_workspace(int32_t n_tokens, int32_t topk, int64_t h, int64_t i) {
    if (n_tokens < 0 || topk <= 0 || h <= 0 || i <= 0) return -1;
    return static_cast<int64_t>(moe_ws(n_tokens, topk, h, i).total);
}

namespace {
bool moe_quant_type(int32_t t) {
    return t == TYPE_Q4_K || t == TYPE_Q6_K || t == TYPE_Q8_0 || t == TYPE_Q5_K || t == TYPE_Q4_0 || t == TYPE_Q4_1 ||
           t == TYPE_Q5_0 || t == TYPE_Q5_1;
}
}  // namespace

extern "C" int vb_moe_grouped_ffn_types(const void* const* wg, const void* const* wu, const void* const* wd,
                                        int32_t n_exp, const float* x, int32_t n_tokens, const float* router_logits,
                                        int32_t topk, float* y, int32_t* out_idx, float* out_w, int64_t h, int64_t i,
                                        int32_t gate_up_type, int32_t down_type, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    hipStream_t st = as_stream(stream);
    if (n_exp <= 0 || n_exp > MOE_MAX_EXPERTS || topk <= 0 || topk > MOE_MAX_TOPK || topk > n_exp ||
        n_tokens < 0 || static_cast<int64_t>(n_tokens) * topk > MOE_MAX_SLOTS || h <= 0 || i <= 0 || !wg ||
        !wu || !wd || (n_tokens > 0 && (!x || !router_logits || !y))) {
        set_error("vb_moe_grouped_ffn: bad arguments (n_exp<=%d, topk<=%d, tokens*topk<=%d)", MOE_MAX_EXPERTS,
                  MOE_MAX_TOPK, MOE_MAX_SLOTS);
        return E_INVAL;
    }
    const bool f32 = gate_up_type == TYPE_F32 && down_type == TYPE_F32;
    if (!(f32 || (moe_quant_type(gate_up_type) && moe_quant_type(down_type))) || h % 256 != 0 || i % 256 != 0) {
        set_error("vb_moe_grouped_ffn: experts of Q4_K / Q6_K / Q8_0 / Q5_K / Q4_0 / Q4_1 / Q5_0 / Q5_1 (gate/up "
                  "and down each; or F32 throughout) with h, i multiples of 256 are supported (got gate/up %d, down "
                  "%d)", gate_up_type, down_type);
        return E_UNSUPPORTED;
    }
    if (n_tokens == 0) return OK;
    if (reinterpret_cast<uintptr_t>(x) % 16) {
        set_error("vb_moe_grouped_ffn: x must be 16-byte aligned");
        return E_INVAL;
    }
    const MoeWs ws = moe_ws(n_tokens, topk, h, i);
    if (!workspace || workspace_bytes < ws.total) {
        set_error("vb_moe_grouped_ffn: workspace of %zu bytes needed", ws.total);
        return E_NOMEM;
    }
    ExpertPtrs pg{}, pu{}, pd{};
    for (int e = 0; e < n_exp; e++) {
        if (!wg[e] || !wu[e] || !wd[e] || reinterpret_cast<uintptr_t>(wg[e]) % 16 ||
            reinterpret_cast<uintptr_t>(wu[e]) % 16 || reinterpret_cast<uintptr_t>(wd[e]) % 16) {
            set_error("vb_moe_grouped_ffn: expert %d weights null or not 16-byte aligned", e);
            return E_INVAL;
        }
        pg.p[e] = static_cast<const uint8_t*>(wg[e]);
        pu.p[e] = static_cast<const uint8_t*>(wu[e]);
        pd.p[e] = static_cast<const uint8_t*>(wd[e]);
    }
    float* hbuf = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + ws.hbuf);
    float* obuf = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + ws.obuf);
    const int64_t slots = static_cast<int64_t>(n_tokens) * topk;
    const int64_t nx = static_cast<int64_t>(n_tokens) * h;
    if (h > INT32_MAX || i > INT32_MAX || nx * 2 >= (int64_t(1) << 31) || slots * i * 2 >= (int64_t(1) << 31)) {
        set_error("vb_moe_grouped_ffn: activation tensors too large for 32-bit offsets");
        return E_INVAL;
    }
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    _Float16* xh = reinterpret_cast<_Float16*>(wsb + ws.xh);
    int32_t* ridx = reinterpret_cast<int32_t*>(wsb + ws.ridx);
    float* rw = reinterpret_cast<float*>(wsb + ws.rw);
    int32_t* eoff = reinterpret_cast<int32_t*>(wsb + ws.eoff);
    int32_t* elist = reinterpret_cast<int32_t*>(wsb + ws.elist);
    // 1. routing, per-expert slot lists, fp16 activations
    const dim3 prep(static_cast<uint32_t>(1 + (nx / 8 + PREP_THREADS - 1) / PREP_THREADS));
    // top-k <= 2 on the quantized experts: the down kernels add each slot's
    // weighted output into y (zeroed here), so no combine launch follows
    const bool fused_combine = !f32 && topk <= 2;
    float* yacc = fused_combine ? y : nullptr;
    moe_prep_kernel<<<prep, dim3(PREP_THREADS), 0, st>>>(x, router_logits, n_tokens, n_exp, topk, nx, xh, ridx, rw,
                                                         eoff, elist, yacc, out_idx, out_w);
    int rc = check_launch("vb_moe_grouped_ffn");
    if (rc != OK) return rc;
    // 2, 3. experts
    if (!f32) {
        const int64_t rb_gu = row_bytes(gate_up_type, h), rb_d = row_bytes(down_type, i);
        if (i * rb_gu + 4 >= (int64_t(1) << 32) || h * rb_d + 4 >= (int64_t(1) << 32)) {
            set_error("vb_moe_grouped_ffn: expert tensors too large for 32-bit offsets");
            return E_INVAL;
        }
        _Float16* hb16 = reinterpret_cast<_Float16*>(hbuf);
        // Q4_K on the skinny tiles (one activation fragment per 16 slots
        // serves four 16-row column groups); the other types on the
        // expert-grouped K-split kernel (gemm_kq.hip), gate/up with the same
        // SwiGLU epilogue
        if (gate_up_type == TYPE_Q4_K) {
            const dim3 gu(static_cast<uint32_t>((i + skinny::ROWS - 1) / skinny::ROWS), n_exp);
            moe_gate_up_q4k<MOE_WAVES><<<gu, dim3(64 * MOE_WAVES), skinny::lds_bytes<MOE_WAVES>(), st>>>(
                pg, pu, xh, eoff, elist, static_cast<int>(slots), topk, static_cast<int>(h), static_cast<int>(i),
                static_cast<int>(rb_gu),
                static_cast<uint32_t>(i * rb_gu), static_cast<uint32_t>(nx * 2), hb16);
            if ((rc = check_launch("vb_moe_grouped_ffn")) != OK) return rc;
        } else if ((rc = moe_kq(gate_up_type, true, wg, wu, n_exp, xh, nx * 2, topk, eoff, elist,
                                static_cast<int>(slots), i, h, hb16, nullptr, nullptr, nullptr, st)) != OK) {
            return rc;
        }
        if (down_type == TYPE_Q4_K) {
            const dim3 dn(static_cast<uint32_t>((h + skinny::ROWS - 1) / skinny::ROWS), n_exp);
            moe_down_q4k<MOE_WAVES><<<dn, dim3(64 * MOE_WAVES), skinny::lds_bytes<MOE_WAVES>(), st>>>(
                pd, hb16, eoff, elist, static_cast<int>(slots), static_cast<int>(h), static_cast<int>(i),
                static_cast<int>(rb_d),
                static_cast<uint32_t>(h * rb_d), static_cast<uint32_t>(slots * i * 2), obuf, rw, topk, yacc);
        } else if ((rc = moe_kq(down_type, false, wd, nullptr, n_exp, hb16, slots * i * 2, topk, eoff, elist,
                                static_cast<int>(slots), h, i, nullptr, obuf, rw, yacc, st)) != OK) {
            return rc;
        }
    } else {
        const dim3 gu_grid(static_cast<uint32_t>((i + 15) / 16), n_exp), dn_grid(static_cast<uint32_t>((h + 15) / 16), n_exp);
        moe_gate_up_kernel<TYPE_F32><<<gu_grid, dim3(256), 0, st>>>(pg, pu, x, eoff, elist, static_cast<int>(slots),
                                                                    topk, h, i,
                                                                    row_bytes(TYPE_F32, h), hbuf);
        if ((rc = check_launch("vb_moe_grouped_ffn")) != OK) return rc;
        moe_down_kernel<TYPE_F32><<<dn_grid, dim3(256), 0, st>>>(pd, hbuf, eoff, elist, static_cast<int>(slots), h,
                                                                 i, row_bytes(TYPE_F32, i),
                                                                 obuf);
    }
    if ((rc = check_launch("vb_moe_grouped_ffn")) != OK) return rc;
    // 4. weighted combine (F32 experts, top-k > 2)
    if (fused_combine) return OK;
    moe_combine_routed<<<dim3(static_cast<uint32_t>(n_tokens), static_cast<uint32_t>((h + 1023) / 1024)), dim3(256), 0,
                         st>>>(obuf, ridx, rw, topk, h, y, out_idx, out_w);
    return check_launch("vb_moe_grouped_ffn");
}

extern "C" int vb_moe_grouped_ffn(const void* const* wg, const void* const* wu, const void* const* wd,
                                  int32_t n_exp, const float* x, int32_t n_tokens, const float* router_logits,
                                  int32_t topk, float* y, int32_t* out_idx, float* out_w, int64_t h,
                                  int64_t i, int32_t ggml_type, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    return vb_moe_grouped_ffn_types(wg, wu, wd, n_exp, x, n_tokens, router_logits, topk, y, out_idx, out_w, h, i,
                                    ggml_type, ggml_type, workspace, workspace_bytes, stream);
}

namespace vb {
namespace {
__global__ void __launch_bounds__(256) moe_route_kernel(const float* __restrict__ logits, int t_n, int e_n, int topk,
                                                        int32_t* __restrict__ out_idx, float* __restrict__ out_w) {
    const int t = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);  // one wave per token
    if (t >= t_n) return;
    route_token_wave(logits + static_cast<int64_t>(t) * e_n, e_n, topk, out_idx + t * topk, out_w + t * topk,
                     nullptr);
}
}  // namespace
}  // namespace vb

extern "C" int vb_moe_route(const float* router_logits, int32_t n_tokens, int32_t n_exp, int32_t topk,
                            int32_t* out_idx, float* out_w, void* stream) {
    if (n_exp <= 0 || n_exp > MOE_MAX_EXPERTS || topk <= 0 || topk > MOE_MAX_TOPK || topk > n_exp || n_tokens < 0 ||
        (n_tokens > 0 && (!router_logits || !out_idx || !out_w))) {
        set_error("vb_moe_route: bad arguments");
        return E_INVAL;
    }
    if (n_tokens == 0) return OK;
    moe_route_kernel<<<dim3(static_cast<uint32_t>((n_tokens + 3) / 4)), dim3(256), 0, as_stream(stream)>>>(
        router_logits, n_tokens, n_exp, topk, out_idx, out_w);
    return check_launch("vb_moe_route");
}
