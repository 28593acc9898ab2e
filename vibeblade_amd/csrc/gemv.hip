// Dequant-fused GEMV, M = 1:  y[n] = sum_k W[n, k] x[k]  (GGUF layout).
//
// Replaces gemv_dequant (cpp/src/dequant.cpp:739-780), which decodes every
// weight to an fp32 scratch row and does a saxpy per row.  Here no weight is
// ever materialised: each lane owns a 64-element "unit" of a row and streams
// the packed bytes of that unit straight into integer dot products against
// the activation encoding of gemv_core.hpp.
//
// Launch shape.  A row's units are split over `wpr` waves ("k-slices" of
// upw <= 64 units, upw a multiple of 4 so a Q4_K super-block never straddles
// two lanes' quads); each wave keeps its activation slice in registers for
// the whole launch and walks `rpg` consecutive rows, with D rows in flight
// (all of them when rpg <= D).  Per-row wave sums go to LDS; the workgroup
// writes y (adding the wpr partial sums in a fixed order) at the end.
#include <cstdlib>
#include <cstring>

#include "gemv_core.hpp"
#include "vb_common.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

using namespace gemvc;

// Row sources.  ROWS_PLAIN: row r of w.  ROWS_PAIRS: row r is row gidx[r/2]
// of w (r even) or of w2 (r odd) -- gate/up pairs of the active neurons of a
// sparse FFN, one launch and one activation encode for both matrices.
// ROWS_DPAIRS: row r is row r/2 of w or w2 -- the gate/up pairs of every
// neuron (a dense FFN block).
constexpr int ROWS_PLAIN = 0;
constexpr int ROWS_PAIRS = 1;
constexpr int ROWS_DPAIRS = 2;

// Row indices are 32-bit (the host checks n and nsrc < 2^31): 64-bit compares
// have no scalar form on gfx9, and would pull the wave-uniform row
// addressing onto the VALU.
template <int MODE>
__device__ __forceinline__ const uint8_t* row_ptr(const uint8_t* w, const uint8_t* w2,
                                                  const int32_t* gidx, int nsrc, int row, int64_t rb) {
    if constexpr (MODE == ROWS_PLAIN) {
        return w + static_cast<int64_t>(row) * rb;
    } else if constexpr (MODE == ROWS_DPAIRS) {
        return ((row & 1) ? w2 : w) + static_cast<int64_t>(row >> 1) * rb;
    } else {
        int src = gidx[row >> 1];
        src = src < 0 ? 0 : (src >= nsrc ? nsrc - 1 : src);  // never read outside the tensor
        return ((row & 1) ? w2 : w) + static_cast<int64_t>(src) * rb;
    }
}

// Weight loads are staged.  A wave's share of a row (its k-slice: up to 64
// units, e.g. 2304 B of Q4_K, 3360 B of Q6_K, 4352 B of Q8_0) is read as
// contiguous 16-byte pieces, piece p of lane L at byte 16 L + 1024 p of the
// slice, with non-temporal buffer loads (the weights are streamed once), and
// written to a per-wave LDS buffer; the lanes then read their unit's bytes
// from LDS with the type's unit loader.  Every load instruction covers whole
// cache lines, where per-lane unit loads touch parts of many lines per
// instruction (on MI355X, 14336 x 4096 Q4_K loads alone: 6.6 us per launch
// against 7.4 us).  A slice that starts 2 bytes past a dword (Q6_K / Q3_K
// blocks) is read from the dword below, and the LDS copy is addressed with
// the same shift.  Loads past the slice (and whole padding rows) use a
// buffer resource that ends there: they return zeros and read nothing (the
// range check is per dword, measured on MI355X: a 16-byte load straddling the
// end returns the dwords inside it).
template <int TYPE>
constexpr int slice_bytes_max() {  // 64 units
    return TYPE == TYPE_Q4_K ? 2304 : TYPE == TYPE_Q5_K ? 2816 : TYPE == TYPE_Q6_K ? 3360
         : TYPE == TYPE_Q8_0 ? 4352 : TYPE == TYPE_Q2_K ? 1344 : TYPE == TYPE_Q3_K ? 1760
         : TYPE == TYPE_Q4_0 ? 2304 : TYPE == TYPE_Q4_1 ? 2560 : TYPE == TYPE_Q5_0 ? 2816 : 3072;
}
template <int TYPE>
constexpr int stage_pieces() {
    constexpr int slack = (TYPE == TYPE_Q6_K || TYPE == TYPE_Q3_K) ? 2 : 0;
    return (slice_bytes_max<TYPE>() + slack + 1023) / 1024;
}
constexpr int CACHE_NT = 2;  // buffer-load cache policy: non-temporal

// Register budget: a 16-wave workgroup leaves 128 VGPRs per lane, enough
// for a ring of 4 staged Q4_K row slices (3 pieces = 12 VGPRs each) or 2 of
// the larger ones; deeper rings run in 8-wave workgroups (256 VGPRs).
template <int TYPE>
constexpr int max_d16() { return stage_pieces<TYPE>() <= 3 && TYPE != TYPE_Q3_K ? 4 : 2; }
template <int TYPE, int D>
constexpr int gemv_max_threads() { return D <= max_d16<TYPE>() ? 1024 : 512; }

// One workgroup: `wpg` waves = (wpg / wpr) row groups x wpr k-slices.  Row
// group g owns rows [row0, row0 + rpg); k-slice kw covers units
// [kw*upw, kw*upw + upw) of each of them, lane = unit.  Rows stream through a
// ring of D register buffers (staged slices, above): the loads of row s + D
// are issued as soon as row s has been computed.  The row count is padded to
// a multiple of D; padding rows issue loads of an empty resource (no memory
// access) and compute nothing, which keeps every load outside branches (a
// branch around loads makes the compiler's wait counts conservative).
//
// zbuf / zn: an int buffer the first workgroup clears (the counters of a
// following kernel; a fill inside this launch keeps memsets out of captured
// graphs).
//
// FUSE: the GemvFuse work (vb_internal.hpp) -- RMSNorm of x inside the
// encode, the gate/up activation epilogue (rows_wg even, so a neuron's two
// rows never straddle workgroups), the residual add.  FUSE = false is the
// plain GEMV, and its code does not change.
template <int TYPE, int D, int MODE, bool FUSE>
__global__ void __launch_bounds__((gemv_max_threads<TYPE, D>())) gemv_q_kernel(
        const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, const int32_t* __restrict__ gidx,
        int nsrc, const float* __restrict__ x, float* __restrict__ y, int n_bound, int64_t rb, int units,
        int slots, int upw, int wpr, int rpg, int* __restrict__ zbuf, int zn, GemvFuse fz,
        const int32_t* __restrict__ n_dev, uint32_t slice_stride) {
    if (zn > 0 && blockIdx.x == 0) {
        for (int i = threadIdx.x; i < zn; i += blockDim.x) zbuf[i] = 0;
    }
    // gathered pairs with a device count: rows past 2 * count are not computed
    int n = n_bound;
    if constexpr (MODE == ROWS_PAIRS) n = 2 * active_count(n_bound / 2, n_dev);
    using Unit = typename UnitOf<TYPE>::T;
    constexpr int P = stage_pieces<TYPE>();
    struct Raw {
        u32x4 p[P];
        uint32_t shift;  // the slice's start past the dword it was read from
    };
    extern __shared__ uint4 xq[];
    const int lane = threadIdx.x & 63;
    // wave-uniform (readfirstlane): row addressing then runs on the scalar unit
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    // (integer division runs on the VALU: re-assert uniformity afterwards)
    const int groups = __builtin_amdgcn_readfirstlane(static_cast<int>(blockDim.x >> 6) / wpr);
    const int g = __builtin_amdgcn_readfirstlane(wave / wpr), kw = wave - g * wpr;
    const int rows_wg = groups * rpg;
    float* red = reinterpret_cast<float*>(xq + XQ_QUADS * slots);  // [wpr][rows_wg]
    // the wave's LDS slice buffer, after red (padded to 16 bytes)
    u32x4* stage_buf = reinterpret_cast<u32x4*>(xq + XQ_QUADS * slots + (wpr * rows_wg + 3) / 4) + wave * (P * 64);
    const uint8_t* stage_bytes = reinterpret_cast<const uint8_t*>(stage_buf);
    const int wg_row0 = static_cast<int>(blockIdx.x) * rows_wg;
    if constexpr (MODE == ROWS_PAIRS) {
        if (wg_row0 >= n) return;  // uniform: before any load or barrier
    }
    const int row0 = wg_row0 + g * rpg;
    const int u = kw * upw + lane;
    const bool valid = lane < upw && u < units;
    // Idle lanes load a real unit (discarded).  Q4_K / Q5_K keep u % 4 ==
    // lane % 4 (units and upw are multiples of 4 there) so every quad reads
    // one super-block; rows of fewer than 4 units (32-element types, k < 256)
    // take unit 0.
    const int ui = units - 4 + (lane & 3);
    const int uc = valid ? u : (ui < 0 ? 0 : ui);
    const auto usel = make_unit_sel<TYPE>(uc);
    // the lane's unit inside the slice (idle lanes: one of the slice's first
    // four, same parity as uc)
    const int ul = valid ? lane : (lane & 3);
    const int nsteps_p = ((rpg + D - 1) / D) * D;
    const int64_t slice_off = static_cast<int64_t>(kw) * slice_stride;
    const int64_t slice_left = rb - slice_off;
    const uint32_t slice_len = slice_left < slice_stride ? static_cast<uint32_t>(slice_left) : slice_stride;

    auto issue = [&](Raw& r, int step) {
        const bool live = step < rpg && row0 + step < n;  // wave-uniform
        step = step < rpg ? step : rpg - 1;
        int row = row0 + step;
        row = row < n ? row : n - 1;
        const uint8_t* sp = row_ptr<MODE>(w, w2, gidx, nsrc, row, rb) + slice_off;
        const uint32_t shift = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sp) & 3u);
        // the range check is per dword: end the resource at the dword that holds
        // the slice's last byte (at most 3 bytes past it, in the same dword)
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(sp - shift, live ? (slice_len + shift + 3u) & ~3u : 0u);
#pragma unroll
        for (int p = 0; p < P; p++)
            r.p[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(16 * lane + 1024 * p), 0, CACHE_NT);
        r.shift = shift;
    };
    // the slice through the wave's LDS buffer; the lane's unit from there
    // (LDS operations of one wave run in order: one buffer is enough)
    auto stage = [&](const Raw& r, Unit& v) {
#pragma unroll
        for (int p = 0; p < P; p++) stage_buf[lane + 64 * p] = r.p[p];
        load_unit(stage_bytes + r.shift, ul, v);
    };

    // x first, then the first D rows of weights, then the encode: the encode
    // only waits for x, and the weights are in flight meanwhile.
    Raw v[D];
    const bool x_in_regs = slots * 8 <= XT_MAX * static_cast<int>(blockDim.x);
    XTasks xt;
    [[maybe_unused]] XTasks nt;  // norm weights of the same tasks (FUSE)
    [[maybe_unused]] const bool norm = FUSE && fz.norm_w != nullptr;
    if (x_in_regs) prefetch_x<TYPE>(x, units, slots, xt);
    if constexpr (FUSE) {
        if (x_in_regs && norm) prefetch_x<TYPE>(fz.norm_w, units, slots, nt);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < D; j++) issue(v[j], j);
    __builtin_amdgcn_sched_barrier(0);  // keep the weight loads ahead of the encode
    if constexpr (FUSE) {
        if (norm) {
            // red is free until the main loop; it holds >= one float per wave
            const float ss = wg_sum_fixed(x_in_regs ? sumsq_tasks(units, slots, xt)
                                                    : sumsq_loop(x, units * 64), red);
            const float rinv = rms_inv(ss, units * 64, fz.eps);
            if (x_in_regs) {
                scale_tasks(xt, nt, rinv);
                encode_x_regs<TYPE>(units, slots, xt, xq);
            } else {
                encode_x_loop_norm<TYPE>(x, fz.norm_w, rinv, units, slots, xq);
            }
        } else if (x_in_regs) {
            encode_x_regs<TYPE>(units, slots, xt, xq);
        } else {
            encode_x_loop<TYPE>(x, units, slots, xq);
        }
    } else {
        if (x_in_regs)
            encode_x_regs<TYPE>(units, slots, xt, xq);
        else
            encode_x_loop<TYPE>(x, units, slots, xq);
    }
    __syncthreads();

    XSlice xs;
    read_xslice(xq, slots, valid ? u : 0, xs);
    float* myred = red + kw * rows_wg + g * rpg;

    auto compute = [&](const Raw& rr, int step) {
        if (step >= rpg) return;  // padding step (uniform)
        Unit vv;
        stage(rr, vv);
        float a = unit_dot(vv, xs, usel);
        a = valid ? a : 0.f;
        const float tot = wave_sum_dpp(a);
        if (lane == 0) myred[step] = tot;
    };

    int s = 0;
    for (; s + D < nsteps_p; s += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            compute(v[j], s + j);
            issue(v[j], s + j + D);
        }
    }
#pragma unroll
    for (int j = 0; j < D; j++) compute(v[j], s + j);

    __syncthreads();
    if constexpr (FUSE) {
        if (fz.act >= 0) {  // neuron p = (wg_row0 + 2i) / 2: rows 2p (gate), 2p + 1 (up)
            for (int i = threadIdx.x; 2 * i < rows_wg; i += blockDim.x) {
                float g = red[2 * i], uu = red[2 * i + 1];
                for (int k = 1; k < wpr; k++) {
                    g += red[k * rows_wg + 2 * i];
                    uu += red[k * rows_wg + 2 * i + 1];
                }
                const int r = wg_row0 + 2 * i;
                if (r + 1 < n) y[r >> 1] = act_pair(g, uu, fz.act);
            }
            return;
        }
    }
    for (int i = threadIdx.x; i < rows_wg; i += blockDim.x) {
        float t = red[i];
        for (int k = 1; k < wpr; k++) t += red[k * rows_wg + i];
        if constexpr (FUSE) {
            if (fz.resid && wg_row0 + i < n) t += fz.resid[wg_row0 + i];
        }
        if (wg_row0 + i < n) y[wg_row0 + i] = t;
    }
}

// F32 / F16 weights: plain fp32 dot products, one wave per R rows (rows
// plain or gathered gate/up pairs, as in the block-quantized kernel).
template <int TYPE, int R, int MODE>
__global__ void __launch_bounds__(256) gemv_plain_kernel(const uint8_t* __restrict__ w,
                                                         const uint8_t* __restrict__ w2,
                                                         const int32_t* __restrict__ gidx, int nsrc,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int n, int64_t k,
                                                         int* __restrict__ zbuf, int zn) {
    if (zn > 0 && blockIdx.x == 0) {
        for (int i = threadIdx.x; i < zn; i += blockDim.x) zbuf[i] = 0;
    }
    const int lane = threadIdx.x & 63;
    const int row0 = (static_cast<int>(blockIdx.x) * static_cast<int>(blockDim.x >> 6) +
                      __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6))) * R;
    constexpr int64_t ES = TYPE == TYPE_F32 ? 4 : 2;  // F16 and BF16: 2
    const uint8_t* rp[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int row = row0 + r;
        row = row < n ? row : n - 1;
        rp[r] = row_ptr<MODE>(w, w2, gidx, nsrc, row, k * ES);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (int64_t i = lane; i < k; i += 64) {
        const float xv = x[i];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float wv;
            if constexpr (TYPE == TYPE_F32)
                wv = reinterpret_cast<const float*>(rp[r])[i];
            else if constexpr (TYPE == TYPE_BF16)
                wv = __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(rp[r])[i]) << 16);
            else
                wv = __half2float(reinterpret_cast<const __half*>(rp[r])[i]);
            acc[r] += wv * xv;
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum_dpp(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++)
            if (row0 + r < n) y[row0 + r] = acc[r];
    }
}

constexpr size_t kLdsBytes = 160 * 1024;  // LDS per CU (gfx950)

struct GemvShape {
    int units, slots, upw, wpr, wpg, rpg, depth;
    int64_t grid;
    size_t lds;
};

// Ring depth for rpg rows per wave (sweeps on MI355X with the staged
// loads): two rows in flight for every type and shape, one for a single row
// (no ring) and for Q3_K (its 20-VGPR units keep 16-wave workgroups only
// without a ring).  Deeper rings slowed every shape: Q6_K lm_head 128256 x
// 4096 ran 78.1 us at 2 against 86.0 us at 4, Q4_K 4096 x 14336 9.6 against
// 10.9 us, Q8_0 4096 x 4096 5.35 against 6.5 us at 3.
template <int TYPE>
int ring_depth(int rpg, int) {
    if (rpg <= 1 || TYPE == TYPE_Q3_K) return 1;
    return 2;
}

template <int TYPE>
int gemv_max_threads_host(int depth) { return depth <= max_d16<TYPE>() ? 1024 : 512; }

// Launch geometry.  k-slices: wpr = ceil(units / 64) waves per row, upw the
// units per slice rounded up to a multiple of 4.  Rows (rules from sweeps on
// MI355X, 256 CUs): single-slice rows run in one 8-wave workgroup per CU
// with ceil(n / (8 CUs)) rows per wave (14336 rows: 7; Q6_K lm_head, 128256
// rows: 63; Q8_0 4096 rows: 2, 5.35 us against 5.8 us at one row per wave
// in two workgroups per CU).  Multi-slice rows (k > 4096) use 16-wave
// workgroups.  VB_GEMV_CFG="wpg,rpg" and VB_GEMV_RING=d override
// (tuning sweeps; Knobs).
template <int TYPE>
GemvShape gemv_shape(int64_t n, int units, bool even_rows = false) {
    GemvShape s;
    s.units = units;
    s.wpr = (units + 63) / 64;
    s.upw = ((units + s.wpr - 1) / s.wpr + 3) & ~3;
    s.slots = (((s.wpr - 1) * s.upw + 64) + 7) & ~7;
    if (s.wpr == 1) {  // one 8-wave workgroup per CU, every row count
        s.wpg = 8;
        const int64_t cus = num_cus();
        s.rpg = static_cast<int>((n + cus * 8 - 1) / (cus * 8));
    } else {
        s.wpg = s.wpr <= 4 ? 16 / s.wpr * s.wpr : s.wpr;
        if (s.wpg > 16) s.wpg = s.wpr;  // > 4096 * 16 elements: one row group per workgroup
        const int groups = s.wpg / s.wpr;
        const int64_t cus = num_cus();
        s.rpg = static_cast<int>((n + cus * groups - 1) / (cus * groups));
    }
    if (s.rpg < 1) s.rpg = 1;
    const int64_t max_rpg = kMaxRedFloats / (static_cast<int64_t>(s.wpg / s.wpr) * s.wpr);
    if (s.rpg > max_rpg) s.rpg = static_cast<int>(max_rpg);
    const int ring = knobs().gemv_ring > 4 ? 4 : knobs().gemv_ring;  // ring-depth override (0: none)
    auto depth_of = [&](int rpg) { return ring ? ring : ring_depth<TYPE>(rpg, s.wpr); };
    // the block size must fit the launch bounds of the kernel of that depth
    if (64 * s.wpg > gemv_max_threads_host<TYPE>(depth_of(s.rpg))) s.wpg = 8 / s.wpr * s.wpr;
    if (s.wpg < s.wpr) s.wpg = s.wpr;
    if (knobs().gemv_cfg_wpg > 0) {
        const int a = knobs().gemv_cfg_wpg, b = knobs().gemv_cfg_rpg;
        if (a <= 16 && a % s.wpr == 0 &&
            static_cast<int64_t>(a / s.wpr) * b * s.wpr <= kMaxRedFloats &&
            64 * a <= gemv_max_threads_host<TYPE>(depth_of(b))) {
            s.wpg = a;
            s.rpg = b;
        }
    }
    // pair epilogue: a neuron's gate and up rows in one workgroup
    if (even_rows && ((s.wpg / s.wpr) * s.rpg) % 2 != 0) {
        if (s.rpg > 1 && static_cast<int64_t>(s.wpg / s.wpr) * (s.rpg + 1) * s.wpr > kMaxRedFloats)
            s.rpg -= 1;
        else
            s.rpg += 1;
        if (64 * s.wpg > gemv_max_threads_host<TYPE>(depth_of(s.rpg))) s.wpg = 8 / s.wpr * s.wpr;
        if (s.wpg < s.wpr) s.wpg = s.wpr;
    }
    s.depth = depth_of(s.rpg);
    int64_t rows_wg = static_cast<int64_t>(s.wpg / s.wpr) * s.rpg;
    auto lds_of = [&](int wpg) {
        const int64_t rw = static_cast<int64_t>(wpg / s.wpr) * s.rpg;
        return static_cast<size_t>(s.slots) * XQ_QUADS * sizeof(uint4) + ((rw * s.wpr + 3) / 4) * sizeof(uint4) +
               static_cast<size_t>(wpg) * stage_pieces<TYPE>() * 1024;
    };
    // the per-wave slice buffers must fit the CU's LDS with the encoding
    while (lds_of(s.wpg) > kLdsBytes && s.wpg > s.wpr) s.wpg -= s.wpr;
    rows_wg = static_cast<int64_t>(s.wpg / s.wpr) * s.rpg;
    s.grid = (n + rows_wg - 1) / rows_wg;
    s.lds = lds_of(s.wpg);
    return s;
}

template <int TYPE, int D>
int launch_gemv_d(const GemvShape& s, const void* w, const RowSrc& src, const GemvFuse& fz, const float* x,
                  float* y, int64_t n, int64_t rb, hipStream_t st) {
    if (64 * s.wpg > gemv_max_threads<TYPE, D>()) {  // never launch past the kernel's launch bounds
        set_error("vb_gemv: %d threads exceed the %d of the depth-%d kernel", 64 * s.wpg,
                  gemv_max_threads<TYPE, D>(), D);
        return E_INVAL;
    }
    const dim3 g(static_cast<uint32_t>(s.grid)), b(64 * s.wpg);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const uint8_t* w2 = static_cast<const uint8_t*>(src.w2);
    const int ni = static_cast<int>(n), nsrc = static_cast<int>(src.nsrc);
    const uint32_t stride = static_cast<uint32_t>(row_bytes(TYPE, 64 * static_cast<int64_t>(s.upw)));
#define VB_GEMV_LAUNCH(MODE, FUSE)                                                                      \
    gemv_q_kernel<TYPE, D, MODE, FUSE><<<g, b, s.lds, st>>>(wb, w2, src.gidx, nsrc, x, y, ni, rb, s.units, \
                                                            s.slots, s.upw, s.wpr, s.rpg, src.zbuf, src.zn, fz,  \
                                                            src.n_dev, stride)
    if (fz.any()) {
        if (src.dense_pairs)
            VB_GEMV_LAUNCH(ROWS_DPAIRS, true);
        else if (src.gidx)
            VB_GEMV_LAUNCH(ROWS_PAIRS, true);
        else
            VB_GEMV_LAUNCH(ROWS_PLAIN, true);
    } else if (src.dense_pairs) {
        VB_GEMV_LAUNCH(ROWS_DPAIRS, false);
    } else if (src.gidx) {
        VB_GEMV_LAUNCH(ROWS_PAIRS, false);
    } else {
        VB_GEMV_LAUNCH(ROWS_PLAIN, false);
    }
#undef VB_GEMV_LAUNCH
    return check_launch("vb_gemv");
}

template <int TYPE>
int launch_gemv_q(const void* w, const RowSrc& src, const GemvFuse& fz, const float* x, float* y, int64_t n,
                  int64_t k, int64_t rb, hipStream_t st) {
    const int units = static_cast<int>(k / 64);
    const GemvShape s = gemv_shape<TYPE>(n, units, fz.act >= 0);
    if (s.slots > kMaxSlots || s.lds > kLdsBytes) {
        set_error("vb_gemv: k=%lld exceeds the supported maximum of 32768", static_cast<long long>(k));
        return E_UNSUPPORTED;
    }
    if (fz.act >= 0 && ((s.wpg / s.wpr) * s.rpg) % 2 != 0) {  // never split a neuron's rows
        set_error("vb_gemv: internal: odd rows per workgroup in a pair epilogue");
        return E_INVAL;
    }
    switch (s.depth) {
    case 1: return launch_gemv_d<TYPE, 1>(s, w, src, fz, x, y, n, rb, st);
    case 2: return launch_gemv_d<TYPE, 2>(s, w, src, fz, x, y, n, rb, st);
    case 3: return launch_gemv_d<TYPE, 3>(s, w, src, fz, x, y, n, rb, st);
    default: return launch_gemv_d<TYPE, 4>(s, w, src, fz, x, y, n, rb, st);
    }
}

}  // namespace

// Shared with the other translation units (sparse / moe / ffn).  `src`
// selects gathered or dense gate/up pairs and an int buffer to clear (see
// RowSrc); `fz` the fused work (see GemvFuse).
int gemv_dispatch_fused(const void* w, const RowSrc& src, const GemvFuse& fz, const float* x, float* y,
                        int64_t n, int64_t k, int32_t type, hipStream_t st) {
    const int64_t rb = row_bytes(type, k);
    if (rb < 0) {
        set_error("vb_gemv: unsupported type %d or k=%lld not a whole number of blocks", type,
                  static_cast<long long>(k));
        return E_INVAL;
    }
    if (n < 0 || (n > 0 && (!w || !x || !y))) {
        set_error("vb_gemv: bad arguments (n=%lld)", static_cast<long long>(n));
        return E_INVAL;
    }
    if (n == 0) return OK;
    if (n > INT32_MAX || src.nsrc > INT32_MAX) {
        set_error("vb_gemv: n=%lld rows exceeds the supported maximum of 2^31-1", static_cast<long long>(n));
        return E_UNSUPPORTED;
    }
    if (is_block_type(type) && k % 64 != 0) {
        set_error("vb_gemv: k=%lld must be a multiple of 64 for type %d", static_cast<long long>(k), type);
        return E_UNSUPPORTED;
    }
    const bool blockq = is_block_type(type);
    if ((blockq && reinterpret_cast<uintptr_t>(x) % 16 != 0) || reinterpret_cast<uintptr_t>(x) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(w) % 4 != 0) {
        set_error("vb_gemv: x must be 16-byte aligned for block types (4-byte otherwise), W 4-byte aligned");
        return E_INVAL;
    }
    if ((type == TYPE_Q4_K || type == TYPE_Q5_K) && reinterpret_cast<uintptr_t>(w) % 16 != 0) {
        set_error("vb_gemv: Q4_K / Q5_K weights must be 16-byte aligned");
        return E_INVAL;
    }
    if ((fz.any() || src.dense_pairs) && !blockq) {
        set_error("vb_gemv: fused work and dense pairs need a Q4_K / Q6_K / Q8_0 weight (type %d)", type);
        return E_UNSUPPORTED;
    }
    if ((fz.act >= 0 || src.dense_pairs) && (n % 2 != 0 || !src.w2)) {
        set_error("vb_gemv: gate/up pairs need an even row count and both matrices");
        return E_INVAL;
    }
    if (fz.norm_w && reinterpret_cast<uintptr_t>(fz.norm_w) % 16 != 0) {
        set_error("vb_gemv: the norm weight must be 16-byte aligned");
        return E_INVAL;
    }
    switch (type) {
    case TYPE_Q4_K: {
        // v_dot4 kernel by default (fastest measured); VB_GEMV_Q4K_PATH=mfma
        // selects the int8-MFMA kernel (same arithmetic) for plain launches
        const bool plain = !fz.any() && !src.dense_pairs && !src.n_dev && !src.gidx && src.zn == 0;
        if (knobs().gemv_q4k_mfma && !fz.any() && !src.dense_pairs && !src.n_dev)
            return gemv_q4k_mfma(w, src, x, y, n, k, st);
        // short rows (k <= 4096) at <= 8 rows per wave: the dedicated kernel
        if (plain && !knobs().gemv_q4k_general && k <= 4096 && gemv_q4k_rpw(n) > 0)
            return gemv_q4k_short(w, x, y, n, k, st);
        // dense gate/up pairs with the activation epilogue (FFN block launch
        // 1), k <= 4096: the short-row arithmetic, RMSNorm in its encode
        if (src.dense_pairs && fz.act >= 0 && !fz.resid && !src.n_dev && !src.gidx && src.zn == 0 &&
            !knobs().gemv_q4k_general && k <= 4096 && k % 256 == 0 && gemv_q4k_pairs_npw(n / 2) > 0)
            return gemv_q4k_pairs(w, src.w2, x, fz.norm_w, fz.eps, fz.act, y, n / 2, k, st);
        // split rows (4096 < k <= 16384), plain or with the residual epilogue
        const bool resid_only = !fz.norm_w && fz.act < 0 && !src.dense_pairs && !src.n_dev && !src.gidx &&
                                src.zn == 0;
        if (resid_only && !knobs().gemv_q4k_general && k > 4096 && k % 256 == 0 && gemv_q4k_split_rpw(n, k) > 0)
            return gemv_q4k_split(w, x, y, fz.resid, n, k, st);
        return launch_gemv_q<TYPE_Q4_K>(w, src, fz, x, y, n, k, rb, st);
    }
    case TYPE_Q6_K:
    case TYPE_Q8_0: {
        // plain rows of whole 16-byte slots, k <= 4096 (the lm_head and the
        // Q8_0 4096 x 4096 shapes): the short-row kernel
        const bool plain = !fz.any() && !src.dense_pairs && !src.n_dev && !src.gidx && src.zn == 0;
        const bool general = type == TYPE_Q6_K ? knobs().gemv_q6k_general : knobs().gemv_q8_general;
        if (plain && !general && reinterpret_cast<uintptr_t>(w) % 16 == 0 && gemv_short_rpw(type, n, k) > 0)
            return gemv_short(type, w, x, y, n, k, st);
        // 4096 < k <= 16384 (a Q4_K_M file's Q6_K FFN down), plain or with
        // the residual epilogue: the split-row kernel
        const bool resid_only = !fz.norm_w && fz.act < 0 && !src.dense_pairs && !src.n_dev && !src.gidx &&
                                src.zn == 0;
        if (resid_only && !general && k > 4096 && gemv_split_rpw(type, n, k) > 0)
            return gemv_split(type, w, x, y, fz.resid, n, k, st);
        if (type == TYPE_Q6_K) return launch_gemv_q<TYPE_Q6_K>(w, src, fz, x, y, n, k, rb, st);
        return launch_gemv_q<TYPE_Q8_0>(w, src, fz, x, y, n, k, rb, st);
    }
    case TYPE_Q5_K: return launch_gemv_q<TYPE_Q5_K>(w, src, fz, x, y, n, k, rb, st);
    case TYPE_Q2_K: return launch_gemv_q<TYPE_Q2_K>(w, src, fz, x, y, n, k, rb, st);
    case TYPE_Q3_K: return launch_gemv_q<TYPE_Q3_K>(w, src, fz, x, y, n, k, rb, st);
    case TYPE_Q4_0: return launch_gemv_q<TYPE_Q4_0>(w, src, fz, x, y, n, k, rb, st);
    case TYPE_Q4_1: return launch_gemv_q<TYPE_Q4_1>(w, src, fz, x, y, n, k, rb, st);
    case TYPE_Q5_0: return launch_gemv_q<TYPE_Q5_0>(w, src, fz, x, y, n, k, rb, st);
    case TYPE_Q5_1: return launch_gemv_q<TYPE_Q5_1>(w, src, fz, x, y, n, k, rb, st);
    case TYPE_F32:
    case TYPE_F16:
    case TYPE_BF16: {
        constexpr int R = 4;
        const int64_t grid = (n + 4 * R - 1) / (4 * R);
        const int ni = static_cast<int>(n), nsrc = static_cast<int>(src.nsrc);
        const dim3 g(static_cast<uint32_t>(grid)), b(256);
        const uint8_t* wb = static_cast<const uint8_t*>(w);
        const uint8_t* w2 = static_cast<const uint8_t*>(src.w2);
        if (type == TYPE_F32) {
            if (src.gidx)
                gemv_plain_kernel<TYPE_F32, R, ROWS_PAIRS><<<g, b, 0, st>>>(wb, w2, src.gidx, nsrc, x, y, ni, k,
                                                                           src.zbuf, src.zn);
            else
                gemv_plain_kernel<TYPE_F32, R, ROWS_PLAIN><<<g, b, 0, st>>>(wb, w2, src.gidx, nsrc, x, y, ni, k,
                                                                           src.zbuf, src.zn);
        } else if (type == TYPE_BF16) {
            if (src.gidx)
                gemv_plain_kernel<TYPE_BF16, R, ROWS_PAIRS><<<g, b, 0, st>>>(wb, w2, src.gidx, nsrc, x, y, ni, k,
                                                                            src.zbuf, src.zn);
            else
                gemv_plain_kernel<TYPE_BF16, R, ROWS_PLAIN><<<g, b, 0, st>>>(wb, w2, src.gidx, nsrc, x, y, ni, k,
                                                                            src.zbuf, src.zn);
        } else {
            if (src.gidx)
                gemv_plain_kernel<TYPE_F16, R, ROWS_PAIRS><<<g, b, 0, st>>>(wb, w2, src.gidx, nsrc, x, y, ni, k,
                                                                           src.zbuf, src.zn);
            else
                gemv_plain_kernel<TYPE_F16, R, ROWS_PLAIN><<<g, b, 0, st>>>(wb, w2, src.gidx, nsrc, x, y, ni, k,
                                                                           src.zbuf, src.zn);
        }
        return check_launch("vb_gemv");
    }
    default:
        set_error("vb_gemv: unsupported type %d", type);
        return E_UNSUPPORTED;
    }
}

int gemv_dispatch_src(const void* w, const RowSrc& src, const float* x, float* y, int64_t n, int64_t k,
                      int32_t type, hipStream_t st) {
    return gemv_dispatch_fused(w, src, GemvFuse{}, x, y, n, k, type, st);
}

int gemv_dispatch(const void* w, const float* x, float* y, int64_t n, int64_t k, int32_t type,
                  hipStream_t st) {
    return gemv_dispatch_src(w, RowSrc{}, x, y, n, k, type, st);
}

}  // namespace vb

extern "C" int vb_gemv(const void* w, const float* x, float* y, int64_t n, int64_t k,
                       int32_t ggml_type, void* stream) {
    return vb::gemv_dispatch(w, x, y, n, k, ggml_type, vb::as_stream(stream));
}
