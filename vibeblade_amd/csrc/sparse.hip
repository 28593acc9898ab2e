// TurboSparse activation-sparse FFN (single token) and top-k selection.
//
// Reference semantics: vibeblade/sparse.py:199-283 (sparse_ffn_silu: gate ->
// top-k -> up on the active rows -> silu(gate)*up -> hidden @ down^T[active])
// and the dense-with-mask form of vibeblade/transformer.py:204-206; the
// activation is selectable: silu(g)*u, or relu(g)*relu(u) (the native
// engine's "dReLU" is plain ReLU: src/kernels.cpp:39-57, vibeblade/gpu.py:100).
//
// Given the sorted active neuron set S (|S| = n_active) and one token x[h]:
//   1. gate and up on the rows of S only: one GEMV launch over gathered
//      gate/up row pairs (gemv.hip, ROWS_PAIRS) -> gu[2r], gu[2r+1];
//   2. down:
//      layout 0 (GGUF, W_d is h rows x i): scatter act(gu) into a dense
//        hidden vector (cleared by the gate/up launch, so zeros off S) and
//        run the dense GEMV -- every down
//        super-block holds an active column at 10 % density, so all of W_d
//        is read;
//      layout 1 (neuron-major D = W_d^T, i rows x h, Q4_K): only the |S|
//        rows of D are read: y = sum_r act_r * D[S_r, :].  Workgroup u owns
//        output unit u (64 columns) over every active row; row partials meet
//        in LDS and are added in fixed order (deterministic, one launch).
#include <cstdlib>
#include <mutex>

#include "gemv_core.hpp"
#include "mfma_q4k.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

// layout 0: hid[active[r]] = act(gu[2r], gu[2r+1]); the gate/up launch has
// cleared hid, so positions off S stay 0.  One thread per active entry: one
// load round, no search.  Indices outside [0, i) are dropped; a repeated
// index writes the same value from each of its entries (same row, same x).
__global__ void __launch_bounds__(256) scatter_act_kernel(const int32_t* __restrict__ active, int n_active,
                                                          const int32_t* __restrict__ n_dev,
                                                          const float* __restrict__ gu, int kind,
                                                          float* __restrict__ hid, int64_t i_dim) {
    const int r = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (r >= active_count(n_active, n_dev)) return;
    const int o = active[r];
    const float2 g = *reinterpret_cast<const float2*>(gu + 2 * static_cast<int64_t>(r));
    if (o >= 0 && o < i_dim) hid[o] = act_pair(g.x, g.y, kind);
}

constexpr int DOWN_THREADS = 1024;
constexpr int DOWN_RG = DOWN_THREADS / 4;  // row groups per workgroup
constexpr int DOWN_BATCH = 6;              // rows per thread and load batch

// layout 1, Q4_K: workgroup u owns output unit u (64 columns: chunk u % 4 of
// super-block u / 4 of every row of D) over all active rows, so it writes its
// 64 outputs itself: no partial sums cross workgroups.  Thread t = 4 rg + p
// takes quarter p of the unit (16 of its 64 columns: p < 2 = low nibbles of
// qs bytes 16p .. +16, sub-block 2c; p >= 2 = high nibbles of bytes
// 16(p-2) .., sub-block 2c+1) of active rows rg, rg + DOWN_RG, ...  Rows go
// in batches of DOWN_BATCH per thread with every load of a batch issued
// before any use (indices and activations, then the weight blocks): two
// memory latencies per batch.  Partial sums meet in LDS and are added in a
// fixed order (deterministic).
__global__ void __launch_bounds__(DOWN_THREADS) down_rows_q4k_kernel(
    const uint8_t* __restrict__ d, int64_t rb, int64_t i_dim, const int32_t* __restrict__ active,
    int n_bound, const int32_t* __restrict__ n_dev, const float* __restrict__ gu, int kind, const float* resid,
    float* y) {
    __shared__ float red[DOWN_RG][65];
    const int n_active = active_count(n_bound, n_dev);
    __shared__ float red2[DOWN_THREADS / 64][64];
    const int u = blockIdx.x;
    const int t = threadIdx.x, rg = t >> 2, p = t & 3;
    const int sb = u >> 2, c = u & 3;
    const int jsub = 2 * c + (p >= 2 ? 1 : 0);
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; e++) acc[e] = 0.f;
    float bacc = 0.f;
    constexpr int STRIDE = DOWN_RG;
    for (int r0 = rg; r0 < n_active; r0 += DOWN_BATCH * STRIDE) {
        int nr[DOWN_BATCH];
        float2 gv[DOWN_BATCH];
#pragma unroll
        for (int b = 0; b < DOWN_BATCH; b++) {
            const int r = r0 + b * STRIDE;
            const int rc = r < n_active ? r : 0;
            nr[b] = active[rc];
            gv[b] = *reinterpret_cast<const float2*>(gu + 2 * rc);
        }
        __builtin_amdgcn_sched_barrier(0);  // all index / activation loads first
        float hid[DOWN_BATCH];
#pragma unroll
        for (int b = 0; b < DOWN_BATCH; b++) {
            const int v = nr[b];
            nr[b] = v < 0 ? 0 : (v >= i_dim ? static_cast<int>(i_dim) - 1 : v);
            hid[b] = r0 + b * STRIDE < n_active ? act_pair(gv[b].x, gv[b].y, kind) : 0.f;
        }
        // native vector type: arrays of HIP's uint4 struct can land in scratch
        u32x4 hdv[DOWN_BATCH], qv[DOWN_BATCH];
#pragma unroll
        for (int b = 0; b < DOWN_BATCH; b++) {
            const uint8_t* blk = d + static_cast<int64_t>(nr[b]) * rb + static_cast<int64_t>(sb) * 144;
            hdv[b] = *reinterpret_cast<const u32x4*>(blk);
            qv[b] = *reinterpret_cast<const u32x4*>(blk + 16 + 32 * c + 16 * (p & 1));
        }
        __builtin_amdgcn_sched_barrier(0);  // all weight loads before the math
#pragma unroll
        for (int b = 0; b < DOWN_BATCH; b++) {
            const u32x4 hd = hdv[b], q = qv[b];
            uint8_t s8[12];
            const uint32_t sw[3] = {hd.y, hd.z, hd.w};
#pragma unroll
            for (int k = 0; k < 12; k++) s8[k] = static_cast<uint8_t>(sw[k >> 2] >> (8 * (k & 3)));
            float sc, m;
            if (jsub < 4) {
                sc = static_cast<float>(s8[jsub] & 63);
                m = static_cast<float>(s8[jsub + 4] & 63);
            } else {
                sc = static_cast<float>((s8[jsub + 4] & 0xF) | ((s8[jsub - 4] >> 6) << 4));
                m = static_cast<float>((s8[jsub + 4] >> 4) | ((s8[jsub] >> 6) << 4));
            }
            const float a = hid[b] * (f16lo(hd.x) * sc);
            bacc += hid[b] * (f16hi(hd.x) * m);
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
            const int shift = p >= 2 ? 4 : 0;
#pragma unroll
            for (int e = 0; e < 16; e++)
                acc[e] += a * static_cast<float>((qw[e >> 2] >> (8 * (e & 3) + shift)) & 0xF);
        }
    }
#pragma unroll
    for (int e = 0; e < 16; e++) red[rg][16 * p + e] = acc[e] - bacc;
    __syncthreads();
    {  // thread t: column t % 64 over row groups 16 (t / 64) .. +16
        const int col = t & 63, g0 = (t >> 6) * 16;
        float sum = 0.f;
#pragma unroll
        for (int k = 0; k < 16; k++) sum += red[g0 + k][col];
        red2[t >> 6][col] = sum;
    }
    __syncthreads();
    if (t < 64) {
        float sum = 0.f;
#pragma unroll
        for (int k = 0; k < DOWN_THREADS / 64; k++) sum += red2[k][t];
        const int64_t col = 64 * static_cast<int64_t>(u) + t;
        y[col] = resid ? sum + resid[col] : sum;  // resid may be y: read before the write
    }
}

// ---- fused neuron-major path (one launch + a small reduction) ----------------
//
// For h <= 4096 (a row of h elements is one wave: lane = 64-element unit) the
// gate/up dot products and the down rows of an active neuron run in one
// wave: wave w of workgroup b takes neurons r = b * 8 NPW + w + 8 k, k <
// NPW.  All of its gate, up and D rows are requested at kernel start (their
// addresses need only the active indices), the workgroup encodes x into LDS
// as the GEMV does (gemv_core.hpp), then per neuron: g = gate . x and
// u = up . x with the integer unit dot products, one pair_sum for both,
// h = act(g, u), and lane u adds h * D[S_r, 64u .. 64u+63] (decoded: d*sc*q -
// dmin*m) to its 64 partial outputs.  The 8 waves' partials meet in LDS and
// the workgroup writes one partial y (4096 floats); sparse_reduce_kernel adds
// the workgroups' partials in a fixed order (deterministic).  The partials
// go through LDS in 16-byte accesses: 32 LDS instructions per thread where
// 4-byte accesses take 128.
// Neurons per wave of this row-split kernel: 1 (VB_SPARSE_NPW=1) or 2
// (VB_SPARSE_NPW=2; 1 measured faster: more workgroups, less serial work per
// wave, at twice the partial sums).  The default is the column-split kernel
// below.
constexpr int FUSED_STRIDE = 4096;        // floats per partial y (h <= 4096)
// LDS row of one lane's 64 partials (floats): 16-byte writes of 16 lanes at
// a pitch of 68 floats (4 mod 64 dwords) fall on distinct banks
constexpr int FUSED_RED_PITCH = 68;

__device__ __forceinline__ float pair_sum(float a0, float a1) {
    // lane 31: total of a0, lane 63: total of a1 (see gemv.hip)
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(a0), __float_as_int(a1), false, false);
    float v = __int_as_float(sw[0]) + __int_as_float(sw[1]);
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    v += dpp_rows_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
    return v;
}

// yp[e] += h * (d * sc_j) * q_e for the 64 elements of a Q4_K unit (e < 32:
// low nibbles, sub-block 2c; e >= 32: high nibbles, sub-block 2c+1); the
// min terms h * dmin * m_j go to mb0 / mb1 (subtracted once at the end).
// Scale selection as in the unit dot product (get_scale_min_k4,
// cpp/src/dequant.cpp:258-266).
__device__ __forceinline__ void unit_axpy(const gemvc::Q4KUnit& v, const gemvc::Q4KSel& q, float h, float* yp,
                                          float& mb0, float& mb1) {
    using gemvc::quad_bcast;
    const uint32_t hx = quad_bcast<0>(v.hw);
    const uint32_t A = quad_bcast<1>(v.hw), B = quad_bcast<2>(v.hw), C = quad_bcast<3>(v.hw);
    const uint32_t SC = (((q.hi ? C : A) >> q.sh) & q.m1) | ((A >> q.sh2) & q.m2);
    const uint32_t M = (((q.hi ? C : B) >> q.shm) & q.m1) | ((B >> q.sh2) & q.m2);
    const float hd = h * f16lo(hx), hm = h * f16hi(hx);
    const float a0 = hd * static_cast<float>(SC & 0xFFu), a1 = hd * static_cast<float>((SC >> 8) & 0xFFu);
    mb0 += hm * static_cast<float>(M & 0xFFu);
    mb1 += hm * static_cast<float>((M >> 8) & 0xFFu);
    const uint32_t qd[8] = {v.qa.x, v.qa.y, v.qa.z, v.qa.w, v.qb.x, v.qb.y, v.qb.z, v.qb.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t lo = qd[i] & 0x0F0F0F0Fu, hi = (qd[i] >> 4) & 0x0F0F0F0Fu;
        yp[4 * i + 0] += a0 * static_cast<float>(lo & 0xFFu);
        yp[4 * i + 1] += a0 * static_cast<float>((lo >> 8) & 0xFFu);
        yp[4 * i + 2] += a0 * static_cast<float>((lo >> 16) & 0xFFu);
        yp[4 * i + 3] += a0 * static_cast<float>(lo >> 24);
        yp[32 + 4 * i + 0] += a1 * static_cast<float>(hi & 0xFFu);
        yp[32 + 4 * i + 1] += a1 * static_cast<float>((hi >> 8) & 0xFFu);
        yp[32 + 4 * i + 2] += a1 * static_cast<float>((hi >> 16) & 0xFFu);
        yp[32 + 4 * i + 3] += a1 * static_cast<float>(hi >> 24);
    }
}

template <int NPW, bool NORM>
__global__ void __launch_bounds__(512) sparse_fused_q4k_kernel(
    const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu, const uint8_t* __restrict__ wd, int64_t rb,
    int64_t i_dim, const float* __restrict__ x, const int32_t* __restrict__ active, int n_bound,
    const int32_t* __restrict__ n_dev, int kind, float* __restrict__ partial, int units, int slots,
    const float* __restrict__ norm_w, float eps) {
    using namespace gemvc;
    // with a device count, workgroups past it do nothing (the reduction reads
    // the same count and never their partials)
    const int n_active = active_count(n_bound, n_dev);
    if (static_cast<int>(blockIdx.x) * (8 * NPW) >= n_active) return;
    // the x encoding (slots x 11 uint4), later the 8 waves' partials
    __shared__ uint4 lds[8 * 64 * FUSED_RED_PITCH / 4];  // 139,264 B
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const bool valid = lane < units;
    // idle lanes load a real unit (discarded); u % 4 == lane % 4 keeps every
    // quad on one super-block (units is a multiple of 4)
    const int uc = valid ? lane : units - 4 + (lane & 3);
    const Q4KSel usel = make_unit_sel<TYPE_Q4_K>(uc);
    const int rbase = static_cast<int>(blockIdx.x) * (8 * NPW) + wave;

    int nidx[NPW];
    bool nval[NPW];
#pragma unroll
    for (int k = 0; k < NPW; k++) {
        const int r = rbase + 8 * k;
        nval[k] = r < n_active;
        int v = active[nval[k] ? r : 0];
        v = v < 0 ? 0 : (v >= i_dim ? static_cast<int>(i_dim) - 1 : v);  // never read outside the tensors
        nidx[k] = __builtin_amdgcn_readfirstlane(v);
    }
    // x first, then every weight row of the wave, then the encode (which
    // waits for x only)
    XTasks xt;
    [[maybe_unused]] XTasks nt;  // norm weights of the same tasks (NORM)
    const bool x_in_regs = slots * 8 <= XT_MAX * static_cast<int>(blockDim.x);
    if (x_in_regs) prefetch_x<TYPE_Q4_K>(x, units, slots, xt);
    if constexpr (NORM) {
        if (x_in_regs) prefetch_x<TYPE_Q4_K>(norm_w, units, slots, nt);
    }
    __builtin_amdgcn_sched_barrier(0);
    Q4KUnit vg[NPW], vu[NPW], vd[NPW];
#pragma unroll
    for (int k = 0; k < NPW; k++) {
        const int64_t off = static_cast<int64_t>(nidx[k]) * rb;
        load_unit(wg + off, uc, vg[k]);
        load_unit(wu + off, uc, vu[k]);
        load_unit(wd + off, uc, vd[k]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
        // RMSNorm inside the encode; the reduction's scratch sits past the
        // x encoding and is read before the barrier after the encode
        float* scratch = reinterpret_cast<float*>(lds + XQ_QUADS * slots);
        const float ss = wg_sum_fixed(x_in_regs ? sumsq_tasks(units, slots, xt) : sumsq_loop(x, units * 64),
                                      scratch);
        const float rinv = rms_inv(ss, units * 64, eps);
        if (x_in_regs) {
            scale_tasks(xt, nt, rinv);
            encode_x_regs<TYPE_Q4_K>(units, slots, xt, lds);
        } else {
            encode_x_loop_norm<TYPE_Q4_K>(x, norm_w, rinv, units, slots, lds);
        }
    } else {
        if (x_in_regs)
            encode_x_regs<TYPE_Q4_K>(units, slots, xt, lds);
        else
            encode_x_loop<TYPE_Q4_K>(x, units, slots, lds);
    }
    __syncthreads();
    XSlice xs;
    read_xslice(lds, slots, valid ? lane : 0, xs);

    float yp[64];
#pragma unroll
    for (int e = 0; e < 64; e++) yp[e] = 0.f;
    float mb0 = 0.f, mb1 = 0.f;
#pragma unroll
    for (int k = 0; k < NPW; k++) {
        const float g = valid ? unit_dot(vg[k], xs, usel) : 0.f;
        const float u = valid ? unit_dot(vu[k], xs, usel) : 0.f;
        const float t = pair_sum(g, u);
        const float gt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 31));
        const float ut = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 63));
        const float h = nval[k] ? act_pair(gt, ut, kind) : 0.f;
        unit_axpy(vd[k], usel, h, yp, mb0, mb1);
    }
    // the 8 waves' partials (lanes >= units hold junk and are never read)
    __syncthreads();  // the x encoding is dead: LDS now holds the partials
    // row (wave, lane): the lane's 64 partials (columns 64 lane + e), four per
    // 16-byte write
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float m = i < 8 ? mb0 : mb1;
        *reinterpret_cast<float4*>(red + (wave * 64 + lane) * FUSED_RED_PITCH + 4 * i) =
            make_float4(yp[4 * i] - m, yp[4 * i + 1] - m, yp[4 * i + 2] - m, yp[4 * i + 3] - m);
    }
    __syncthreads();
    // column quad q = (unit q / 16, columns 4 (q % 16) ..): the 8 waves' rows
    // added in wave order, one 16-byte store
    float* out = partial + static_cast<int64_t>(blockIdx.x) * FUSED_STRIDE;
    const int nquads = 16 * units;
    for (int q = static_cast<int>(threadIdx.x); q < nquads; q += static_cast<int>(blockDim.x)) {
        const int l = q >> 4, e0 = 4 * (q & 15);
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const float4 v = *reinterpret_cast<const float4*>(red + (w * 64 + l) * FUSED_RED_PITCH + e0);
            sum.x += v.x;
            sum.y += v.y;
            sum.z += v.z;
            sum.w += v.w;
        }
        *reinterpret_cast<float4*>(out + 64 * l + e0) = sum;
    }
}

// Column-split variant (the default): each wave still computes one neuron's
// gate and up dot products, but the down rows are split by output columns.
// Once the 8 h values meet in LDS, wave w adds h_r * D[S_r, 512 w .. 512 w +
// 511] for the workgroup's 8 neurons r and writes its 512 columns of the
// partial straight from registers: no LDS sum of 8 partial vectors.  Wave
// w's slice of a down row is 2 super-blocks (288 B); the 8 slices are read as
// contiguous 16-byte pieces (requested at kernel start with the gate and up
// rows) and staged in the wave's LDS area.  Lane L takes unit 8 w + L / 8,
// qs bytes 4 (L % 8) .. + 3 of it: elements 4 (L % 8) + j (low nibbles,
// sub-block 2c) and 32 + 4 (L % 8) + j (high nibbles, 2c + 1).
constexpr int COLS_SLICE = 288;   // bytes of a wave's down-row slice (8 units)
constexpr int COLS_PIECES = 8 * COLS_SLICE / 16;  // 144 16-byte pieces per wave (8 rows)

template <bool NORM>
__global__ void __launch_bounds__(512) sparse_fused_cols_kernel(
    const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu, const uint8_t* __restrict__ wd, int64_t rb,
    int64_t i_dim, const float* __restrict__ x, const int32_t* __restrict__ active, int n_bound,
    const int32_t* __restrict__ n_dev, int kind, float* __restrict__ partial, int units, int slots,
    const float* __restrict__ norm_w, float eps) {
    using namespace gemvc;
    const int n_active = active_count(n_bound, n_dev);
    if (static_cast<int>(blockIdx.x) * 8 >= n_active) return;
    __shared__ uint4 lds[XQ_QUADS * 64 + 16];      // the x encoding (slots <= 64) and a norm scratch
    __shared__ uint4 dst[8][COLS_PIECES];          // the waves' down-row slices
    __shared__ float hbuf[8];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const bool valid = lane < units;
    const int uc = valid ? lane : units - 4 + (lane & 3);
    const Q4KSel usel = make_unit_sel<TYPE_Q4_K>(uc);
    const int r0 = static_cast<int>(blockIdx.x) * 8;

    // the workgroup's 8 neurons (clamped indices: never read outside the tensors)
    auto neuron = [&](int r) {
        int v = active[r < n_active ? r : 0];
        v = v < 0 ? 0 : (v >= i_dim ? static_cast<int>(i_dim) - 1 : v);
        return v;
    };
    // the 8 indices in one round trip: lanes 0-7 load, the wave reads them
    // out (wave-uniform, in scalar registers) before any other load is issued
    const int nl = neuron(r0 + (lane & 7));
    int nid[8];
#pragma unroll
    for (int k = 0; k < 8; k++) nid[k] = __builtin_amdgcn_readlane(nl, k);
    const int nidx = __builtin_amdgcn_readlane(nl, wave);
    const bool nval = r0 + wave < n_active;
    // slice pieces of this lane: p = lane + 64 i < 144, row p / 18, part p % 18
    // (parts past the row, for h < 4096, read the row's start and are never used)
    int64_t poff[3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const int p = lane + 64 * i < COLS_PIECES ? lane + 64 * i : lane;
        const int row = p / 18, part = p - 18 * row;
        int v = nid[0];
#pragma unroll
        for (int k = 1; k < 8; k++) v = row == k ? nid[k] : v;
        const int64_t b = static_cast<int64_t>(COLS_SLICE) * wave + 16 * part;
        poff[i] = static_cast<int64_t>(v) * rb + (b + 16 <= rb ? b : 0);
    }

    XTasks xt;
    [[maybe_unused]] XTasks nt;
    const bool x_in_regs = slots * 8 <= XT_MAX * static_cast<int>(blockDim.x);
    if (x_in_regs) prefetch_x<TYPE_Q4_K>(x, units, slots, xt);
    if constexpr (NORM) {
        if (x_in_regs) prefetch_x<TYPE_Q4_K>(norm_w, units, slots, nt);
    }
    __builtin_amdgcn_sched_barrier(0);
    Q4KUnit vg, vu;
    {
        const int64_t off = static_cast<int64_t>(nidx) * rb;
        load_unit(wg + off, uc, vg);
        load_unit(wu + off, uc, vu);
    }
    const uint4 dv0 = *reinterpret_cast<const uint4*>(wd + poff[0]);
    const uint4 dv1 = *reinterpret_cast<const uint4*>(wd + poff[1]);
    const uint4 dv2 = *reinterpret_cast<const uint4*>(wd + poff[2]);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
        float* scratch = reinterpret_cast<float*>(lds + XQ_QUADS * slots);
        const float ss = wg_sum_fixed(x_in_regs ? sumsq_tasks(units, slots, xt) : sumsq_loop(x, units * 64),
                                      scratch);
        const float rinv = rms_inv(ss, units * 64, eps);
        if (x_in_regs) {
            scale_tasks(xt, nt, rinv);
            encode_x_regs<TYPE_Q4_K>(units, slots, xt, lds);
        } else {
            encode_x_loop_norm<TYPE_Q4_K>(x, norm_w, rinv, units, slots, lds);
        }
    } else {
        if (x_in_regs)
            encode_x_regs<TYPE_Q4_K>(units, slots, xt, lds);
        else
            encode_x_loop<TYPE_Q4_K>(x, units, slots, lds);
    }
    __syncthreads();
    XSlice xs;
    read_xslice(lds, slots, valid ? lane : 0, xs);

    // this wave's neuron: h into LDS; the slices into the wave's LDS area
    {
        const float g = valid ? unit_dot(vg, xs, usel) : 0.f;
        const float u = valid ? unit_dot(vu, xs, usel) : 0.f;
        const float t = pair_sum(g, u);
        const float gt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 31));
        const float ut = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 63));
        if (lane == 0) hbuf[wave] = nval ? act_pair(gt, ut, kind) : 0.f;
    }
    dst[wave][lane] = dv0;
    dst[wave][64 + lane] = dv1;
    if (128 + lane < COLS_PIECES) dst[wave][128 + lane] = dv2;
    __syncthreads();

    // the wave's 512 columns: unit 8 w + L / 8 of every neuron's row
    const int ul = lane >> 3, i8 = lane & 7;
    const int u = 8 * wave + ul;
    const Q4KSel csel = make_unit_sel<TYPE_Q4_K>(ul & 3);
    const uint8_t* sb = reinterpret_cast<const uint8_t*>(dst[wave]) + 144 * (ul >> 2);
    float yp[8];
#pragma unroll
    for (int e = 0; e < 8; e++) yp[e] = 0.f;
    float mb0 = 0.f, mb1 = 0.f;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const float h = hbuf[r];
        const uint8_t* rp = sb + COLS_SLICE * r;
        const uint4 hd = *reinterpret_cast<const uint4*>(rp);
        const uint32_t q = *reinterpret_cast<const uint32_t*>(rp + 16 + 32 * (ul & 3) + 4 * i8);
        const uint32_t A = hd.y, B = hd.z, C = hd.w;
        const uint32_t SC = (((csel.hi ? C : A) >> csel.sh) & csel.m1) | ((A >> csel.sh2) & csel.m2);
        const uint32_t M = (((csel.hi ? C : B) >> csel.shm) & csel.m1) | ((B >> csel.sh2) & csel.m2);
        const float hdd = h * f16lo(hd.x), hm = h * f16hi(hd.x);
        const float a0 = hdd * static_cast<float>(SC & 0xFFu), a1 = hdd * static_cast<float>((SC >> 8) & 0xFFu);
        mb0 += hm * static_cast<float>(M & 0xFFu);
        mb1 += hm * static_cast<float>((M >> 8) & 0xFFu);
        const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            yp[j] += a0 * static_cast<float>((lo >> (8 * j)) & 0xFFu);
            yp[4 + j] += a1 * static_cast<float>((hi >> (8 * j)) & 0xFFu);
        }
    }
    if (u < units) {
        float* out = partial + static_cast<int64_t>(blockIdx.x) * FUSED_STRIDE + 64 * u + 4 * i8;
        *reinterpret_cast<float4*>(out) = make_float4(yp[0] - mb0, yp[1] - mb0, yp[2] - mb0, yp[3] - mb0);
        *reinterpret_cast<float4*>(out + 32) = make_float4(yp[4] - mb1, yp[5] - mb1, yp[6] - mb1, yp[7] - mb1);
    }
}

// y[64 b + c] = sum over the nblk partials in order; thread t: column c = t %
// 64, partials t / 64, t / 64 + 16, ...
__global__ void __launch_bounds__(1024) sparse_reduce_kernel(const float* __restrict__ partial, int nblk_bound,
                                                             const int32_t* __restrict__ n_dev, int per_blk,
                                                             const float* resid, float* y) {
    __shared__ float red[16][64];
    // partials of the workgroups that ran (all of them without a device count)
    const int nblk = n_dev ? (active_count(nblk_bound * per_blk, n_dev) + per_blk - 1) / per_blk : nblk_bound;
    const int c = threadIdx.x & 63, bg = threadIdx.x >> 6;
    const int col = static_cast<int>(blockIdx.x) * 64 + c;
    // every load of a round of 16 (up to 256 partials: one round at config
    // shapes) is issued before the adds, which run in partial order
    // bg, bg + 16, ... (fixed)
    float sum = 0.f;
    for (int b0 = bg; b0 < nblk; b0 += 16 * 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int b = b0 + 16 * k;
            v[k] = partial[static_cast<int64_t>(b < nblk ? b : bg) * FUSED_STRIDE + col];
        }
#pragma unroll
        for (int k = 0; k < 16; k++) sum += b0 + 16 * k < nblk ? v[k] : 0.f;
    }
    red[bg][c] = sum;
    __syncthreads();
    if (threadIdx.x < 64) {
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 16; k++) t += red[k][c];
        y[col] = resid ? t + resid[col] : t;  // resid may be y: read before the write
    }
}

// ---- top-k indices (single workgroup radix select) ---------------------------

// Ascending key == ascending float; -0.0 and +0.0 share a key, as they
// compare equal (numpy's orderings, which the top-k rules follow, treat them
// as ties).
__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t b = __float_as_uint(f);
    b = b == 0x80000000u ? 0u : b;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The k-th largest key of v[0..n) (1 <= k <= n) by a 4-pass radix select
// over LDS histograms, and how many elements equal to it belong to the top k
// (ties go to the lowest indices).  Every thread of the workgroup calls it.
struct KthKey {
    uint32_t key;
    int ties;
};

__device__ KthKey radix_kth(const float* __restrict__ v, int n, int k) {
    __shared__ int hist[256];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_remaining;
    const int tid = threadIdx.x;
    if (tid == 0) {
        s_prefix = 0;
        s_mask = 0;
        s_remaining = k;
    }
    for (int pass = 3; pass >= 0; pass--) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix, mask = s_mask;
        for (int i = tid; i < n; i += blockDim.x) {
            const uint32_t key = order_key(v[i]);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> (8 * pass)) & 255], 1);
        }
        __syncthreads();
        if (tid == 0) {
            int rem = s_remaining, cum = 0, b = 255;
            for (; b > 0; b--) {
                if (cum + hist[b] >= rem) break;
                cum += hist[b];
            }
            s_prefix = prefix | (static_cast<uint32_t>(b) << (8 * pass));
            s_mask = mask | (255u << (8 * pass));
            s_remaining = rem - cum;
        }
        __syncthreads();
    }
    KthKey r;
    r.key = s_prefix;
    r.ties = s_remaining;
    __syncthreads();  // every thread has read the result before a next call resets it
    return r;
}

// Exclusive rank of this thread's flag among the flags of all threads before
// it in thread order, plus *base; then *base advances by the workgroup's
// count.  wcnt: one int per wave.  Every thread calls it.
__device__ int block_rank(bool f, int* wcnt, int* base) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = static_cast<int>(blockDim.x >> 6);
    const uint64_t b = __ballot(f);
    if (lane == 0) wcnt[wave] = __popcll(b);
    __syncthreads();
    int r = *base + __popcll(b & ((1ull << lane) - 1ull));
    int tot = 0;
    for (int w = 0; w < nw; w++) {
        tot += wcnt[w];
        if (w < wave) r += wcnt[w];
    }
    __syncthreads();  // every thread has read *base and wcnt
    if (threadIdx.x == 0) *base += tot;
    return r;
}

__global__ void __launch_bounds__(1024) topk_kernel(const float* __restrict__ v, int n, int k,
                                                    int32_t* __restrict__ out) {
    __shared__ int hist[256];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_remaining;
    __shared__ int wave_cnt[2][16];
    __shared__ int s_base[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) {
        s_prefix = 0;
        s_mask = 0;
        s_remaining = k;
    }
    for (int pass = 3; pass >= 0; pass--) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix, mask = s_mask;
        for (int i = tid; i < n; i += blockDim.x) {
            const uint32_t key = order_key(v[i]);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> (8 * pass)) & 255], 1);
        }
        __syncthreads();
        if (tid == 0) {
            int rem = s_remaining, cum = 0, b = 255;
            for (; b > 0; b--) {
                if (cum + hist[b] >= rem) break;
                cum += hist[b];
            }
            s_prefix = prefix | (static_cast<uint32_t>(b) << (8 * pass));
            s_mask = mask | (255u << (8 * pass));
            s_remaining = rem - cum;
        }
        __syncthreads();
    }
    const uint32_t kth = s_prefix;
    const int ties = s_remaining;  // elements equal to kth to take
    if (tid == 0) {
        s_base[0] = 0;  // selected so far
        s_base[1] = 0;  // equal-to-kth seen so far
    }
    __syncthreads();
    for (int i0 = 0; i0 < n; i0 += blockDim.x) {
        const int i = i0 + tid;
        const uint32_t key = i < n ? order_key(v[i]) : 0u;
        const bool eq = i < n && key == kth;
        const bool gt = i < n && key > kth;
        const uint64_t beq = __ballot(eq);
        const int eq_rank_w = __popcll(beq & ((1ull << lane) - 1ull));
        if (lane == 0) wave_cnt[1][wave] = __popcll(beq);
        __syncthreads();
        int eq_before = s_base[1];
        for (int w = 0; w < wave; w++) eq_before += wave_cnt[1][w];
        const bool sel = gt || (eq && eq_before + eq_rank_w < ties);
        const uint64_t bsel = __ballot(sel);
        if (lane == 0) wave_cnt[0][wave] = __popcll(bsel);
        __syncthreads();
        int pos = s_base[0] + __popcll(bsel & ((1ull << lane) - 1ull));
        for (int w = 0; w < wave; w++) pos += wave_cnt[0][w];
        if (sel && pos < k) out[pos] = i;
        __syncthreads();
        if (tid == 0) {
            int a = 0, b = 0;
            for (int w = 0; w < static_cast<int>(blockDim.x >> 6); w++) {
                a += wave_cnt[0][w];
                b += wave_cnt[1][w];
            }
            s_base[0] += a;
            s_base[1] += b;
        }
        __syncthreads();
    }
}

// ---- EMA neuron predictor (EMANeuronPredictor, vibeblade/sparse.py:431-650) ----

// probs = alpha * mask + (1 - alpha) * probs, rounded as the reference's
// float32 numpy expression (sparse.py:510-512): the product (1 - alpha) * p is
// rounded, alpha * mask is exact (mask is 0 or 1), then one rounded add.
// Contraction into a fused multiply-add is switched off (hipcc contracts by
// default, and an unrounded product changes the result after a few steps),
// so the result is bit-identical.
__global__ void __launch_bounds__(256) ema_update_kernel(float* __restrict__ probs, const uint8_t* __restrict__ mask,
                                                         int64_t n, float alpha, float beta) {
#pragma clang fp contract(off)
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float t = beta * probs[i];
    probs[i] = (mask[i] ? alpha : 0.f) + t;
}

constexpr int PRED_WARM = 1;      // more than 5 updates: select by EMA probability
constexpr int PRED_GATE = 2;      // gate values given
constexpr int PRED_COMBINED = 4;  // predict_combined: EMA prediction | gate top-k

// One workgroup.  The selected set (sparse.py:534-569, :571-598):
//   warm:                    top-k(probs) | {probs >= threshold}
//                            (equal to the reference's threshold set topped
//                            up with the most probable neurons to k)
//   cold, gate, !combined:   top-k(gate)
//   cold otherwise:          neurons 0 .. k-1
//   combined:                the above (without gate) | top-k(gate)
// Top-k ties go to the lowest indices.  Writes mask (n bytes), the selected
// indices in ascending order (active, room for n) and their count.
__global__ void __launch_bounds__(1024) ema_predict_kernel(const float* __restrict__ probs,
                                                           const float* __restrict__ gate, int n, int k,
                                                           float threshold, int flags,
                                                           uint8_t* __restrict__ mask, int32_t* __restrict__ active,
                                                           int32_t* __restrict__ count) {
    __shared__ int wcnt[3][16];
    __shared__ int base[3];
    const bool warm = flags & PRED_WARM, has_gate = flags & PRED_GATE, combined = flags & PRED_COMBINED;
    const bool use_p = warm;                               // top-k over probs
    const bool use_g = has_gate && (combined || !warm);    // top-k over gate
    KthKey kp{0u, 0}, kg{0u, 0};
    if (use_p) kp = radix_kth(probs, n, k);
    if (use_g) kg = radix_kth(gate, n, k);
    if (threadIdx.x < 3) base[threadIdx.x] = 0;
    __syncthreads();
    for (int i0 = 0; i0 < n; i0 += blockDim.x) {
        const int i = i0 + static_cast<int>(threadIdx.x);
        const bool in = i < n;
        const float pv = in && use_p ? probs[i] : 0.f;
        const float gv = in && use_g ? gate[i] : 0.f;
        const uint32_t pk = order_key(pv), gk = order_key(gv);
        const bool peq = in && use_p && pk == kp.key, geq = in && use_g && gk == kg.key;
        const int prank = block_rank(peq, wcnt[0], &base[0]);
        const int grank = block_rank(geq, wcnt[1], &base[1]);
        const bool ptop = in && use_p && (pk > kp.key || (peq && prank < kp.ties));
        const bool gtop = in && use_g && (gk > kg.key || (geq && grank < kg.ties));
        bool sel;
        if (warm)
            sel = ptop || (in && pv >= threshold);
        else if (has_gate && !combined)
            sel = gtop;
        else
            sel = in && i < k;
        if (combined) sel = sel || gtop;
        const int pos = block_rank(sel, wcnt[2], &base[2]);
        if (in) {
            mask[i] = sel ? 1 : 0;
            if (sel) active[pos] = i;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) *count = base[2];
}

// ---- register-resident predictor (n <= 1024 * PER) ---------------------------
//
// Thread t holds elements e = j * 1024 + t, slots j < PER: loads and mask
// stores are coalesced, and index order is slot-major.  A rank in index
// order = the count of flags in earlier (slot, wave) cells + the in-wave
// rank; the cells' counts go through LDS and wave 0 turns them into
// exclusive prefixes (two barriers for up to two flag sets at once).

// Index-order ranks of the flagged elements of two flag sets (fa, fb: bit j
// = this thread's slot j).  Phase 1: each (slot, wave) cell's count into LDS;
// wave 0 turns each set's cells into exclusive prefixes; phase 2 recomputes
// the in-wave ranks (ballots are cheap; nothing is held across barriers) and
// hands rank(j) to `use(set, j, rank)`.  cells: PER * 32 + 2 ints of LDS.
// Returns the totals in *ta / *tb.  Every thread calls it.
template <int PER, class Use>
__device__ void slot_ranks(uint32_t fa, uint32_t fb, int* cells, int* ta, int* tb, Use use) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const uint64_t ba = __ballot((fa >> j) & 1u), bb = __ballot((fb >> j) & 1u);
        if (lane == 0) {
            cells[j * 16 + wave] = __popcll(ba);
            cells[PER * 16 + j * 16 + wave] = __popcll(bb);
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) {  // wave 0: exclusive prefix over each set's PER * 16 cells, in order
        constexpr int PL = PER * 16 / 64;  // cells per lane
#pragma unroll
        for (int set = 0; set < 2; set++) {
            int* c = cells + set * PER * 16;
            int v[PL], sum = 0;
#pragma unroll
            for (int q = 0; q < PL; q++) {
                v[q] = c[lane * PL + q];
                sum += v[q];
            }
            int inc = sum;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int t = __shfl_up(inc, d, 64);
                if (lane >= d) inc += t;
            }
            int run = inc - sum;
#pragma unroll
            for (int q = 0; q < PL; q++) {
                c[lane * PL + q] = run;
                run += v[q];
            }
            if (lane == 63) cells[PER * 32 + set] = inc;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const uint64_t ba = __ballot((fa >> j) & 1u), bb = __ballot((fb >> j) & 1u);
        if ((fa >> j) & 1u) use(0, j, cells[j * 16 + wave] + __popcll(ba & lt));
        if ((fb >> j) & 1u) use(1, j, cells[PER * 16 + j * 16 + wave] + __popcll(bb & lt));
    }
    *ta = cells[PER * 32];
    *tb = cells[PER * 32 + 1];
    __syncthreads();  // cells are free for the next call
}

// k-th largest key among all threads' values (valid slots: bit j of vmask)
// and how many keys equal to it are inside the top k.  Three passes over
// digits of 11, 11 and 10 bits (2048-bin LDS histogram, one atomic per live
// key: measured faster than aggregating equal digits first); wave 0 finds
// the digit, lane l scanning bins 32 l .. 32 l + 31.
template <int PER>
__device__ KthKey radix_kth_regs(const float* vals, uint32_t vmask, int k) {
    __shared__ int hist[2048];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_remaining;
    if (threadIdx.x == 0) {
        s_prefix = 0;
        s_mask = 0;
        s_remaining = k;
    }
    constexpr int kShift[3] = {21, 10, 0};
    constexpr int kBits[3] = {11, 11, 10};
#pragma unroll
    for (int pass = 0; pass < 3; pass++) {
        const int sh = kShift[pass];
        const uint32_t dmask = (1u << kBits[pass]) - 1u;
        for (int b = threadIdx.x; b < 2048; b += blockDim.x) hist[b] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix, mask = s_mask;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const uint32_t key = order_key(vals[j * 1024 + static_cast<int>(threadIdx.x)]);
            if (((vmask >> j) & 1u) && (key & mask) == prefix) atomicAdd(&hist[(key >> sh) & dmask], 1);
        }
        __syncthreads();
        if (threadIdx.x < 64) {  // wave 0: lane l holds bins 32 l .. 32 l + 31
            const int l = threadIdx.x;
            int mine = 0;
            for (int b = 0; b < 32; b++) mine += hist[32 * l + b];
            int suf = mine;  // sum over lanes >= l
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int t = __shfl_down(suf, d, 64);
                if (l + d < 64) suf += t;
            }
            const int rem = s_remaining;
            int cum = suf - mine;  // keys in higher bins
            if (cum < rem && suf >= rem) {  // the digit is in this lane's bins
                for (int b = 31; b >= 0; b--) {
                    const int h = hist[32 * l + b];
                    if (cum + h >= rem) {
                        s_prefix = prefix | (static_cast<uint32_t>(32 * l + b) << sh);
                        s_mask = mask | (dmask << sh);
                        s_remaining = rem - cum;
                        break;
                    }
                    cum += h;
                }
            }
        }
        __syncthreads();
    }
    KthKey r;
    r.key = s_prefix;
    r.ties = s_remaining;
    __syncthreads();
    return r;
}

template <int PER>  // PER <= 32 (a thread's flags fit one word)
__global__ void __launch_bounds__(1024) ema_predict_reg_kernel(const float* __restrict__ probs,
                                                               const float* __restrict__ gate, int n, int k,
                                                               float threshold, int flags,
                                                               uint8_t* __restrict__ mask,
                                                               int32_t* __restrict__ active,
                                                               int32_t* __restrict__ count) {
    // The values live in LDS (slot-major: thread t's slot j at j * 1024 + t,
    // conflict-free); registers hold only per-thread flag words.  The gate
    // array's space takes the active list once the selection is made.
    __shared__ int cells[PER * 32 + 2];
    __shared__ float vals_p[PER * 1024];
    __shared__ float vals_g[PER * 1024];
    __shared__ uint8_t mask_lds[PER * 1024];
    const bool warm = flags & PRED_WARM, has_gate = flags & PRED_GATE, combined = flags & PRED_COMBINED;
    const bool use_p = warm, use_g = has_gate && (combined || !warm);
    const int t = static_cast<int>(threadIdx.x);
    uint32_t vmask = 0, above = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = j * 1024 + t;
        const bool in = e < n;
        vmask |= (in ? 1u : 0u) << j;
        const float pv = use_p && in ? probs[e] : 0.f;
        vals_p[e] = pv;
        above |= (use_p && in && pv >= threshold ? 1u : 0u) << j;
        vals_g[e] = use_g && in ? gate[e] : 0.f;
    }
    __syncthreads();
    int ta = 0, tb = 0;
    auto none = [](int, int, int) {};
    // warm: when the threshold set holds k or more neurons it contains the
    // top k, and the selection is that set alone (no select needed)
    bool need_p = false;
    if (use_p) {
        slot_ranks<PER>(above, 0u, cells, &ta, &tb, none);  // the count only
        need_p = ta < k;
    }
    KthKey kp{0xFFFFFFFFu, 0}, kg{0xFFFFFFFFu, 0};
    if (need_p) kp = radix_kth_regs<PER>(vals_p, vmask, k);
    if (use_g) kg = radix_kth_regs<PER>(vals_g, vmask, k);
    // top-k membership, ties to the lowest indices: rank among equal keys
    uint32_t peq = 0, geq = 0, pgt = 0, ggt = 0;
    if (need_p || use_g) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const bool in = (vmask >> j) & 1u;
            const uint32_t kpj = order_key(vals_p[j * 1024 + t]), kgj = order_key(vals_g[j * 1024 + t]);
            peq |= (need_p && in && kpj == kp.key ? 1u : 0u) << j;
            pgt |= (need_p && in && kpj > kp.key ? 1u : 0u) << j;
            geq |= (use_g && in && kgj == kg.key ? 1u : 0u) << j;
            ggt |= (use_g && in && kgj > kg.key ? 1u : 0u) << j;
        }
    }
    uint32_t ptie = 0, gtie = 0;  // equal keys inside the top k
    if (need_p || use_g) {
        slot_ranks<PER>(peq, geq, cells, &ta, &tb, [&](int set, int j, int r) {
            if (set == 0 && r < kp.ties) ptie |= 1u << j;
            if (set == 1 && r < kg.ties) gtie |= 1u << j;
        });
    }
    const uint32_t ptop = pgt | ptie, gtop = ggt | gtie;
    uint32_t sel;
    if (warm)
        sel = ptop | above;
    else if (has_gate && !combined)
        sel = gtop;
    else {
        sel = 0;
#pragma unroll
        for (int j = 0; j < PER; j++) sel |= (((vmask >> j) & 1u) && j * 1024 + t < k ? 1u : 0u) << j;
    }
    if (combined) sel |= gtop;
    // mask and active list staged in LDS, then written with 16-byte stores
    int32_t* act_lds = reinterpret_cast<int32_t*>(vals_g);  // the gate values are dead
#pragma unroll
    for (int j = 0; j < PER; j++) mask_lds[j * 1024 + t] = (sel >> j) & 1u;
    slot_ranks<PER>(sel, 0u, cells, &ta, &tb, [&](int, int j, int r) { act_lds[r] = j * 1024 + t; });
    // (slot_ranks ends with a barrier: mask_lds and act_lds are complete)
    const bool mvec = (reinterpret_cast<uintptr_t>(mask) & 15) == 0;
    for (int e = 16 * t; e < n; e += 16 * 1024) {
        if (mvec && e + 16 <= n)
            *reinterpret_cast<uint4*>(mask + e) = *reinterpret_cast<const uint4*>(mask_lds + e);
        else
            for (int q = e; q < e + 16 && q < n; q++) mask[q] = mask_lds[q];
    }
    const bool avec = (reinterpret_cast<uintptr_t>(active) & 15) == 0;
    for (int e = 4 * t; e < ta; e += 4 * 1024) {
        if (avec && e + 4 <= ta)
            *reinterpret_cast<int4*>(active + e) = *reinterpret_cast<const int4*>(act_lds + e);
        else
            for (int q = e; q < e + 4 && q < ta; q++) active[q] = act_lds[q];
    }
    if (t == 0) *count = ta;
}

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

struct SparseWs {
    size_t gu, hid, xn, total;
};

// The fused layout-1 path (h <= 4096) takes ceil(n_active / (8 * neurons per
// wave)) partial outputs of FUSED_STRIDE floats; the other paths take the gate/up
// results (and the dense hidden vector for layout 0).
bool fused_path(int64_t h, int32_t layout) {
    if (layout != 1 || h > 4096) return false;
    return knobs().sparse_fused;
}

SparseWs sparse_ws(int64_t h, int64_t i, int32_t n_active, int32_t layout) {
    SparseWs w;
    w.gu = 0;
    w.hid = align256(static_cast<size_t>(2 * (n_active > 0 ? n_active : 1)) * sizeof(float));
    size_t off = w.hid + (layout == 0 ? align256(static_cast<size_t>(i) * sizeof(float)) : 0);
    if (layout == 1 && h <= 4096) {  // room for the fused path too
        const size_t nblk = static_cast<size_t>((n_active + 7) / 8);  // the most partials (1 neuron per wave)
        const size_t fused = align256((nblk > 0 ? nblk : 1) * FUSED_STRIDE * sizeof(float));
        off = off > fused ? off : fused;
    }
    // the normalised x of the block entry when its types cannot fuse the norm
    w.xn = off;
    w.total = off + align256(static_cast<size_t>(h) * sizeof(float));
    return w;
}

__global__ void fill_zero_kernel(float* p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

// y = a + b (y may be a or b)
__global__ void add_vec_kernel(const float* a, const float* b, float* y, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}

__global__ void copy_vec_kernel(const float* a, float* y, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i];
}

bool block_type(int32_t t) { return is_block_type(t); }

template <int NPW>
void launch_fused(bool norm, dim3 g, hipStream_t st, const void* wg, const void* wu, const void* wd, int64_t rb,
                  int64_t i, const float* x, const int32_t* active, int n_active, const int32_t* n_dev, int act_kind,
                  float* part, int units, int slots, const float* norm_w, float eps) {
    const uint8_t* a = static_cast<const uint8_t*>(wg);
    const uint8_t* b = static_cast<const uint8_t*>(wu);
    const uint8_t* c = static_cast<const uint8_t*>(wd);
    if constexpr (NPW == 0) {  // the column-split kernel (one neuron per wave)
        if (norm)
            sparse_fused_cols_kernel<true><<<g, dim3(512), 0, st>>>(a, b, c, rb, i, x, active, n_active, n_dev,
                                                                    act_kind, part, units, slots, norm_w, eps);
        else
            sparse_fused_cols_kernel<false><<<g, dim3(512), 0, st>>>(a, b, c, rb, i, x, active, n_active, n_dev,
                                                                     act_kind, part, units, slots, norm_w, eps);
    } else if (norm) {
        sparse_fused_q4k_kernel<NPW, true><<<g, dim3(512), 0, st>>>(a, b, c, rb, i, x, active, n_active, n_dev,
                                                                     act_kind, part, units, slots, norm_w, eps);
    } else {
        sparse_fused_q4k_kernel<NPW, false><<<g, dim3(512), 0, st>>>(a, b, c, rb, i, x, active, n_active, n_dev,
                                                                      act_kind, part, units, slots, norm_w, eps);
    }
}

// The sparse FFN with an optional RMSNorm of x (norm_w) and residual (the x
// term added to y).  y may be x.
// n_dev: optional device count of the active set (then n_active is the
// host's bound: launches are sized by it and the kernels stop at the count).
int sparse_ffn_impl(const void* wg, const void* wu, const void* wd, int32_t down_layout, const float* x,
                    const float* norm_w, float eps, const int32_t* active, int32_t n_active, const int32_t* n_dev,
                    int32_t act_kind, bool residual, float* y, int64_t h, int64_t i, int32_t ggml_type,
                    void* workspace, size_t workspace_bytes, hipStream_t st, const char* fn) {
    if (h <= 0 || i <= 0 || h > INT32_MAX || i > INT32_MAX || n_active < 0 || n_active > i ||
        (down_layout != 0 && down_layout != 1) ||
        (act_kind != ACT_SILU && act_kind != ACT_RELU2 && act_kind != ACT_GELU_TANH) || !wg || !wu || !wd || !x ||
        !y || (n_active > 0 && !active) || !(eps >= 0.f)) {
        set_error("%s: bad arguments", fn);
        return E_INVAL;
    }
    if (row_bytes(ggml_type, h) < 0 || row_bytes(ggml_type, i) < 0) {
        set_error("%s: type %d unsupported for h=%lld i=%lld", fn, ggml_type, static_cast<long long>(h),
                  static_cast<long long>(i));
        return E_UNSUPPORTED;
    }
    if (down_layout == 1 && (ggml_type != TYPE_Q4_K || h % 64 != 0)) {
        set_error("%s: neuron-major down (layout 1) needs Q4_K and h %% 64 == 0", fn);
        return E_UNSUPPORTED;
    }
    const SparseWs ws = sparse_ws(h, i, n_active, down_layout);
    if (!workspace || workspace_bytes < ws.total) {
        set_error("%s: workspace of %zu bytes needed", fn, ws.total);
        return E_NOMEM;
    }
    if (norm_w && (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(norm_w) % 16 != 0)) {
        set_error("%s: x and norm_w must be 16-byte aligned", fn);
        return E_INVAL;
    }
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    float* gu = reinterpret_cast<float*>(wsb + ws.gu);
    const float* resid = residual ? x : nullptr;
    const dim3 vec_grid(static_cast<uint32_t>((h + 255) / 256));

    if (n_active == 0) {  // no active neuron: y = x or 0
        if (residual) {
            if (y != x) copy_vec_kernel<<<vec_grid, dim3(256), 0, st>>>(x, y, h);
        } else {
            fill_zero_kernel<<<vec_grid, dim3(256), 0, st>>>(y, h);
        }
        return check_launch(fn);
    }
    // a norm the gate/up launch cannot fuse (F32 / F16 weights) runs first
    const float* xin = x;
    const float* nw = norm_w;
    if (norm_w && !block_type(ggml_type)) {
        float* xn = reinterpret_cast<float*>(wsb + ws.xn);
        const int rc = vb_rms_norm(x, norm_w, xn, 1, h, eps, st);
        if (rc != OK) return rc;
        xin = xn;
        nw = nullptr;
    }
    if (fused_path(h, down_layout)) {
        // one launch for gate/up/act/down, one for the partial sums
        if (reinterpret_cast<uintptr_t>(xin) % 16 != 0) {
            set_error("%s: x must be 16-byte aligned", fn);
            return E_INVAL;
        }
        const int units = static_cast<int>(h / 64);
        const int slots = (units + 7) & ~7;  // gemv_core.hpp: encoded units, a multiple of 8
        // VB_SPARSE_NPW=1 / 2: the row-split kernel with 1 or 2 neurons per wave;
        // default the column-split kernel (1 neuron per wave)
        const int npw_knob = knobs().sparse_npw;
        const int npw = npw_knob == 2 ? 2 : 1;
        const int nblk = (n_active + 8 * npw - 1) / (8 * npw);
        float* part = reinterpret_cast<float*>(wsb);
        const dim3 g(static_cast<uint32_t>(nblk));
        const int64_t rb = row_bytes(TYPE_Q4_K, h);
        if (npw_knob == 2)
            launch_fused<2>(nw != nullptr, g, st, wg, wu, wd, rb, i, xin, active, n_active, n_dev, act_kind, part,
                            units, slots, nw, eps);
        else if (npw_knob == 1)
            launch_fused<1>(nw != nullptr, g, st, wg, wu, wd, rb, i, xin, active, n_active, n_dev, act_kind, part,
                            units, slots, nw, eps);
        else
            launch_fused<0>(nw != nullptr, g, st, wg, wu, wd, rb, i, xin, active, n_active, n_dev, act_kind, part,
                            units, slots, nw, eps);
        int rcf = check_launch(fn);
        if (rcf != OK) return rcf;
        sparse_reduce_kernel<<<dim3(static_cast<uint32_t>(units)), dim3(1024), 0, st>>>(part, nblk, n_dev, 8 * npw,
                                                                                       resid, y);
        return check_launch(fn);
    }
    // GGUF down, Q4_K gate/up with h <= 4096: one launch writes the whole
    // hidden vector (act(g, u) on the active set, zeros elsewhere) on the
    // short-row arithmetic, then the down GEMV (with the residual)
    if (down_layout == 0 && ggml_type == TYPE_Q4_K && h <= 4096 && h % 256 == 0 && !knobs().gemv_q4k_general &&
        gemv_q4k_pairs_npw(n_active) > 0 && reinterpret_cast<uintptr_t>(xin) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(wg) % 16 == 0 && reinterpret_cast<uintptr_t>(wu) % 16 == 0) {
        float* hid = reinterpret_cast<float*>(wsb + ws.hid);
        int rc = gemv_q4k_pairs(wg, wu, xin, nw, eps, act_kind, hid, n_active, h, st, active, n_dev, i);
        if (rc != OK) return rc;
        if (!residual) return gemv_dispatch(wd, hid, y, h, i, ggml_type, st);
        GemvFuse fd;
        fd.resid = x;
        return gemv_dispatch_fused(wd, RowSrc{}, fd, hid, y, h, i, ggml_type, st);
    }
    // 1. gate/up on the active rows (with the norm in the encode)
    RowSrc src;
    src.w2 = wu;
    src.gidx = active;
    src.nsrc = i;
    src.n_dev = n_dev;
    float* hid = reinterpret_cast<float*>(wsb + ws.hid);
    if (down_layout == 0) {  // the dense hidden vector starts at zero
        src.zbuf = reinterpret_cast<int*>(hid);
        src.zn = static_cast<int>(i);
    }
    GemvFuse fz;
    fz.norm_w = nw;
    fz.eps = eps;
    int rc = gemv_dispatch_fused(wg, src, fz, xin, gu, 2 * static_cast<int64_t>(n_active), h, ggml_type, st);
    if (rc != OK) return rc;
    // 2. down (with the residual in the launch that writes y)
    if (down_layout == 0) {
        scatter_act_kernel<<<dim3(static_cast<uint32_t>((n_active + 255) / 256)), dim3(256), 0, st>>>(
            active, n_active, n_dev, gu, act_kind, hid, i);
        if ((rc = check_launch(fn)) != OK) return rc;
        if (!residual) return gemv_dispatch(wd, hid, y, h, i, ggml_type, st);
        if (block_type(ggml_type)) {
            GemvFuse fd;
            fd.resid = x;
            return gemv_dispatch_fused(wd, RowSrc{}, fd, hid, y, h, i, ggml_type, st);
        }
        // F32 / F16 down: the product into the workspace, then the add
        float* dn = reinterpret_cast<float*>(wsb + ws.xn);
        if ((rc = gemv_dispatch(wd, hid, dn, h, i, ggml_type, st)) != OK) return rc;
        add_vec_kernel<<<vec_grid, dim3(256), 0, st>>>(x, dn, y, h);
        return check_launch(fn);
    }
    down_rows_q4k_kernel<<<dim3(static_cast<uint32_t>(h / 64)), dim3(DOWN_THREADS), 0, st>>>(
        static_cast<const uint8_t*>(wd), row_bytes(TYPE_Q4_K, h), i, active, n_active, n_dev, gu, act_kind, resid,
        y);
    return check_launch(fn);
}

}  // namespace
}  // namespace vb

using namespace vb;

extern "C" int64_t vb_sparse_ffn_workspace(int64_t h, int64_t i, int32_t n_active, int32_t down_layout) {
    if (h <= 0 || i <= 0 || n_active < 0 || (down_layout != 0 && down_layout != 1)) return -1;
    return static_cast<int64_t>(sparse_ws(h, i, n_active, down_layout).total);
}

extern "C" int vb_sparse_ffn(const void* wg, const void* wu, const void* wd, int32_t down_layout,
                             const float* x, const int32_t* active, int32_t n_active, int32_t act_kind,
                             float* y, int64_t h, int64_t i, int32_t ggml_type, void* workspace,
                             size_t workspace_bytes, void* stream) {
    return sparse_ffn_impl(wg, wu, wd, down_layout, x, nullptr, 0.f, active, n_active, nullptr, act_kind, false, y,
                           h, i, ggml_type, workspace, workspace_bytes, as_stream(stream), "vb_sparse_ffn");
}

extern "C" int vb_sparse_ffn_block(const void* wg, const void* wu, const void* wd, int32_t down_layout,
                                   const float* x, const float* norm_w, float eps, const int32_t* active,
                                   int32_t n_active, const int32_t* n_active_dev, int32_t act_kind,
                                   int32_t add_residual, float* y, int64_t h, int64_t i, int32_t ggml_type,
                                   void* workspace, size_t workspace_bytes, void* stream) {
    return sparse_ffn_impl(wg, wu, wd, down_layout, x, norm_w, eps, active, n_active, n_active_dev, act_kind,
                           add_residual != 0, y, h, i, ggml_type, workspace, workspace_bytes, as_stream(stream),
                           "vb_sparse_ffn_block");
}

// ---- allocation-free variant (static scratch) ------------------------------
//
// vb_sparse_ffn_noalloc runs vb_sparse_ffn with its workspace in `scratch`, a
// file-scope device array of kSparseScratchBytes per GPU (held until the
// process ends), for callers that cannot allocate device memory.  The array's
// name is a host-side stand-in: its device address is resolved once per
// device with hipGetSymbolAddress (vb_init, or the first call on a device)
// and only that address is handed to kernels.  Every call on one GPU shares
// the array: calls that overlap on one GPU (different streams or threads)
// race.  Nothing in it needs clearing between calls: the fused path writes
// every partial it reads, and the GGUF-down path's hidden vector is cleared
// inside its gate/up launch.
namespace {
constexpr size_t kSparseScratchBytes = size_t(8) << 20;  // 8 MiB
__device__ __align__(256) uint8_t scratch[kSparseScratchBytes];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};
}  // namespace

namespace vb {

// Device address of `scratch` on the current device (resolved once per device).
int sparse_scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("vb_sparse_ffn_noalloc: hipGetDevice: %s", hipGetErrorString(e));
        return E_HIP;
    }
    if (dev < 0 || dev >= kScratchDevices) {
        set_error("vb_sparse_ffn_noalloc: device %d beyond the %d supported", dev, kScratchDevices);
        return E_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("vb_sparse_ffn_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            return E_HIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return OK;
}

}  // namespace vb

extern "C" int vb_sparse_ffn_noalloc(const void* wg, const void* wu, const void* wd, int32_t down_layout,
                                     const float* x, const int32_t* active, int32_t n_active, int32_t act_kind,
                                     float* y, int64_t h, int64_t i, int32_t ggml_type, void* stream) {
    const int64_t need = vb_sparse_ffn_workspace(h, i, n_active, down_layout);
    if (need < 0) {
        set_error("vb_sparse_ffn_noalloc: bad shape (h=%lld, i=%lld, n_active=%d, down_layout=%d)",
                  static_cast<long long>(h), static_cast<long long>(i), n_active, down_layout);
        return E_INVAL;
    }
    if (static_cast<uint64_t>(need) > kSparseScratchBytes) {
        set_error("vb_sparse_ffn_noalloc: h=%lld, i=%lld, n_active=%d, down_layout=%d needs %lld bytes of "
                  "scratch, beyond the %zu of the static scratch; use vb_sparse_ffn with a workspace",
                  static_cast<long long>(h), static_cast<long long>(i), n_active, down_layout,
                  static_cast<long long>(need), kSparseScratchBytes);
        return E_INVAL;
    }
    void* ws = nullptr;
    const int rc = sparse_scratch_ptr(&ws);
    if (rc != OK) return rc;
    return sparse_ffn_impl(wg, wu, wd, down_layout, x, nullptr, 0.f, active, n_active, nullptr, act_kind, false, y,
                           h, i, ggml_type, ws, kSparseScratchBytes, as_stream(stream), "vb_sparse_ffn_noalloc");
}

extern "C" int vb_ema_update(float* probs, int64_t n, const uint8_t* mask, double alpha, void* stream) {
    if (n < 0 || (n > 0 && (!probs || !mask)) || !(alpha >= 0.0 && alpha <= 1.0)) {
        set_error("vb_ema_update: bad arguments");
        return E_INVAL;
    }
    if (n == 0) return OK;
    // the reference's scalars as numpy rounds them for float32 arrays: alpha
    // and (1 - alpha), each computed in double and rounded to fp32 once
    const float a = static_cast<float>(alpha);
    const float beta = static_cast<float>(1.0 - alpha);
    ema_update_kernel<<<dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(
        probs, mask, n, a, beta);
    return check_launch("vb_ema_update");
}

extern "C" int vb_ema_predict(const float* probs, const float* gate_values, int64_t n, int32_t k, float threshold,
                              int32_t warm, int32_t combined, uint8_t* mask_out, int32_t* active_out,
                              int32_t* count_out, void* stream) {
    if (n <= 0 || n > 0x7fffffff || k < 1 || k > n || !mask_out || !active_out || !count_out ||
        (warm && !probs) || (combined && !gate_values)) {
        set_error("vb_ema_predict: bad arguments (n=%lld, k=%d)", static_cast<long long>(n), k);
        return E_INVAL;
    }
    const int flags = (warm ? PRED_WARM : 0) | (gate_values ? PRED_GATE : 0) | (combined ? PRED_COMBINED : 0);
    const int ni = static_cast<int>(n);
    hipStream_t st = as_stream(stream);
    // register-resident for n <= 16384 (16 values per thread; 32 would spill
    // at 1024 threads), the streaming kernel above
    if (n <= 1024 * 16)
        ema_predict_reg_kernel<16><<<dim3(1), dim3(1024), 0, st>>>(probs, gate_values, ni, k, threshold, flags,
                                                                   mask_out, active_out, count_out);
    else
        ema_predict_kernel<<<dim3(1), dim3(1024), 0, st>>>(probs, gate_values, ni, k, threshold, flags, mask_out,
                                                           active_out, count_out);
    return check_launch("vb_ema_predict");
}

extern "C" int vb_topk_indices(const float* v, int64_t n, int32_t k, int32_t* out_idx, void* stream) {
    if (n < 0 || n > 0x7fffffff || k < 0 || (n > 0 && (!v || (k > 0 && !out_idx)))) {
        set_error("vb_topk_indices: bad arguments");
        return E_INVAL;
    }
    if (k == 0 || n == 0) return OK;
    if (k > n) {
        set_error("vb_topk_indices: k=%d > n=%lld", k, static_cast<long long>(n));
        return E_INVAL;
    }
    topk_kernel<<<dim3(1), dim3(1024), 0, as_stream(stream)>>>(v, static_cast<int>(n), k, out_idx);
    return check_launch("vb_topk_indices");
}
