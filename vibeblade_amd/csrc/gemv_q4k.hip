// Q4_K GEMV for rows of k <= 4096 (one 64-element unit per lane):
// y[n] = sum_k W[n, k] x[k], W in the GGUF layout.  The headline decode
// shape (Llama-3-8B FFN gate/up, 14336 x 4096) runs here.  The same
// short-row arithmetic serves the Q6_K GEMV for k = 2048 / 4096 (the lm_head),
// the Q4_K gate/up pairs of the FFN block and the split-row Q4_K GEMV for
// 4096 < k <= 16384 (further down).
//
// Replaces gemv_dequant (cpp/src/dequant.cpp:739-780) for Q4_K weights: no
// weight is decoded to floats.  Per row and lane the work is integer dot
// products of the 64 nibbles of one unit against the activation encoding,
// then one scale/min combination:
//
//   unit u (lane), super-block u / 4, chunk c = u % 4: sub-blocks 2c (low
//   nibbles of qs[32c, 32c + 32)) and 2c + 1 (high nibbles), elements
//   64u .. 64u + 63 of the row (cpp/src/dequant.cpp:278-299).
//
// Activation encoding (one per workgroup, in LDS): x ~= s_u * x16 with one
// fp32 scale s_u per unit, |x16| <= 16383 (15-bit fixed point), x16 = 256 xh
// + xl with xh, xl signed bytes, and the integer run sums I0, I1 of x16 over
// the unit's two 32-element runs.  Then, exactly in integers,
//   D_r = sum_{e in run r} q_e x16_e   (two v_dot4 per 4 weights: xh and xl)
//   S   = sc0 D0 + sc1 D1,   M = m0 I0 + m1 I1   (24-bit multiplies: |D_r| <=
//         32 * 15 * 16383 < 2^23)
// and the lane's share of the row is s_u (d S - dmin M): 3 fp32 roundings
// per unit.  The encoding error |x - s_u x16| <= s_u / 2 = amax_u / 32766
// puts the GEMV rel-L2 near 5e-5 (the fp32-accumulate bar is 1e-3).
//
// Schedule.  One workgroup of 8 waves per CU; wave w owns RPW consecutive
// rows and streams them through a ring of NS register buffers: the loads of
// row s + NS - 1 are issued before row s is computed, and row s + 1 is
// staged (below) while row s is computed.
//
// Loads.  A row (2304 B at k = 4096) is read contiguously: lane L takes the
// 16 B at 16 L, 1024 + 16 L and (L < 16) 2048 + 16 L, three buffer loads with
// the row offset in an SGPR, marked non-temporal (the weights are streamed
// once).  Every load instruction then covers whole cache lines.  Measured on
// MI355X with the loads alone (14336 x 4096): 6.6 us per launch, against
// 7.4 us for per-lane unit loads (a 16 B header and two 16 B pieces of one
// unit per lane, each instruction touching parts of 16 lines; non-temporal
// made that pattern slower still, 8.8 us, since the other parts of a line
// are no longer found in the cache).  The wave writes its row into a private
// LDS row buffer and reads it back in the unit layout (header, qs[32c, +16),
// qs[32c + 16, +16)); LDS operations of one wave run in order, so one buffer
// per wave is enough.
//
// Each row leaves one partial per lane in a register; after the last row the
// wave reduces all RPW rows at once with a transposed butterfly (permlane32
// / permlane16 swaps, then DPP), about 18 instructions for up to 8 rows, and
// lanes 8g store y.  No LDS reduction and no barrier at the end.
#include <cstdint>
#include <type_traits>

#include "vb_common.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int X15_MAX = 16383;
constexpr int UNITS_MAX = 64;       // k <= 4096
constexpr int XQ_UNIT_QUADS = 9;    // xh[16], xl[16] dwords, {s, I0, I1, 128 I1}

struct XU {
    uint32_t h[16], l[16];
    float s;
    int i0, i1, c1;
};

template <int CTRL>
__device__ __forceinline__ float dpp_mov_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Task t = 8 consecutive elements (part p = t % 8) of unit t / 8; the 8
// tasks of a unit sit on adjacent lanes.  Units at or past `units` encode
// as zeros (their lanes contribute nothing).  US is the unit stride of the
// encoding (the most units it holds).
// LDS stores the compiler does not see (ds_write in asm; "memory" keeps
// them in order with the surrounding code).  The DMA kernel's encode uses
// them: a compiler-visible LDS store issued while LDS DMA is in flight gets
// a full vmcnt(0) wait whenever the compiler cannot tell it apart from the
// DMA's destination (merged ds_write2 stores lose that information).  The
// caller makes them visible with lgkmcnt(0) before its barrier.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    typedef const __attribute__((address_space(3))) char* lds_cptr;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cptr)p));
}
__device__ __forceinline__ void lds_st64(void* p, uint2 v) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 d = {v.x, v.y};
    asm volatile("ds_write_b64 %0, %1" : : "v"(lds_addr(p)), "v"(d) : "memory");
}
__device__ __forceinline__ void lds_st128(void* p, uint4 v) {
    const u32x4 d = {v.x, v.y, v.z, v.w};
    asm volatile("ds_write_b128 %0, %1" : : "v"(lds_addr(p)), "v"(d) : "memory");
}

template <int US = UNITS_MAX, bool ASM_ST = false>
__device__ __forceinline__ void encode_task(const float* v_in, int task, int units, uint4* xq, bool store = true) {
    const int u = task >> 3, p = task & 7;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = u < units ? v_in[i] : 0.f;
    // all-reductions over the unit's 8 adjacent lanes with DPP (no LDS round
    // trip): quad butterflies, then row_half_mirror (lane i <-> 7 - i)
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, dpp_mov_f<0xB1>(amax));   // quad_perm [1,0,3,2]
    amax = fmaxf(amax, dpp_mov_f<0x4E>(amax));   // quad_perm [2,3,0,1]
    amax = fmaxf(amax, dpp_mov_f<0x141>(amax));  // row_half_mirror
    const float inv = amax > 0.f ? static_cast<float>(X15_MAX) / amax : 0.f;
    uint32_t ph[2] = {0, 0}, pl[2] = {0, 0};
    int isum = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int q = static_cast<int>(rintf(v[i] * inv));
        q = q > X15_MAX ? X15_MAX : (q < -X15_MAX ? -X15_MAX : q);
        isum += q;
        const int lo = ((q + 128) & 255) - 128;
        const int hi = (q - lo) >> 8;
        ph[i >> 2] |= static_cast<uint32_t>(hi & 255) << (8 * (i & 3));
        pl[i >> 2] |= static_cast<uint32_t>(lo & 255) << (8 * (i & 3));
    }
    isum += dpp_mov_i<0xB1>(isum);
    isum += dpp_mov_i<0x4E>(isum);              // sum over the run's 4 tasks (a quad)
    const int isum1 = dpp_mov_i<0x141>(isum);   // part 0 reads run 1's sum from part 7
    if (!store) return;
    uint4* b = xq + u;
    uint4 m;
    m.x = __float_as_uint(amax / static_cast<float>(X15_MAX));
    m.y = static_cast<uint32_t>(isum);
    m.z = static_cast<uint32_t>(isum1);
    m.w = static_cast<uint32_t>(128 * isum1);
    if constexpr (ASM_ST) {
        lds_st64(&reinterpret_cast<uint2*>(&b[(p >> 1) * US])[p & 1], make_uint2(ph[0], ph[1]));
        lds_st64(&reinterpret_cast<uint2*>(&b[(4 + (p >> 1)) * US])[p & 1], make_uint2(pl[0], pl[1]));
        if (p == 0) lds_st128(&b[8 * US], m);
    } else {
        reinterpret_cast<uint2*>(&b[(p >> 1) * US])[p & 1] = make_uint2(ph[0], ph[1]);
        reinterpret_cast<uint2*>(&b[(4 + (p >> 1)) * US])[p & 1] = make_uint2(pl[0], pl[1]);
        if (p == 0) b[8 * US] = m;
    }
}

template <int US = UNITS_MAX>
__device__ __forceinline__ XU read_unit(const uint4* xq, int u) {
    XU x;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 h = xq[i * US + u], l = xq[(4 + i) * US + u];
        x.h[4 * i] = h.x; x.h[4 * i + 1] = h.y; x.h[4 * i + 2] = h.z; x.h[4 * i + 3] = h.w;
        x.l[4 * i] = l.x; x.l[4 * i + 1] = l.y; x.l[4 * i + 2] = l.z; x.l[4 * i + 3] = l.w;
    }
    const uint4 m = xq[8 * US + u];
    x.s = __uint_as_float(m.x);
    x.i0 = static_cast<int>(m.y);
    x.i1 = static_cast<int>(m.z);
    x.c1 = static_cast<int>(m.w);
    return x;
}

struct RowBuf { u32x4 hdr, qa, qb; };
struct RowRaw { u32x4 a, b, c; };  // the row's bytes 16 L, 1024 + 16 L, 2048 + 16 (L % 16)

constexpr int CACHE_NT = 2;  // buffer-load cache policy: non-temporal (streamed once)
constexpr int ROW_SLOTS = 144;  // 16-byte slots of a k = 4096 row buffer (2304 B)

// Lane-constant selectors of the scale / min bytes of sub-blocks 2c, 2c + 1
// (get_scale_min_k4, cpp/src/dequant.cpp:258-266).  With A, B, C = scales[0:4],
// [4:8], [8:12] and c' = c % 2:
//   P = bytes (A[2c'], A[2c'+1], B[2c'], B[2c'+1]), Q = the same bytes of
//   (C, C >> 4);  c < 2: R = P & 0x3F3F3F3F;  c >= 2: R = (Q & 0x0F0F0F0F) |
//   ((P >> 2) & 0x30303030);  R = sc0 | sc1 << 8 | m0 << 16 | m1 << 24.
struct ScaleSel {
    uint32_t sel, kq, kp, sp;
};

__device__ __forceinline__ ScaleSel make_sel(int c) {
    ScaleSel s;
    const uint32_t c2 = 2u * static_cast<uint32_t>(c & 1);
    s.sel = c2 | ((c2 + 1u) << 8) | ((c2 + 4u) << 16) | ((c2 + 5u) << 24);
    const bool hi = c >= 2;
    s.kq = hi ? 0x0F0F0F0Fu : 0u;
    s.kp = hi ? 0x30303030u : 0x3F3F3F3Fu;
    s.sp = hi ? 2u : 0u;
    return s;
}

__device__ __forceinline__ float row_part(const RowBuf& r, const XU& x, const ScaleSel& ss) {
    const uint32_t qd[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
    int dh0 = 0, dl0 = 0, dh1 = 0, dl1 = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t lo = qd[i] & 0x0F0F0F0Fu;
        const uint32_t hi = (qd[i] ^ 0x80808080u) & 0xF0F0F0F0u;  // 16 (q - 8), signed bytes
        dh0 = sdot4(lo, x.h[i], dh0);
        dl0 = sdot4(lo, x.l[i], dl0);
        dh1 = sdot4(hi, x.h[8 + i], dh1);
        dl1 = sdot4(hi, x.l[8 + i], dl1);
    }
    const int d0 = dh0 * 256 + dl0;
    const int d1 = (dh1 * 256 + dl1 + x.c1) >> 4;  // sum 16 (q - 8) x16 = 16 D1 - 128 I1
    const uint32_t A = r.hdr.y, B = r.hdr.z, C = r.hdr.w;
    const uint32_t P = __builtin_amdgcn_perm(B, A, ss.sel);
    const uint32_t Q = __builtin_amdgcn_perm(C >> 4, C, ss.sel);
    const uint32_t R = (Q & ss.kq) | ((P >> ss.sp) & ss.kp);
    const int S = __mul24(static_cast<int>(R & 0xFFu), d0) + __mul24(static_cast<int>((R >> 8) & 0xFFu), d1);
    const int M = __mul24(static_cast<int>((R >> 16) & 0xFFu), x.i0) + __mul24(static_cast<int>(R >> 24), x.i1);
    const float d = f16lo(r.hdr.x), dmin = f16hi(r.hdr.x);
    return (d * static_cast<float>(S) - dmin * static_cast<float>(M)) * x.s;
}

// Sum over the 64 lanes of each of a[0..7]; lanes 8g .. 8g + 7 end with the
// total of row rows_of(g) = 4 (g % 2) + {0, 2, 1, 3}[g / 2].  Fixed order.
__device__ __forceinline__ float reduce8(const float (&a)[8]) {
    float b[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {  // lanes < 32: row 2p, lanes >= 32: row 2p + 1
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[2 * p]), __float_as_uint(a[2 * p + 1]),
                                                         false, false);
        b[p] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    float c[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {  // 16-lane rows: 4q, 4q + 2, 4q + 1, 4q + 3
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(b[2 * q]), __float_as_uint(b[2 * q + 1]),
                                                         false, false);
        c[q] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const bool odd8 = (threadIdx.x & 8) != 0;
    const float own = odd8 ? c[1] : c[0];
    const float other = odd8 ? c[0] : c[1];
    // lane i takes `other` from lane i ^ 8 (row_ror:8 within the 16-lane row)
    float v = own + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(other), 0x128, 0xF, 0xF, false));
    v += dpp_f<0x141>(v);  // row_half_mirror: i <-> 7 - i within 8 lanes
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    return v;
}

__device__ __forceinline__ int row_of_group(int g) {
    return 4 * (g & 1) + ((0x3120 >> (4 * (g >> 1))) & 0xF);
}

// XH: x in fp16 (a one-row GEMM with fp16 activations), converted as loaded.
template <int RPW, int NS, int WPG, bool XH = false>
__global__ void __launch_bounds__(64 * WPG) gemv_q4k_kernel(const uint8_t* __restrict__ w, const void* __restrict__ xp,
                                                            float* __restrict__ y, int n, int units, uint32_t rb) {
    static_assert(WPG == 8 || WPG == 16, "8 or 16 waves: one encode task per thread for the first 512");
    __shared__ uint4 xq[XQ_UNIT_QUADS * UNITS_MAX];
    __shared__ u32x4 rowbuf[WPG][ROW_SLOTS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row0 = (static_cast<int>(blockIdx.x) * WPG + wave) * RPW;
    const int rlast = n - 1;
    // the wave's rows, clamped into the tensor (rows past n load row n - 1
    // again and store nothing)
    const int rbase = row0 < rlast ? row0 : rlast;
    const uint8_t* wb = w + static_cast<int64_t>(rbase) * rb;
    const int64_t span64 = static_cast<int64_t>(n - rbase) * rb;
    const uint32_t span = span64 < 0xFFFFFFFFll ? static_cast<uint32_t>(span64) : 0xFFFFFFFFu;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(wb, span);
    const bool valid = lane < units;
    const int u = valid ? lane : (lane & 3);  // idle lanes read unit (lane % 4) of the row, discarded
    // contiguous pieces of the row (rb = 144 * units / 4 bytes = 16 * slots):
    // slots lane, 64 + lane, 128 + lane % 16.  A piece past the row's end reads
    // an in-row address instead (coalesced: nothing extra is read) and lands in
    // a buffer slot that no unit reads; lanes 16..63 repeat lanes 0..15's
    // third piece, writing the same value to the same slot.
    // (a row has at least 9 slots, k >= 256, so lane % 8 is always in it)
    const int slots = static_cast<int>(rb >> 4);
    const int pc = 128 + (lane & 15);
    const uint32_t va = 16u * static_cast<uint32_t>(lane < slots ? lane : lane & 7);
    const uint32_t vb = 16u * static_cast<uint32_t>(64 + lane < slots ? 64 + lane : lane & 7);
    const uint32_t vc = 16u * static_cast<uint32_t>(pc < slots ? pc : lane & 7);
    u32x4* rbuf = rowbuf[wave];
    const int sh = 9 * (u >> 2), sq = sh + 1 + 2 * (u & 3);  // unit slots: header, qs pieces

    auto soff = [&](int s) -> uint32_t {
        int r = row0 + s;
        r = r < rlast ? r : rlast;
        return static_cast<uint32_t>(r - rbase) * rb;
    };
    auto issue = [&](RowRaw& b, int s) {
        const uint32_t so = soff(s);
        b.a = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(va), static_cast<int>(so), CACHE_NT);
        b.b = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(vb), static_cast<int>(so), CACHE_NT);
        b.c = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(vc), static_cast<int>(so), CACHE_NT);
    };
    // the row through the wave's LDS buffer into the unit layout
    auto stage = [&](const RowRaw& b) -> RowBuf {
        rbuf[lane] = b.a;
        rbuf[64 + lane] = b.b;
        rbuf[pc] = b.c;
        RowBuf r;
        r.hdr = rbuf[sh];
        r.qa = rbuf[sq];
        r.qb = rbuf[sq + 1];
        return r;
    };

    // x first (the encode waits only for it, loads retiring in order), then
    // the first rows' weights.  Every thread runs one encode task (64 units
    // x 8 tasks; threads past 512 repeat task t - 512 and store nothing): an
    // encode under a branch would let the compiler sink the x loads into it,
    // behind the weight loads.
    float xv[8];
    const int task = static_cast<int>(threadIdx.x) & 511;
    {
        const int tu = task >> 3;
        const int off = (tu < units ? tu : units - 1) * 64 + 8 * (task & 7);
        if constexpr (XH) {
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 hv = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(xp) + off);
#pragma unroll
            for (int i = 0; i < 8; i++) xv[i] = static_cast<float>(hv[i]);
        } else {
            const float* x = static_cast<const float*>(xp);
            const float4 a = *reinterpret_cast<const float4*>(x + off);
            const float4 b = *reinterpret_cast<const float4*>(x + off + 4);
            xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
            xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    RowRaw ring[NS];
#pragma unroll
    for (int s = 0; s < NS - 1 && s < RPW; s++) issue(ring[s], s);
    __builtin_amdgcn_sched_barrier(0);
    encode_task(xv, task, units, xq, WPG == 8 || threadIdx.x < 512);
    __syncthreads();
    const XU xu = read_unit(xq, u);
    const ScaleSel ss = make_sel(u & 3);

    float acc[8];
#pragma unroll
    for (int s = 0; s < 8; s++) acc[s] = 0.f;
    // Row s + 1 goes through the LDS row buffer while row s is computed
    // (the buffer's write and read-back overlap the arithmetic; row s was
    // read back into registers in the previous iteration, and one wave's LDS
    // operations complete in order).  The wave then waits for row s + 1's
    // loads with NS - 2 rows behind them still in flight.  On MI355X at
    // 14336 x 4096: 7.29 us against 7.42 us staging each row just before it
    // is computed (NS = 5 with this order: 7.53 us).
    if (NS - 1 < RPW) issue(ring[(NS - 1) % NS], NS - 1);
    RowBuf cur = stage(ring[0]);
#pragma unroll
    for (int s = 0; s < RPW; s++) {
        if (s >= 1 && s + NS - 1 < RPW) issue(ring[(s + NS - 1) % NS], s + NS - 1);
        RowBuf nxt = cur;
        if (s + 1 < RPW) nxt = stage(ring[(s + 1) % NS]);
        const float part = row_part(cur, xu, ss);
        acc[s] = valid ? part : 0.f;  // idle lanes: nothing, even from a non-finite scale
        cur = nxt;
        __builtin_amdgcn_sched_barrier(0);
    }
    const float tot = reduce8(acc);
    const int g = lane >> 3;
    const int r = row_of_group(g);
    if ((lane & 7) == 0 && r < RPW && row0 + r < n) y[row0 + r] = tot;
}

// ---- The same GEMV with the rows landing in LDS by DMA ---------------------
//
// Rows are read with buffer_load ... lds: lane L's 16 bytes of a piece go
// straight to LDS at slot L of the wave's ring buffer, so no row passes
// through VGPRs and nothing is staged by hand; the wave reads its unit
// layout (header, qs pieces) back from the slot when the row is due.  The
// ring is NS slots per wave, each its own __shared__ array: the compiler's
// wait counting for LDS DMA separates LDS objects, so reading slot s waits
// only for the DMA of row s (loads retire in order: vmcnt = the loads issued
// after it) and the x encoding's LDS traffic waits for none.  The encode is
// published with lgkmcnt(0) and a bare s_barrier: __syncthreads' release
// fence would wait for every DMA in flight.  Piece c is loaded by all 64
// lanes (lanes 16..63 repeat lanes 0..15's addresses), so a slot holds
// 192 16-byte slots, 144 of them the row.  Same arithmetic, same results as
// gemv_q4k_kernel.
constexpr int DMA_SLOTS = 192;

template <int RPW, int NS>
__global__ void __launch_bounds__(512) gemv_q4k_dma_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                           float* __restrict__ y, int n, int units, uint32_t rb) {
    static_assert(NS >= 2 && NS <= 5, "ring of 2..5 rows");
    constexpr int WPG = 8;
    __shared__ uint4 xq[XQ_UNIT_QUADS * UNITS_MAX];
    __shared__ u32x4 ring0[WPG][DMA_SLOTS], ring1[WPG][DMA_SLOTS], ring2[WPG][DMA_SLOTS], ring3[WPG][DMA_SLOTS],
            ring4[WPG][DMA_SLOTS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row0 = (static_cast<int>(blockIdx.x) * WPG + wave) * RPW;
    const int rlast = n - 1;
    const int rbase = row0 < rlast ? row0 : rlast;
    const uint8_t* wb = w + static_cast<int64_t>(rbase) * rb;
    const int64_t span64 = static_cast<int64_t>(n - rbase) * rb;
    const uint32_t span = span64 < 0xFFFFFFFFll ? static_cast<uint32_t>(span64) : 0xFFFFFFFFu;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(wb, span);
    const bool valid = lane < units;
    const int u = valid ? lane : (lane & 3);
    const int slots = static_cast<int>(rb >> 4);
    const uint32_t va = 16u * static_cast<uint32_t>(lane < slots ? lane : lane & 7);
    const uint32_t vb = 16u * static_cast<uint32_t>(64 + lane < slots ? 64 + lane : lane & 7);
    const uint32_t vc = 16u * static_cast<uint32_t>(128 + (lane & 15) < slots ? 128 + (lane & 15) : lane & 7);
    const int sh = 9 * (u >> 2), sq = sh + 1 + 2 * (u & 3);

    auto slot_base = [&](auto k_c) __attribute__((always_inline)) -> u32x4* {
        constexpr int k = decltype(k_c)::value;
        if constexpr (k == 0) return ring0[wave];
        else if constexpr (k == 1) return ring1[wave];
        else if constexpr (k == 2) return ring2[wave];
        else if constexpr (k == 3) return ring3[wave];
        else return ring4[wave];
    };
    auto issue = [&](auto k_c, int s) __attribute__((always_inline)) {
        int r = row0 + s;
        r = r < rlast ? r : rlast;
        const uint32_t so = static_cast<uint32_t>(r - rbase) * rb;
        u32x4* b = slot_base(k_c);
        typedef __attribute__((address_space(3))) void* lds_ptr;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)b, 16, static_cast<int>(va), static_cast<int>(so), 0,
                                                 CACHE_NT);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(b + 64), 16, static_cast<int>(vb),
                                                 static_cast<int>(so), 0, CACHE_NT);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(b + 128), 16, static_cast<int>(vc),
                                                 static_cast<int>(so), 0, CACHE_NT);
    };

    float xv[8];
    const int task = static_cast<int>(threadIdx.x);
    {
        const int tu = task >> 3;
        const int off = (tu < units ? tu : units - 1) * 64 + 8 * (task & 7);
        const float4 a = *reinterpret_cast<const float4*>(x + off);
        const float4 b = *reinterpret_cast<const float4*>(x + off + 4);
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NS - 1 >= 1) if (0 < RPW) issue(std::integral_constant<int, 0>{}, 0);
    if constexpr (NS - 1 >= 2) if (1 < RPW) issue(std::integral_constant<int, 1>{}, 1);
    if constexpr (NS - 1 >= 3) if (2 < RPW) issue(std::integral_constant<int, 2>{}, 2);
    if constexpr (NS - 1 >= 4) if (3 < RPW) issue(std::integral_constant<int, 3>{}, 3);
    __builtin_amdgcn_sched_barrier(0);
    encode_task<UNITS_MAX, true>(xv, task, units, xq, true);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the encode is in LDS
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const XU xu = read_unit(xq, u);
    const ScaleSel ss = make_sel(u & 3);

    float acc[8];
#pragma unroll
    for (int s = 0; s < 8; s++) acc[s] = 0.f;
    auto step = [&](auto s_c) __attribute__((always_inline)) {
        constexpr int s = decltype(s_c)::value;
        if constexpr (s < RPW) {
            if constexpr (s + NS - 1 < RPW) issue(std::integral_constant<int, (s + NS - 1) % NS>{}, s + NS - 1);
            // row s is complete once at most the loads issued after it remain
            constexpr int after = 3 * (s + NS - 1 < RPW ? NS - 1 : RPW - 1 - s);
            static_assert(after < 16, "vmcnt field");
            __builtin_amdgcn_s_waitcnt(0x0F70 | after);
            const u32x4* b = slot_base(std::integral_constant<int, s % NS>{});
            RowBuf r;
            r.hdr = b[sh];
            r.qa = b[sq];
            r.qb = b[sq + 1];
            const float part = row_part(r, xu, ss);
            acc[s] = valid ? part : 0.f;
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
    step(std::integral_constant<int, 4>{});
    step(std::integral_constant<int, 5>{});
    step(std::integral_constant<int, 6>{});
    step(std::integral_constant<int, 7>{});
    const float tot = reduce8(acc);
    const int g = lane >> 3;
    const int r = row_of_group(g);
    if ((lane & 7) == 0 && r < RPW && row0 + r < n) y[row0 + r] = tot;
}

// ---- Q6_K short rows (k = 2048 or 4096): the lm_head shape ------------------
//
// Unit u (lane) = quarter c = u % 4 of super-block u / 4 (210 B: ql[128],
// qh[64], int8 scales[16], fp16 d; the GGUF Q6_K layout), h = c / 2, l0 =
// 16 (c % 2): four 16-element runs t at super-block elements 128 h + 32 t +
// l0 + [0, 16), y = d sc_t (q6 - 32) with
//   q6 = nibble | (qh bits 2t, 2t + 1) << 4,
//   nibble: low (t < 2) or high (t >= 2) half of ql[64 h + 32 (t % 2) + l0 + i],
//   qh bits from qh[32 h + l0 + i], sc_t = scales[8 h + c % 2 + 2 t]
// (the vb_dequant_rows formula; the reference decodes these rows in
// gemv_dequant, cpp/src/dequant.cpp:739-780, through dequantize_row).
//
// Activations: the short-row encoding (one fp32 scale per unit, 15-bit x16
// split into signed bytes), its element order run-major (element 16 t + i of
// the unit is run t's element i), and the four run sums I_t kept as 32 I_t.
// Per run, in integers: D_t = sum (q6 - 32) x16 = sum q6 x16 - 32 I_t, with
// the unsigned code q6 (0..63) in the v_dot4 bytes (two per 4 weights);
// |D_t| <= 16 * 32 * 16383 <
// 2^23, so the 24-bit multiplies give S_01 = sc_0 D_0 + sc_1 D_1 and S_23 =
// sc_2 D_2 + sc_3 D_3 exactly (each below 2^31), and the lane's share of the
// row is d s_u (S_01 + S_23).
//
// The code bytes come from ql and qh with one bit-select per 4 bytes: qh is
// split once per unit into its even fields (qh & 0x33333333) and odd fields
// (qh & 0xCC..), each shifted so field t lands on bits 4-5 of the byte and
// bits 6-7 stay clear; the select keeps the nibble's bits 0-3.
//
// Rows: a 3360 B row is read as contiguous 16-byte pieces (slots L, 64 + L,
// 128 + L, 192 + L of the row for lane L, the last for L < 18) into the
// wave's LDS row buffer; units at odd super-blocks sit 2 bytes past a dword
// there and are read as 20 aligned bytes plus v_alignbyte.  Rows stream
// through a ring of NS, G rows per batched reduction (reduce8), the wave's
// rows in ceil(rpw / G) groups.
constexpr int XQ_Q6_QUADS = 10;    // xh[16], xl[16] dwords, {32 I_t}, {s}

struct XU6 {
    uint32_t h[16], l[16];
    int c[4];  // 32 I_t
    float s;
};

// Task t = 8 consecutive elements (run p / 2, half p % 2) of unit t / 8; the
// caller loads them.  Units at or past `units` encode as zeros.
template <int US = UNITS_MAX>
__device__ __forceinline__ void encode_task_q6(const float* v_in, int task, int units, uint4* xq, bool store) {
    const int u = task >> 3, p = task & 7;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = u < units ? v_in[i] : 0.f;
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, dpp_mov_f<0xB1>(amax));
    amax = fmaxf(amax, dpp_mov_f<0x4E>(amax));
    amax = fmaxf(amax, dpp_mov_f<0x141>(amax));
    const float inv = amax > 0.f ? static_cast<float>(X15_MAX) / amax : 0.f;
    uint32_t ph[2] = {0, 0}, pl[2] = {0, 0};
    int isum = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int q = static_cast<int>(rintf(v[i] * inv));
        q = q > X15_MAX ? X15_MAX : (q < -X15_MAX ? -X15_MAX : q);
        isum += q;
        const int lo = ((q + 128) & 255) - 128;
        const int hi = (q - lo) >> 8;
        ph[i >> 2] |= static_cast<uint32_t>(hi & 255) << (8 * (i & 3));
        pl[i >> 2] |= static_cast<uint32_t>(lo & 255) << (8 * (i & 3));
    }
    isum += dpp_mov_i<0xB1>(isum);  // the run's two tasks (lanes 2t, 2t + 1)
    if (!store) return;
    uint4* b = xq + u;
    reinterpret_cast<uint2*>(&b[(p >> 1) * US])[p & 1] = make_uint2(ph[0], ph[1]);
    reinterpret_cast<uint2*>(&b[(4 + (p >> 1)) * US])[p & 1] = make_uint2(pl[0], pl[1]);
    if ((p & 1) == 0) reinterpret_cast<uint32_t*>(&b[8 * US])[p >> 1] = static_cast<uint32_t>(32 * isum);
    if (p == 0) reinterpret_cast<uint32_t*>(&b[9 * US])[0] = __float_as_uint(amax / static_cast<float>(X15_MAX));
}

template <int US = UNITS_MAX>
__device__ __forceinline__ XU6 read_unit_q6(const uint4* xq, int u) {
    XU6 x;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 h = xq[i * US + u], l = xq[(4 + i) * US + u];
        x.h[4 * i] = h.x; x.h[4 * i + 1] = h.y; x.h[4 * i + 2] = h.z; x.h[4 * i + 3] = h.w;
        x.l[4 * i] = l.x; x.l[4 * i + 1] = l.y; x.l[4 * i + 2] = l.z; x.l[4 * i + 3] = l.w;
    }
    const uint4 c = xq[8 * US + u];
    x.c[0] = static_cast<int>(c.x); x.c[1] = static_cast<int>(c.y);
    x.c[2] = static_cast<int>(c.z); x.c[3] = static_cast<int>(c.w);
    x.s = __uint_as_float(reinterpret_cast<const uint32_t*>(&xq[9 * US + u])[0]);
    return x;
}

// (a & 0x0F0F0F0F) | (b & 0xF0F0F0F0): one v_bitop3 (0xCA: s0 ? s1 : s2 per
// bit; written out, the compiler narrows the masks from the known-zero bits
// of b and emits two instructions)
__device__ __forceinline__ uint32_t nib_sel(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_bitop3_b32(0x0F0F0F0Fu, a, b, 0xCA);
}

// 16 bytes at p + sh (sh 0 or 2) from the 20 bytes at the 4-aligned p
__device__ __forceinline__ uint4 lds_realign(const uint8_t* p, uint32_t sh) {
    const uint4 a = ld_b128_a4(p);
    const uint32_t e = ld_b32(p + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(a.y, a.x, sh), __builtin_amdgcn_alignbyte(a.z, a.y, sh),
                      __builtin_amdgcn_alignbyte(a.w, a.z, sh), __builtin_amdgcn_alignbyte(e, a.w, sh));
}

// Per-type parts of the short-row kernel: the row in 16-byte slots (k =
// 4096), the activation encoding (element offset of task part p of unit u,
// encode, read), the unit's bytes in the LDS row buffer and its dot product.
template <int TYPE> struct ShortRow;

template <> struct ShortRow<TYPE_Q6_K> {
    static constexpr int SLOTS = 210;     // 3360 B
    static constexpr int XQUADS = XQ_Q6_QUADS;
    using X = XU6;
    struct Row { uint4 la, lb, qh; int sc[4]; uint32_t d; };
    struct Addr { const uint8_t *la, *qh; const int8_t* sc; const uint16_t* d; uint32_t sh; };
    static constexpr int bytes(int units) { return 210 * (units / 4); }
    static __device__ int x_off(int u, int p) {
        return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 16 * (u & 1) + 32 * (p >> 1) + 8 * (p & 1);
    }
    template <int US = UNITS_MAX>
    static __device__ void encode(const float* v, int task, int units, uint4* xq) {
        encode_task_q6<US>(v, task, units, xq, true);
    }
    template <int US = UNITS_MAX>
    static __device__ X read_x(const uint4* xq, int u) { return read_unit_q6<US>(xq, u); }
    // super-block B = 210 (u / 4) of the row buffer, 2 bytes past a dword
    // when u / 4 is odd
    static __device__ Addr addr(const uint8_t* rb, int u) {
        const int sbo = 210 * (u >> 2), c = u & 3, hh = c >> 1, l0 = 16 * (c & 1);
        Addr a;
        a.sh = static_cast<uint32_t>(sbo & 2);
        a.la = rb + (sbo + 64 * hh + l0 - static_cast<int>(a.sh));
        a.qh = rb + (sbo + 128 + 32 * hh + l0 - static_cast<int>(a.sh));
        a.sc = reinterpret_cast<const int8_t*>(rb + sbo + 192 + 8 * hh + (c & 1));
        a.d = reinterpret_cast<const uint16_t*>(rb + sbo + 208);
        return a;
    }
    static __device__ Row read(const Addr& a) {
        Row r;
        r.la = lds_realign(a.la, a.sh);
        r.lb = lds_realign(a.la + 32, a.sh);
        r.qh = lds_realign(a.qh, a.sh);
#pragma unroll
        for (int t = 0; t < 4; t++) r.sc[t] = a.sc[2 * t];
        r.d = *a.d;
        return r;
    }
    static __device__ float part(const Row& r, const X& x) {
        const uint32_t la[4] = {r.la.x, r.la.y, r.la.z, r.la.w};
        const uint32_t lb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
        const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        int D[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t q[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t ev = qh[j] & 0x33333333u, od = qh[j] & 0xCCCCCCCCu;  // fields 0, 2 / 1, 3
                if (t == 0) q[j] = nib_sel(la[j], ev << 4);
                else if (t == 1) q[j] = nib_sel(lb[j], od << 2);
                else if (t == 2) q[j] = nib_sel(la[j] >> 4, ev);
                else q[j] = nib_sel(lb[j] >> 4, od >> 2);
            }
            // one accumulation chain: the xh sum, times 256 minus 32 I_t, then
            // the xl products (written as 256 dh + dl the compiler rebuilds the
            // sum from shifts, since the 24-bit multiply reads only 24 bits)
            int a = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) a = sdot4(q[j], x.h[4 * t + j], a);
            a = (a << 8) - x.c[t];
#pragma unroll
            for (int j = 0; j < 4; j++) a = sdot4(q[j], x.l[4 * t + j], a);
            D[t] = a;
        }
        const int s01 = __mul24(r.sc[0], D[0]) + __mul24(r.sc[1], D[1]);
        const int s23 = __mul24(r.sc[2], D[2]) + __mul24(r.sc[3], D[3]);
        return (static_cast<float>(s01) + static_cast<float>(s23)) * (f16lo(r.d) * x.s);
    }
};

// Q8_0: unit u = blocks 2u, 2u + 1 (68 B at 68 u, 4-byte aligned in the row
// buffer): d0 = bytes 0-1, block 0's codes at bytes 2-33 (realigned by 2),
// d1 = bytes 34-35, block 1's codes at 36-67.  The encoding is the Q4_K one
// (elements 64 u .. 64 u + 63 in order); per block D = sum q x16 (|D| <=
// 32 * 128 * 16383 < 2^31) and the lane's share s_u (d0 D0 + d1 D1).
template <> struct ShortRow<TYPE_Q8_0> {
    static constexpr int SLOTS = 272;     // 4352 B
    static constexpr int XQUADS = XQ_UNIT_QUADS;
    using X = XU;
    struct Row { uint32_t w[17]; };
    struct Addr { const uint8_t* p; };
    static constexpr int bytes(int units) { return 68 * units; }
    static __device__ int x_off(int u, int p) { return 64 * u + 8 * p; }
    template <int US = UNITS_MAX>
    static __device__ void encode(const float* v, int task, int units, uint4* xq) {
        encode_task<US>(v, task, units, xq, true);
    }
    template <int US = UNITS_MAX>
    static __device__ X read_x(const uint4* xq, int u) { return read_unit<US>(xq, u); }
    static __device__ Addr addr(const uint8_t* rb, int u) { return Addr{rb + 68 * u}; }
    static __device__ Row read(const Addr& a) {
        Row r;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = ld_b128_a4(a.p + 16 * i);
            r.w[4 * i] = v.x; r.w[4 * i + 1] = v.y; r.w[4 * i + 2] = v.z; r.w[4 * i + 3] = v.w;
        }
        r.w[16] = ld_b32(a.p + 64);
        return r;
    }
    static __device__ float part(const Row& r, const X& x) {
        int a0 = 0, a1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            a0 = sdot4(__builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2), x.h[i], a0);
            a1 = sdot4(r.w[9 + i], x.h[8 + i], a1);
        }
        a0 <<= 8;
        a1 <<= 8;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            a0 = sdot4(__builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2), x.l[i], a0);
            a1 = sdot4(r.w[9 + i], x.l[8 + i], a1);
        }
        return (f16lo(r.w[0]) * static_cast<float>(a0) + f16hi(r.w[8]) * static_cast<float>(a1)) * x.s;
    }
};

// y = W x for plain rows of k <= 4096 elements (units = k / 64 lanes busy)
// in rows of whole 16-byte slots; wave w of workgroup b owns rows (8 b + w)
// rpw + [0, rpw).
// XH: x in fp16 (the one-row GEMM with fp16 activations), widened to fp32
// before the encode.
template <int TYPE, int G, int NS, bool XH = false>
__global__ void __launch_bounds__(512) gemv_short_kernel(const uint8_t* __restrict__ w,
                                                         const void* __restrict__ xp, float* __restrict__ y, int n,
                                                         int units, uint32_t rb, int rpw) {
    using T = ShortRow<TYPE>;
    constexpr int P = (T::SLOTS + 63) / 64;  // 16-byte pieces per lane
    constexpr int REM = T::SLOTS - 64 * (P - 1);
    static_assert(G >= 1 && G <= 8 && NS >= 2, "up to 8 rows per reduction");
    static_assert(REM >= 16, "the last piece's lanes past REM repeat lanes 0-15");
    __shared__ uint4 xq[T::XQUADS * UNITS_MAX];
    __shared__ u32x4 rowbuf[8][T::SLOTS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row0 = (static_cast<int>(blockIdx.x) * 8 + wave) * rpw;
    // the wave's rows [row0, row0 + nrow); loads of rows past them fall
    // outside the resource (zeros, no memory access)
    const int left = n - row0;
    const int nrow = left < 0 ? 0 : (left < rpw ? left : rpw);
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(w + static_cast<int64_t>(nrow > 0 ? row0 : 0) * rb, static_cast<uint32_t>(nrow) * rb);
    const bool valid = lane < units;
    const int u = valid ? lane : (lane & 3);  // idle lanes read unit (lane % 4), discarded
    // piece p of lane L: slot 64 p + L (the last piece: L < REM, else L % 16,
    // the same slot and bytes as lane L % 16); a slot past a shorter row loads
    // an in-row slot (its lines are being read anyway) into a buffer slot that
    // no unit reads
    const int slots = static_cast<int>(rb >> 4);
    uint32_t vo[P];
    int so_lds[P];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int slot = 64 * p + (p < P - 1 || lane < REM ? lane : (lane & 15));
        so_lds[p] = slot;
        vo[p] = 16u * static_cast<uint32_t>(slot < slots ? slot : lane & 7);
    }
    u32x4* rbuf = rowbuf[wave];
    const typename T::Addr ad = T::addr(reinterpret_cast<const uint8_t*>(rbuf), u);

    struct Raw { u32x4 p[P]; };
    // the row offset goes into the per-lane offset, which the range check covers
    auto issue = [&](Raw& b, int s) {
        const uint32_t so = static_cast<uint32_t>(s) * rb;
#pragma unroll
        for (int p = 0; p < P; p++)
            b.p[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(vo[p] + so), 0, CACHE_NT);
    };
    auto stage = [&](const Raw& b) {
#pragma unroll
        for (int p = 0; p < P; p++) rbuf[so_lds[p]] = b.p[p];
        return T::read(ad);
    };

    // x first, then the first rows, then the encode (as the Q4_K kernel)
    float xv[8];
    const int task = static_cast<int>(threadIdx.x);
    {
        const int tu0 = task >> 3;
        const int off = T::x_off(tu0 < units ? tu0 : units - 1, task & 7);
        if constexpr (XH) {
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 hv = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(xp) + off);
#pragma unroll
            for (int i = 0; i < 8; i++) xv[i] = static_cast<float>(hv[i]);
        } else {
            const float* x = static_cast<const float*>(xp);
            const float4 a = *reinterpret_cast<const float4*>(x + off);
            const float4 b = *reinterpret_cast<const float4*>(x + off + 4);
            xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
            xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    Raw ring[NS];
#pragma unroll
    for (int s = 0; s < NS - 1; s++) issue(ring[s], s);
    __builtin_amdgcn_sched_barrier(0);
    T::encode(xv, task, units, xq);
    __syncthreads();
    const typename T::X xu = T::read_x(xq, u);

    // G % NS == 0 whenever the wave has more than one group (host), so the
    // ring slot of row g0 + i is i % NS in every group
    for (int g0 = 0; g0 < nrow; g0 += G) {
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = 0.f;
#pragma unroll
        for (int i = 0; i < G; i++) {
            issue(ring[(i + NS - 1) % NS], g0 + i + NS - 1);
            const float part = T::part(stage(ring[i % NS]), xu);
            acc[i] = valid ? part : 0.f;
            __builtin_amdgcn_sched_barrier(0);
        }
        const float tot = reduce8(acc);
        const int r = g0 + row_of_group(lane >> 3);
        if ((lane & 7) == 0 && row_of_group(lane >> 3) < G && r < nrow) y[row0 + r] = tot;
    }
}

// ---- gate/up pairs with the activation epilogue (FFN block launch 1) ---------
//
// y[p] = act(gate_p . n, up_p . n) for neurons p, n = x (or RMSNorm(x) * norm_w
// with NORM), k <= 4096.  The short-row kernel's arithmetic and loads; wave w
// of workgroup b owns neurons (8 b + w) NPW + [0, NPW) and streams each
// neuron's gate row and up row through the same LDS row buffer, NS - 1
// neurons in flight.  NORM: every workgroup reduces sum(x^2) over all of x in
// a fixed order (same bits in every workgroup) and scales x by rinv * norm_w
// before the encode.  The gate and up partials are reduced at once per wave
// (two reduce8) and lanes 8g write act(g, u) of their neuron.
//
// GATHER (the sparse FFN with a GGUF-layout down): neuron p is row active[p]
// of both matrices, for p below the active count (n, or the device count at
// n_dev), and the launch writes the whole hidden vector y[0, i_dim) that the
// down GEMV reads: y[active[p]] = act(g, u), zeros elsewhere.  The active
// set is sorted ascending and unique, so workgroup b owns the positions
// from its first neuron's index (0 for b = 0) up to the next workgroup's
// first index (i_dim for the last one) and writes every one of them once.
template <int NPW, int NS, bool NORM, bool GATHER>
__global__ void __launch_bounds__(512) gemv_q4k_pairs_kernel(const uint8_t* __restrict__ wg,
                                                             const uint8_t* __restrict__ wu,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ norm_w, float eps, int kind,
                                                             float* __restrict__ y, int n, int units, uint32_t rb,
                                                             const int32_t* __restrict__ active,
                                                             const int32_t* __restrict__ n_dev, int i_dim) {
    __shared__ uint4 xq[XQ_UNIT_QUADS * UNITS_MAX];
    __shared__ u32x4 rowbuf[8][ROW_SLOTS];
    __shared__ float wsum[8];
    [[maybe_unused]] __shared__ int gid[8 * NPW];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int p0 = (static_cast<int>(blockIdx.x) * 8 + wave) * NPW;
    int n_act = n;
    if constexpr (GATHER) {
        n_act = active_count(n, n_dev);
        const int e0 = static_cast<int>(blockIdx.x) * 8 * NPW;
        // no neuron here, and no hidden position either (workgroup 0 zeroes
        // the whole vector when the count is 0)
        if (e0 >= n_act && !(e0 == 0 && n_act == 0)) return;
        // the workgroup's hidden positions [lo, hi): zeros where no neuron of
        // it sits (its neurons' indices, clamped, in LDS for the lookup)
        const int e1 = e0 + 8 * NPW < n_act ? e0 + 8 * NPW : n_act;
        auto idx = [&](int e) {
            const int v = active[e];
            return v < 0 ? 0 : (v > i_dim ? i_dim : v);
        };
        if (static_cast<int>(threadIdx.x) < e1 - e0) gid[threadIdx.x] = idx(e0 + threadIdx.x);
        const int lo = e0 == 0 ? 0 : idx(e0);
        const int hi = e1 < n_act ? idx(e1) : i_dim;
        __syncthreads();
        for (int q = lo + static_cast<int>(threadIdx.x); q < hi; q += 512) {
            int a = 0, b = e1 - e0;  // first neuron index >= q
            while (a < b) {
                const int m = (a + b) >> 1;
                if (gid[m] < q) a = m + 1; else b = m;
            }
            if (a == e1 - e0 || gid[a] != q) y[q] = 0.f;
        }
        if (n_act == 0) return;
    }
    const int plast = n_act - 1;
    const int pbase = p0 < plast ? p0 : plast;
    // dense: the wave's rows from pbase on; gathered: the whole matrices,
    // row offsets from the active list
    const int64_t span64 = GATHER ? static_cast<int64_t>(i_dim) * rb : static_cast<int64_t>(n - pbase) * rb;
    const uint32_t span = span64 < 0xFFFFFFFFll ? static_cast<uint32_t>(span64) : 0xFFFFFFFFu;
    const int64_t base = GATHER ? 0 : static_cast<int64_t>(pbase) * rb;
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(wg + base, span);
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(wu + base, span);
    const bool valid = lane < units;
    const int u = valid ? lane : (lane & 3);
    const int slots = static_cast<int>(rb >> 4);
    const int pc = 128 + (lane & 15);
    const uint32_t va = 16u * static_cast<uint32_t>(lane < slots ? lane : lane & 7);
    const uint32_t vb = 16u * static_cast<uint32_t>(64 + lane < slots ? 64 + lane : lane & 7);
    const uint32_t vc = 16u * static_cast<uint32_t>(pc < slots ? pc : lane & 7);
    u32x4* rbuf = rowbuf[wave];
    const int sh = 9 * (u >> 2), sq = sh + 1 + 2 * (u & 3);

    struct Pair { RowRaw g, u; };
    auto soff = [&](int s) -> uint32_t {
        int p = p0 + s;
        p = p < plast ? p : plast;
        if constexpr (GATHER) {
            int v = active[p];
            v = v < 0 ? 0 : (v >= i_dim ? i_dim - 1 : v);  // never read outside the matrices
            return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(v)) * rb;
        } else {
            return static_cast<uint32_t>(p - pbase) * rb;
        }
    };
    auto issue1 = [&](RowRaw& b, __amdgpu_buffer_rsrc_t r, uint32_t so) {
        b.a = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(va), static_cast<int>(so), CACHE_NT);
        b.b = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(vb), static_cast<int>(so), CACHE_NT);
        b.c = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(vc), static_cast<int>(so), CACHE_NT);
    };
    auto issue = [&](Pair& b, int s) {
        const uint32_t so = soff(s);
        issue1(b.g, rg, so);
        issue1(b.u, ru, so);
    };
    auto stage = [&](const RowRaw& b) -> RowBuf {
        rbuf[lane] = b.a;
        rbuf[64 + lane] = b.b;
        rbuf[pc] = b.c;
        RowBuf r;
        r.hdr = rbuf[sh];
        r.qa = rbuf[sq];
        r.qb = rbuf[sq + 1];
        return r;
    };

    // x (and the norm weights) first, then the first neurons' rows, then the
    // norm and the encode
    float xv[8];
    [[maybe_unused]] float nv[8];
    const int task = static_cast<int>(threadIdx.x);
    const int tu = task >> 3;
    {
        const int off = (tu < units ? tu : units - 1) * 64 + 8 * (task & 7);
        const float4 a = *reinterpret_cast<const float4*>(x + off);
        const float4 b = *reinterpret_cast<const float4*>(x + off + 4);
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
        if constexpr (NORM) {
            const float4 c = *reinterpret_cast<const float4*>(norm_w + off);
            const float4 d = *reinterpret_cast<const float4*>(norm_w + off + 4);
            nv[0] = c.x; nv[1] = c.y; nv[2] = c.z; nv[3] = c.w;
            nv[4] = d.x; nv[5] = d.y; nv[6] = d.z; nv[7] = d.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    Pair ring[NS];
#pragma unroll
    for (int s = 0; s < NS - 1 && s < NPW; s++) issue(ring[s], s);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) ss += xv[i] * xv[i];
        ss = wave_sum_dpp(tu < units ? ss : 0.f);
        if (lane == 0) wsum[wave] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) tot += wsum[i];
        const float rinv = 1.0f / sqrtf(tot / static_cast<float>(units * 64) + eps);
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = xv[i] * rinv * nv[i];
    }
    encode_task(xv, task, units, xq);
    __syncthreads();
    const XU xu = read_unit(xq, u);
    const ScaleSel ss = make_sel(u & 3);

    float ag[8], au[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        ag[s] = 0.f;
        au[s] = 0.f;
    }
#pragma unroll
    for (int s = 0; s < NPW; s++) {
        if (s + NS - 1 < NPW) issue(ring[(s + NS - 1) % NS], s + NS - 1);
        const float pg = row_part(stage(ring[s % NS].g), xu, ss);
        const float pu = row_part(stage(ring[s % NS].u), xu, ss);
        ag[s] = valid ? pg : 0.f;
        au[s] = valid ? pu : 0.f;
        __builtin_amdgcn_sched_barrier(0);
    }
    const float tg = reduce8(ag);
    const float tv = reduce8(au);
    const int r = row_of_group(lane >> 3);
    if ((lane & 7) == 0 && r < NPW && p0 + r < n_act) {
        if constexpr (GATHER) {
            const int v = active[p0 + r];
            if (v >= 0 && v < i_dim) y[v] = act_pair(tg, tv, kind);
        } else {
            y[p0 + r] = act_pair(tg, tv, kind);
        }
    }
}

struct PairsArgs {
    const void *wg, *wu;
    const float *x, *norm_w;
    float eps;
    int kind;
    float* y;
    int n, units;
    uint32_t rb;
    const int32_t *active, *n_dev;  // gathered rows (active != nullptr)
    int i_dim;
};

template <int NPW, int NS, bool NORM, bool GATHER>
void launch_pairs_k(const PairsArgs& a, hipStream_t st) {
    const int grid = (a.n + 8 * NPW - 1) / (8 * NPW);
    gemv_q4k_pairs_kernel<NPW, NS, NORM, GATHER><<<dim3(static_cast<uint32_t>(grid)), dim3(512), 0, st>>>(
        static_cast<const uint8_t*>(a.wg), static_cast<const uint8_t*>(a.wu), a.x, a.norm_w, a.eps, a.kind, a.y, a.n,
        a.units, a.rb, a.active, a.n_dev, a.i_dim);
}

template <int NPW, int NS>
void launch_pairs(const PairsArgs& a, hipStream_t st) {
    const bool norm = a.norm_w != nullptr, gather = a.active != nullptr;
    if (gather)
        norm ? launch_pairs_k<NPW, NS, true, true>(a, st) : launch_pairs_k<NPW, NS, false, true>(a, st);
    else
        norm ? launch_pairs_k<NPW, NS, true, false>(a, st) : launch_pairs_k<NPW, NS, false, false>(a, st);
}

template <int NS>
void launch_pairs_npw(int npw, const PairsArgs& a, hipStream_t st) {
    switch (npw) {
    case 1: launch_pairs<1, NS < 2 ? NS : 2>(a, st); break;
    case 2: launch_pairs<2, NS < 3 ? NS : 3>(a, st); break;
    case 3: launch_pairs<3, NS>(a, st); break;
    case 4: launch_pairs<4, NS>(a, st); break;
    case 5: launch_pairs<5, NS>(a, st); break;
    case 6: launch_pairs<6, NS>(a, st); break;
    case 7: launch_pairs<7, NS>(a, st); break;
    default: launch_pairs<8, NS>(a, st); break;
    }
}

// ---- split rows: 64 < units <= 256 (4096 < k <= 16384) ------------------------
//
// A row is split into SL slices of upw units (upw a multiple of 4, so slices
// start on super-block boundaries, 36 upw bytes each, upw <= 56); a 16-wave
// workgroup is 16 / SL row groups x SL slices, and wave (group, slice) takes
// slice `slice` of the group's RPW rows.  Per row the wave reads its slice
// contiguously (two 16-byte pieces per lane: at most 128 slots, 2016 B for 56
// units, fill the wave's 128-slot buffer), stages it through its
// LDS buffer and computes one unit per lane with the short kernel's
// arithmetic; the activation encoding covers all units of x.  Each wave
// reduces its rows at once (reduce8), the slices of a row meet in LDS and are
// added in slice order, and resid (optional, may be y) is added as y is
// written.
constexpr int SPLIT_US = 256;  // unit stride of the encoding (units <= 256)

// XH: x in fp16 (the one-row GEMM), widened to fp32 before the encode.
template <int RPW, int NS, int SL, bool XH = false>
__global__ void __launch_bounds__(1024) gemv_q4k_split_kernel(const uint8_t* __restrict__ w, const void* __restrict__ xp,
                                                              float* y, const float* resid, int n, int units, int upw,
                                                              uint32_t rb) {
    constexpr int WPG = 16;
    constexpr int NG = WPG / SL;  // row groups per workgroup
    __shared__ uint4 xq[XQ_UNIT_QUADS * SPLIT_US];
    __shared__ u32x4 rowbuf[WPG][128];
    __shared__ float red[NG][SL][8];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int grp = wave / SL, slc = wave - grp * SL;
    const int row0 = (static_cast<int>(blockIdx.x) * NG + grp) * RPW;
    const int rlast = n - 1;
    const int rbase = row0 < rlast ? row0 : rlast;
    // this wave's slice: units [u0, u0 + su) of each row, bytes [36 u0, +36 su)
    const int u0 = slc * upw;
    const int su = units - u0 < upw ? units - u0 : upw;  // >= 4 by the host's choice of SL
    const uint8_t* wb = w + static_cast<int64_t>(rbase) * rb + 36u * static_cast<uint32_t>(u0);
    const int64_t span64 = static_cast<int64_t>(n - rbase) * rb - 36 * static_cast<int64_t>(u0);
    const uint32_t span = span64 < 0xFFFFFFFFll ? static_cast<uint32_t>(span64) : 0xFFFFFFFFu;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(wb, span);
    const bool valid = lane < su;
    const int u = valid ? lane : (lane & 3);  // idle lanes read unit (lane % 4) of the slice, discarded
    const int sslots = 9 * su / 4;            // 16-byte slots of the slice
    const uint32_t va = 16u * static_cast<uint32_t>(lane < sslots ? lane : lane & 7);
    const uint32_t vb = 16u * static_cast<uint32_t>(64 + lane < sslots ? 64 + lane : lane & 7);
    u32x4* rbuf = rowbuf[wave];
    const int sh = 9 * (u >> 2), sq = sh + 1 + 2 * (u & 3);

    auto soff = [&](int s) -> uint32_t {
        int r = row0 + s;
        r = r < rlast ? r : rlast;
        return static_cast<uint32_t>(r - rbase) * rb;
    };
    struct Raw2 { u32x4 a, b; };
    auto issue = [&](Raw2& b, int s) {
        const uint32_t so = soff(s);
        b.a = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(va), static_cast<int>(so), CACHE_NT);
        b.b = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(vb), static_cast<int>(so), CACHE_NT);
    };
    auto stage = [&](const Raw2& b) -> RowBuf {
        rbuf[lane] = b.a;
        rbuf[64 + lane] = b.b;
        RowBuf r;
        r.hdr = rbuf[sh];
        r.qa = rbuf[sq];
        r.qb = rbuf[sq + 1];
        return r;
    };

    // x first (8 tasks per unit, up to 2048 tasks: 2 per thread), then the
    // first rows' weights, then the branch-free encode
    float xv[2][8];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int task = static_cast<int>(threadIdx.x) + 1024 * t;
        const int tu = task >> 3;
        const int off = (tu < units ? tu : units - 1) * 64 + 8 * (task & 7);
        if constexpr (XH) {
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 hv = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(xp) + off);
#pragma unroll
            for (int i = 0; i < 8; i++) xv[t][i] = static_cast<float>(hv[i]);
        } else {
            const float* x = static_cast<const float*>(xp);
            const float4 a = *reinterpret_cast<const float4*>(x + off);
            const float4 b = *reinterpret_cast<const float4*>(x + off + 4);
            xv[t][0] = a.x; xv[t][1] = a.y; xv[t][2] = a.z; xv[t][3] = a.w;
            xv[t][4] = b.x; xv[t][5] = b.y; xv[t][6] = b.z; xv[t][7] = b.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    Raw2 ring[NS];
#pragma unroll
    for (int s = 0; s < NS - 1 && s < RPW; s++) issue(ring[s], s);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 2; t++) encode_task<SPLIT_US>(xv[t], static_cast<int>(threadIdx.x) + 1024 * t, units, xq);
    __syncthreads();
    const XU xu = read_unit<SPLIT_US>(xq, u0 + u);
    const ScaleSel ss = make_sel(u & 3);

    float acc[8];
#pragma unroll
    for (int s = 0; s < 8; s++) acc[s] = 0.f;
#pragma unroll
    for (int s = 0; s < RPW; s++) {
        if (s + NS - 1 < RPW) issue(ring[(s + NS - 1) % NS], s + NS - 1);
        const float part = row_part(stage(ring[s % NS]), xu, ss);
        acc[s] = valid ? part : 0.f;  // idle lanes: nothing, even from a non-finite scale
        __builtin_amdgcn_sched_barrier(0);
    }
    const float tot = reduce8(acc);
    const int g8 = lane >> 3;
    const int rr = row_of_group(g8);
    if ((lane & 7) == 0 && rr < RPW) red[grp][slc][rr] = tot;
    __syncthreads();
    if (threadIdx.x < NG * RPW) {
        const int gq = static_cast<int>(threadIdx.x) / RPW, r = static_cast<int>(threadIdx.x) - gq * RPW;
        const int row = (static_cast<int>(blockIdx.x) * NG + gq) * RPW + r;
        if (row < n) {
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < SL; j++) v += red[gq][j][r];
            y[row] = resid ? v + resid[row] : v;  // resid may be y: read before the write
        }
    }
}

// The split-row kernel with the slices landing in LDS by DMA (fp32 x), as
// gemv_q4k_dma_kernel does for short rows: one __shared__ array per ring
// slot, the encode written with asm stores and published with lgkmcnt(0) and
// a bare s_barrier, explicit vmcnt waits for each row.  Same arithmetic and
// results as gemv_q4k_split_kernel.
template <int RPW, int NS, int SL>
__global__ void __launch_bounds__(1024) gemv_q4k_split_dma_kernel(const uint8_t* __restrict__ w,
                                                                  const float* __restrict__ x, float* y,
                                                                  const float* resid, int n, int units, int upw,
                                                                  uint32_t rb) {
    static_assert(NS >= 2 && NS <= 3, "ring of 2..3 slices");
    constexpr int WPG = 16;
    constexpr int NG = WPG / SL;
    __shared__ uint4 xq[XQ_UNIT_QUADS * SPLIT_US];
    __shared__ u32x4 ring0[WPG][128], ring1[WPG][128], ring2[WPG][128];
    __shared__ float red[NG][SL][8];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int grp = wave / SL, slc = wave - grp * SL;
    const int row0 = (static_cast<int>(blockIdx.x) * NG + grp) * RPW;
    const int rlast = n - 1;
    const int rbase = row0 < rlast ? row0 : rlast;
    const int u0 = slc * upw;
    const int su = units - u0 < upw ? units - u0 : upw;
    const uint8_t* wb = w + static_cast<int64_t>(rbase) * rb + 36u * static_cast<uint32_t>(u0);
    const int64_t span64 = static_cast<int64_t>(n - rbase) * rb - 36 * static_cast<int64_t>(u0);
    const uint32_t span = span64 < 0xFFFFFFFFll ? static_cast<uint32_t>(span64) : 0xFFFFFFFFu;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(wb, span);
    const bool valid = lane < su;
    const int u = valid ? lane : (lane & 3);
    const int sslots = 9 * su / 4;
    const uint32_t va = 16u * static_cast<uint32_t>(lane < sslots ? lane : lane & 7);
    const uint32_t vb = 16u * static_cast<uint32_t>(64 + lane < sslots ? 64 + lane : lane & 7);
    const int sh = 9 * (u >> 2), sq = sh + 1 + 2 * (u & 3);

    auto slot_base = [&](auto k_c) __attribute__((always_inline)) -> u32x4* {
        constexpr int k = decltype(k_c)::value;
        if constexpr (k == 0) return ring0[wave];
        else if constexpr (k == 1) return ring1[wave];
        else return ring2[wave];
    };
    auto issue = [&](auto k_c, int s) __attribute__((always_inline)) {
        int r = row0 + s;
        r = r < rlast ? r : rlast;
        const uint32_t so = static_cast<uint32_t>(r - rbase) * rb;
        u32x4* b = slot_base(k_c);
        typedef __attribute__((address_space(3))) void* lds_ptr;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)b, 16, static_cast<int>(va), static_cast<int>(so), 0,
                                                 CACHE_NT);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(b + 64), 16, static_cast<int>(vb),
                                                 static_cast<int>(so), 0, CACHE_NT);
    };

    float xv[2][8];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int task = static_cast<int>(threadIdx.x) + 1024 * t;
        const int tu = task >> 3;
        const int off = (tu < units ? tu : units - 1) * 64 + 8 * (task & 7);
        const float4 a = *reinterpret_cast<const float4*>(x + off);
        const float4 b = *reinterpret_cast<const float4*>(x + off + 4);
        xv[t][0] = a.x; xv[t][1] = a.y; xv[t][2] = a.z; xv[t][3] = a.w;
        xv[t][4] = b.x; xv[t][5] = b.y; xv[t][6] = b.z; xv[t][7] = b.w;
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NS - 1 >= 1) issue(std::integral_constant<int, 0>{}, 0);
    if constexpr (NS - 1 >= 2) if (1 < RPW) issue(std::integral_constant<int, 1>{}, 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 2; t++)
        encode_task<SPLIT_US, true>(xv[t], static_cast<int>(threadIdx.x) + 1024 * t, units, xq);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the encode is in LDS
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const XU xu = read_unit<SPLIT_US>(xq, u0 + u);
    const ScaleSel ss = make_sel(u & 3);

    float acc[8];
#pragma unroll
    for (int s = 0; s < 8; s++) acc[s] = 0.f;
    auto step = [&](auto s_c) __attribute__((always_inline)) {
        constexpr int s = decltype(s_c)::value;
        if constexpr (s < RPW) {
            if constexpr (s + NS - 1 < RPW) issue(std::integral_constant<int, (s + NS - 1) % NS>{}, s + NS - 1);
            constexpr int after = 2 * (s + NS - 1 < RPW ? NS - 1 : RPW - 1 - s);
            __builtin_amdgcn_s_waitcnt(0x0F70 | after);
            const u32x4* b = slot_base(std::integral_constant<int, s % NS>{});
            RowBuf rw;
            rw.hdr = b[sh];
            rw.qa = b[sq];
            rw.qb = b[sq + 1];
            const float part = row_part(rw, xu, ss);
            acc[s] = valid ? part : 0.f;
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
    step(std::integral_constant<int, 4>{});
    step(std::integral_constant<int, 5>{});
    step(std::integral_constant<int, 6>{});
    step(std::integral_constant<int, 7>{});
    const float tot = reduce8(acc);
    const int g8 = lane >> 3;
    const int rr = row_of_group(g8);
    if ((lane & 7) == 0 && rr < RPW) red[grp][slc][rr] = tot;
    __syncthreads();
    if (threadIdx.x < NG * RPW) {
        const int gq = static_cast<int>(threadIdx.x) / RPW, r = static_cast<int>(threadIdx.x) - gq * RPW;
        const int row = (static_cast<int>(blockIdx.x) * NG + gq) * RPW + r;
        if (row < n) {
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < SL; j++) v += red[gq][j][r];
            y[row] = resid ? v + resid[row] : v;
        }
    }
}

// Split rows for Q6_K / Q8_0 (4096 < k <= 16384): the Q4_K split-row kernel's
// work split with the short-row Q6_K / Q8_0 units (ShortRow).  A slice of
// upw units starts on a 4-byte boundary (Q6_K: an even super-block), is read
// as P contiguous 16-byte pieces per lane from there (its last piece may run
// a few bytes past the slice: unread) and staged in the wave's row buffer.
// XH: x in fp16 (the one-row GEMM), widened to fp32 before the encode.
template <int TYPE, int RPW, int NS, int SL, bool XH = false>
__global__ void __launch_bounds__(1024) gemv_split_kernel(const uint8_t* __restrict__ w, const void* __restrict__ xp,
                                                          float* y, const float* resid, int n, int units, int upw,
                                                          uint32_t rb) {
    using T = ShortRow<TYPE>;
    constexpr int WPG = 16;
    constexpr int NG = WPG / SL;                      // row groups per workgroup
    constexpr int P = (T::bytes(56) + 15 + 1023) / 1024;  // pieces per lane of a slice of at most 56 units
    __shared__ uint4 xq[T::XQUADS * SPLIT_US];
    __shared__ u32x4 rowbuf[WPG][64 * P];
    __shared__ float red[NG][SL][8];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int grp = wave / SL, slc = wave - grp * SL;
    const int row0 = (static_cast<int>(blockIdx.x) * NG + grp) * RPW;
    const int rlast = n - 1;
    const int rbase = row0 < rlast ? row0 : rlast;
    // this wave's slice: units [u0, u0 + su) of each row
    const int u0 = slc * upw;
    const int su = units - u0 < upw ? units - u0 : upw;  // >= 4 by the host's choice of SL
    const uint32_t sb0 = static_cast<uint32_t>(T::bytes(u0));
    const uint8_t* wb = w + static_cast<int64_t>(rbase) * rb + sb0;
    const int64_t span64 = static_cast<int64_t>(n - rbase) * rb - sb0;
    const uint32_t span = span64 < 0xFFFFFFFFll ? static_cast<uint32_t>(span64) : 0xFFFFFFFFu;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(wb, span);
    const bool valid = lane < su;
    const int u = valid ? lane : (lane & 3);  // idle lanes read unit (lane % 4) of the slice, discarded
    const int sslots = (T::bytes(su) + 15) / 16;  // 16-byte slots of the slice
    uint32_t vo[P];
#pragma unroll
    for (int p = 0; p < P; p++) vo[p] = 16u * static_cast<uint32_t>(64 * p + lane < sslots ? 64 * p + lane : lane & 7);
    u32x4* rbuf = rowbuf[wave];
    const typename T::Addr ad = T::addr(reinterpret_cast<const uint8_t*>(rbuf), u);

    auto soff = [&](int s) -> uint32_t {
        int r = row0 + s;
        r = r < rlast ? r : rlast;
        return static_cast<uint32_t>(r - rbase) * rb;
    };
    struct Raw { u32x4 p[P]; };
    auto issue = [&](Raw& b, int s) {
        const uint32_t so = soff(s);
#pragma unroll
        for (int p = 0; p < P; p++)
            b.p[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(vo[p]), static_cast<int>(so), CACHE_NT);
    };
    auto stage = [&](const Raw& b) {
#pragma unroll
        for (int p = 0; p < P; p++) rbuf[64 * p + lane] = b.p[p];
        return T::read(ad);
    };

    // x first (8 tasks per unit, up to 2048 tasks: 2 per thread), then the
    // first rows' weights, then the branch-free encode
    float xv[2][8];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int task = static_cast<int>(threadIdx.x) + 1024 * t;
        const int tu = task >> 3;
        const int off = T::x_off(tu < units ? tu : units - 1, task & 7);
        if constexpr (XH) {
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 hv = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(xp) + off);
#pragma unroll
            for (int i = 0; i < 8; i++) xv[t][i] = static_cast<float>(hv[i]);
        } else {
            const float* x = static_cast<const float*>(xp);
            const float4 a = *reinterpret_cast<const float4*>(x + off);
            const float4 b = *reinterpret_cast<const float4*>(x + off + 4);
            xv[t][0] = a.x; xv[t][1] = a.y; xv[t][2] = a.z; xv[t][3] = a.w;
            xv[t][4] = b.x; xv[t][5] = b.y; xv[t][6] = b.z; xv[t][7] = b.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    Raw ring[NS];
#pragma unroll
    for (int s = 0; s < NS - 1 && s < RPW; s++) issue(ring[s], s);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 2; t++)
        T::template encode<SPLIT_US>(xv[t], static_cast<int>(threadIdx.x) + 1024 * t, units, xq);
    __syncthreads();
    const typename T::X xu = T::template read_x<SPLIT_US>(xq, u0 + u);

    float acc[8];
#pragma unroll
    for (int s = 0; s < 8; s++) acc[s] = 0.f;
#pragma unroll
    for (int s = 0; s < RPW; s++) {
        if (s + NS - 1 < RPW) issue(ring[(s + NS - 1) % NS], s + NS - 1);
        const float part = T::part(stage(ring[s % NS]), xu);
        acc[s] = valid ? part : 0.f;
        __builtin_amdgcn_sched_barrier(0);
    }
    const float tot = reduce8(acc);
    const int rr = row_of_group(lane >> 3);
    if ((lane & 7) == 0 && rr < RPW) red[grp][slc][rr] = tot;
    __syncthreads();
    if (threadIdx.x < NG * RPW) {
        const int gq = static_cast<int>(threadIdx.x) / RPW, r = static_cast<int>(threadIdx.x) - gq * RPW;
        const int row = (static_cast<int>(blockIdx.x) * NG + gq) * RPW + r;
        if (row < n) {
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < SL; j++) v += red[gq][j][r];
            y[row] = resid ? v + resid[row] : v;  // resid may be y: read before the write
        }
    }
}

template <int TYPE, int RPW, int D, int SL, bool XH>
void launch_tsplit(const void* w, const void* x, float* y, const float* resid, int n, int units, int upw,
                   uint32_t rb, hipStream_t st) {
    constexpr int NG = 16 / SL;
    constexpr int NS = (RPW < D ? RPW : D) + 1;
    const int grid = (n + NG * RPW - 1) / (NG * RPW);
    gemv_split_kernel<TYPE, RPW, NS, SL, XH><<<dim3(static_cast<uint32_t>(grid)), dim3(1024), 0, st>>>(
        static_cast<const uint8_t*>(w), x, y, resid, n, units, upw, rb);
}

template <int TYPE, int D, int SL, bool XH = false>
void launch_tsplit_rpw(int rpw, const void* w, const void* x, float* y, const float* resid, int n, int units,
                       int upw, uint32_t rb, hipStream_t st) {
    switch (rpw) {
    case 1: launch_tsplit<TYPE, 1, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 2: launch_tsplit<TYPE, 2, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 3: launch_tsplit<TYPE, 3, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 4: launch_tsplit<TYPE, 4, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 5: launch_tsplit<TYPE, 5, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 6: launch_tsplit<TYPE, 6, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 7: launch_tsplit<TYPE, 7, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    default: launch_tsplit<TYPE, 8, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    }
}

template <int TYPE, int SL>
void launch_tsplit_d(int d, int rpw, const void* w, const void* x, float* y, const float* resid, int n, int units,
                     int upw, uint32_t rb, hipStream_t st) {
    switch (d) {
    case 1: launch_tsplit_rpw<TYPE, 1, SL>(rpw, w, x, y, resid, n, units, upw, rb, st); break;
    case 3: launch_tsplit_rpw<TYPE, 3, SL>(rpw, w, x, y, resid, n, units, upw, rb, st); break;
    default: launch_tsplit_rpw<TYPE, 2, SL>(rpw, w, x, y, resid, n, units, upw, rb, st); break;
    }
}

template <int RPW, int D, int SL, bool XH>
void launch_split(const void* w, const void* x, float* y, const float* resid, int n, int units, int upw,
                  uint32_t rb, hipStream_t st) {
    constexpr int NG = 16 / SL;
    constexpr int NS = (RPW < D ? RPW : D) + 1;  // ring: NS - 1 (at most D) rows in flight while computing
    const int grid = (n + NG * RPW - 1) / (NG * RPW);
    gemv_q4k_split_kernel<RPW, NS, SL, XH><<<dim3(static_cast<uint32_t>(grid)), dim3(1024), 0, st>>>(
        static_cast<const uint8_t*>(w), x, y, resid, n, units, upw, rb);
}

template <int D, int SL>
void launch_split_dma_rpw(int rpw, const void* w, const float* x, float* y, const float* resid, int n, int units,
                          int upw, uint32_t rb, hipStream_t st) {
    constexpr int NG = 16 / SL;
    const int grid = (n + NG * rpw - 1) / (NG * rpw);
    const dim3 g(static_cast<uint32_t>(grid)), b(1024);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (rpw) {
    case 1: gemv_q4k_split_dma_kernel<1, 2, SL><<<g, b, 0, st>>>(wb, x, y, resid, n, units, upw, rb); break;
    case 2: gemv_q4k_split_dma_kernel<2, (D < 2 ? D : 2) + 1, SL><<<g, b, 0, st>>>(wb, x, y, resid, n, units, upw, rb); break;
    case 3: gemv_q4k_split_dma_kernel<3, D + 1, SL><<<g, b, 0, st>>>(wb, x, y, resid, n, units, upw, rb); break;
    case 4: gemv_q4k_split_dma_kernel<4, D + 1, SL><<<g, b, 0, st>>>(wb, x, y, resid, n, units, upw, rb); break;
    case 5: gemv_q4k_split_dma_kernel<5, D + 1, SL><<<g, b, 0, st>>>(wb, x, y, resid, n, units, upw, rb); break;
    case 6: gemv_q4k_split_dma_kernel<6, D + 1, SL><<<g, b, 0, st>>>(wb, x, y, resid, n, units, upw, rb); break;
    case 7: gemv_q4k_split_dma_kernel<7, D + 1, SL><<<g, b, 0, st>>>(wb, x, y, resid, n, units, upw, rb); break;
    default: gemv_q4k_split_dma_kernel<8, D + 1, SL><<<g, b, 0, st>>>(wb, x, y, resid, n, units, upw, rb); break;
    }
}

template <int D, int SL, bool XH = false>
void launch_split_rpw(int rpw, const void* w, const void* x, float* y, const float* resid, int n, int units,
                      int upw, uint32_t rb, hipStream_t st) {
    switch (rpw) {
    case 1: launch_split<1, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 2: launch_split<2, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 3: launch_split<3, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 4: launch_split<4, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 5: launch_split<5, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 6: launch_split<6, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    case 7: launch_split<7, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    default: launch_split<8, D, SL, XH>(w, x, y, resid, n, units, upw, rb, st); break;
    }
}

template <int SL>
void launch_split_d(int d, int rpw, const void* w, const void* x, float* y, const float* resid, int n, int units,
                    int upw, uint32_t rb, hipStream_t st) {
    switch (d) {
    case 1: launch_split_rpw<1, SL>(rpw, w, x, y, resid, n, units, upw, rb, st); break;
    case 3: launch_split_rpw<3, SL>(rpw, w, x, y, resid, n, units, upw, rb, st); break;
    case 4: launch_split_rpw<4, SL>(rpw, w, x, y, resid, n, units, upw, rb, st); break;
    default: launch_split_rpw<2, SL>(rpw, w, x, y, resid, n, units, upw, rb, st); break;
    }
}

template <int RPW, int NS, int WPG, bool XH = false>
void launch(const void* w, const void* x, float* y, int n, int units, uint32_t rb, hipStream_t st) {
    const int grid = (n + WPG * RPW - 1) / (WPG * RPW);
    gemv_q4k_kernel<RPW, NS, WPG, XH><<<dim3(static_cast<uint32_t>(grid)), dim3(64 * WPG), 0, st>>>(
        static_cast<const uint8_t*>(w), x, y, n, units, rb);
}

template <int NS, int WPG, bool XH = false>
void launch_rpw(int rpw, const void* w, const void* x, float* y, int n, int units, uint32_t rb, hipStream_t st) {
    switch (rpw) {
    case 1: launch<1, NS, WPG, XH>(w, x, y, n, units, rb, st); break;
    case 2: launch<2, NS, WPG, XH>(w, x, y, n, units, rb, st); break;
    case 3: launch<3, NS, WPG, XH>(w, x, y, n, units, rb, st); break;
    case 4: launch<4, NS, WPG, XH>(w, x, y, n, units, rb, st); break;
    case 5: launch<5, NS, WPG, XH>(w, x, y, n, units, rb, st); break;
    case 6: launch<6, NS, WPG, XH>(w, x, y, n, units, rb, st); break;
    case 7: launch<7, NS, WPG, XH>(w, x, y, n, units, rb, st); break;
    default: launch<8, NS, WPG, XH>(w, x, y, n, units, rb, st); break;
    }
}

template <int NS>
void launch_dma_rpw(int rpw, const void* w, const float* x, float* y, int n, int units, uint32_t rb,
                    hipStream_t st) {
    const int grid = (n + 8 * rpw - 1) / (8 * rpw);
    const dim3 g(static_cast<uint32_t>(grid)), b(512);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (rpw) {
    case 1: gemv_q4k_dma_kernel<1, NS><<<g, b, 0, st>>>(wb, x, y, n, units, rb); break;
    case 2: gemv_q4k_dma_kernel<2, NS><<<g, b, 0, st>>>(wb, x, y, n, units, rb); break;
    case 3: gemv_q4k_dma_kernel<3, NS><<<g, b, 0, st>>>(wb, x, y, n, units, rb); break;
    case 4: gemv_q4k_dma_kernel<4, NS><<<g, b, 0, st>>>(wb, x, y, n, units, rb); break;
    case 5: gemv_q4k_dma_kernel<5, NS><<<g, b, 0, st>>>(wb, x, y, n, units, rb); break;
    case 6: gemv_q4k_dma_kernel<6, NS><<<g, b, 0, st>>>(wb, x, y, n, units, rb); break;
    case 7: gemv_q4k_dma_kernel<7, NS><<<g, b, 0, st>>>(wb, x, y, n, units, rb); break;
    default: gemv_q4k_dma_kernel<8, NS><<<g, b, 0, st>>>(wb, x, y, n, units, rb); break;
    }
}

template <int TYPE, int G, int NS, bool XH>
void launch_short(const void* w, const void* x, float* y, int n, int units, uint32_t rb, int rpw,
                  hipStream_t st) {
    const int grid = (n + 8 * rpw - 1) / (8 * rpw);
    gemv_short_kernel<TYPE, G, NS, XH><<<dim3(static_cast<uint32_t>(grid)), dim3(512), 0, st>>>(
        static_cast<const uint8_t*>(w), x, y, n, units, rb, rpw);
}

// rpw <= 8: one group of rpw rows; above, groups of 8 rows (NS divides 8)
template <int TYPE, int NS, bool XH = false>
void launch_short_rpw(int rpw, const void* w, const void* x, float* y, int n, int units, uint32_t rb,
                      hipStream_t st) {
    switch (rpw) {
    case 1: launch_short<TYPE, 1, NS, XH>(w, x, y, n, units, rb, rpw, st); break;
    case 2: launch_short<TYPE, 2, NS, XH>(w, x, y, n, units, rb, rpw, st); break;
    case 3: launch_short<TYPE, 3, NS, XH>(w, x, y, n, units, rb, rpw, st); break;
    case 4: launch_short<TYPE, 4, NS, XH>(w, x, y, n, units, rb, rpw, st); break;
    case 5: launch_short<TYPE, 5, NS, XH>(w, x, y, n, units, rb, rpw, st); break;
    case 6: launch_short<TYPE, 6, NS, XH>(w, x, y, n, units, rb, rpw, st); break;
    case 7: launch_short<TYPE, 7, NS, XH>(w, x, y, n, units, rb, rpw, st); break;
    default: launch_short<TYPE, 8, NS, XH>(w, x, y, n, units, rb, rpw, st); break;
    }
}

template <int TYPE>
void launch_short_ns(int ns, int rpw, const void* w, const void* x, float* y, int n, int units, uint32_t rb,
                     hipStream_t st) {
    if (ns == 2) launch_short_rpw<TYPE, 2>(rpw, w, x, y, n, units, rb, st);
    else if (ns == 3) launch_short_rpw<TYPE, 3>(rpw, w, x, y, n, units, rb, st);
    else launch_short_rpw<TYPE, 4>(rpw, w, x, y, n, units, rb, st);
}

// Launch shape for n rows: 8-wave workgroups, one per CU, with RPW =
// ceil(n / (8 CUs)) <= 8 rows per wave (14336 rows: 7); 16-wave workgroups
// for up to 16 x 8 rows per CU (measured at 14336 x 4096: 16 waves of 4 rows,
// 224 workgroups, ran 8.1-8.3 us against 7.4 us).  VB_GEMV_CFG="wpg,rpw"
// overrides (wpg 8 or 16).  rpw 0: more than 8 rows per wave (the caller
// takes the general kernel).
struct ShortShape { int wpg, rpw; };

ShortShape short_shape(int64_t n) {
    const int64_t cus = num_cus();
    ShortShape s{8, 0};
    const Knobs& kb = knobs();
    if (kb.gemv_cfg_wpg == 8 || kb.gemv_cfg_wpg == 16) {
        s.wpg = kb.gemv_cfg_wpg;
        s.rpw = kb.gemv_cfg_rpg >= 1 && kb.gemv_cfg_rpg <= 8 ? kb.gemv_cfg_rpg : 0;
        if (s.rpw) return s;
    }
    int64_t rpw = (n + cus * s.wpg - 1) / (cus * s.wpg);
    if (rpw > 8) {  // past 8 rows per wave: 16-wave workgroups, up to 8 rows each
        s.wpg = 16;
        rpw = (n + cus * s.wpg - 1) / (cus * s.wpg);
        if (rpw > 8) {
            s.rpw = 0;
            return s;
        }
    }
    s.rpw = static_cast<int>(rpw < 1 ? 1 : rpw);
    return s;
}

}  // namespace

int gemv_q4k_rpw(int64_t n) { return short_shape(n).rpw; }

// Plain Q4_K GEMV, k <= 4096 (k % 256 == 0), at most 8 rows per wave of one
// workgroup per CU; arguments validated by gemv_dispatch_fused.
int gemv_q4k_short(const void* w, const void* x, float* y, int64_t n, int64_t k, hipStream_t st, bool x_half) {
    const ShortShape sh = short_shape(n);
    const int units = static_cast<int>(k / 64);
    if (sh.rpw == 0 || units > UNITS_MAX || k % 256 != 0 || n > INT32_MAX) {
        set_error("vb_gemv: internal: Q4_K short-row kernel shape (n=%lld, k=%lld)", static_cast<long long>(n),
                  static_cast<long long>(k));
        return E_INVAL;
    }
    const uint32_t rb = static_cast<uint32_t>(row_bytes(TYPE_Q4_K, k));
    const int ni = static_cast<int>(n);
    if (x_half) {  // fp16 x (a one-row GEMM): the default ring only
        if (sh.wpg == 8)
            launch_rpw<4, 8, true>(sh.rpw, w, x, y, ni, units, rb, st);
        else
            launch_rpw<4, 16, true>(sh.rpw, w, x, y, ni, units, rb, st);
        return check_launch("vb_gemm");
    }
    // NS - 1 rows in flight while computing: default 2 with the rows landing
    // in LDS by DMA, 3 with the register ring (VB_GEMV_DMA=0).  On MI355X at
    // 14336 x 4096: DMA 6.98 us (ring 2), 7.07-7.09 (ring 3), 7.15 (ring 4);
    // register ring 7.24 us.
    const int ring = knobs().gemv_ring;
    if (sh.wpg == 8 && knobs().gemv_dma) {
        const float* xf = static_cast<const float*>(x);
        if (ring == 1) launch_dma_rpw<2>(sh.rpw, w, xf, y, ni, units, rb, st);
        else if (ring == 3) launch_dma_rpw<4>(sh.rpw, w, xf, y, ni, units, rb, st);
        else if (ring >= 4) launch_dma_rpw<5>(sh.rpw, w, xf, y, ni, units, rb, st);
        else launch_dma_rpw<3>(sh.rpw, w, xf, y, ni, units, rb, st);
        return check_launch("vb_gemv");
    }
    if (sh.wpg == 8) {
        if (ring == 1) launch_rpw<2, 8>(sh.rpw, w, x, y, ni, units, rb, st);
        else if (ring == 2) launch_rpw<3, 8>(sh.rpw, w, x, y, ni, units, rb, st);
        else if (ring == 4) launch_rpw<5, 8>(sh.rpw, w, x, y, ni, units, rb, st);
        else if (ring >= 5) launch_rpw<6, 8>(sh.rpw, w, x, y, ni, units, rb, st);
        else launch_rpw<4, 8>(sh.rpw, w, x, y, ni, units, rb, st);
    } else {
        if (ring == 1) launch_rpw<2, 16>(sh.rpw, w, x, y, ni, units, rb, st);
        else if (ring == 2) launch_rpw<3, 16>(sh.rpw, w, x, y, ni, units, rb, st);
        else launch_rpw<4, 16>(sh.rpw, w, x, y, ni, units, rb, st);
    }
    return check_launch("vb_gemv");
}

// Short-row Q6_K / Q8_0 kernel: rows per wave for n rows of k elements (one
// 8-wave workgroup per CU; VB_GEMV_CFG="8,rpw" overrides), 0 for shapes it
// does not take: rows must be whole 16-byte slots (Q6_K: k = 2048 or 4096;
// Q8_0: k % 256 == 0, k <= 4096).
int gemv_short_rpw(int32_t type, int64_t n, int64_t k) {
    const bool ok = type == TYPE_Q6_K ? (k == 2048 || k == 4096)
                  : type == TYPE_Q8_0 ? (k % 256 == 0 && k >= 256 && k <= 4096) : false;
    if (!ok || n < 1 || n > INT32_MAX) return 0;
    const Knobs& kb = knobs();
    if (kb.gemv_cfg_wpg == 8 && kb.gemv_cfg_rpg >= 1 && kb.gemv_cfg_rpg <= 4096) return kb.gemv_cfg_rpg;
    const int64_t groups = static_cast<int64_t>(num_cus()) * 8;
    const int64_t rpw = (n + groups - 1) / groups;
    return rpw <= 4096 ? static_cast<int>(rpw) : 0;
}

// Plain Q6_K / Q8_0 GEMV on the short-row kernel, 16-byte aligned rows;
// arguments validated by gemv_dispatch_fused.
int gemv_short(int32_t type, const void* w, const void* x, float* y, int64_t n, int64_t k, hipStream_t st,
               bool x_half) {
    const int rpw = gemv_short_rpw(type, n, k);
    if (rpw == 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0) {
        set_error("vb_gemv: internal: short-row kernel shape (type %d, n=%lld, k=%lld)", type,
                  static_cast<long long>(n), static_cast<long long>(k));
        return E_INVAL;
    }
    const uint32_t rb = static_cast<uint32_t>(row_bytes(type, k));
    const int ni = static_cast<int>(n), units = static_cast<int>(k / 64);
    // NS - 1 rows in flight while computing (VB_GEMV_RING).  Q6_K default 1:
    // on MI355X 65.5 us at 128256 x 4096 against 66.9 us with 2 or 3, 9.4
    // against 9.8 / 10.1 us at 14336 x 4096.  Past 8 rows per wave the ring
    // must divide the 8-row groups.
    int ns = knobs().gemv_ring > 0 ? knobs().gemv_ring + 1 : 2;
    if (rpw > 8 && ns != 2) ns = 4;
    if (x_half) {
        // fp16 x (the one-row GEMM): the default ring only
        if (type == TYPE_Q6_K) launch_short_rpw<TYPE_Q6_K, 2, true>(rpw, w, x, y, ni, units, rb, st);
        else launch_short_rpw<TYPE_Q8_0, 2, true>(rpw, w, x, y, ni, units, rb, st);
        return check_launch("vb_gemm");
    }
    if (type == TYPE_Q6_K) launch_short_ns<TYPE_Q6_K>(ns, rpw, w, x, y, ni, units, rb, st);
    else launch_short_ns<TYPE_Q8_0>(ns, rpw, w, x, y, ni, units, rb, st);
    return check_launch("vb_gemv");
}

// Split-row shape: slices per row (2 up to 112 units, 4 up to 224, 8 above,
// so that a slice is at most 56 units; 16-wave workgroups of 8, 4 or 2 row
// groups) and rows per wave, one workgroup per CU when that covers n; 0 rows
// per wave past 8 or for a last slice under 4 units (the caller then takes
// the general kernel).
struct SplitShape { int sl, upw, rpw; };

SplitShape split_shape(int64_t n, int units) {
    SplitShape s{units <= 112 ? 2 : (units <= 224 ? 4 : 8), 0, 0};
    if (knobs().gemv_split_sl) s.sl = knobs().gemv_split_sl;
    s.upw = ((units + s.sl - 1) / s.sl + 3) & ~3;
    const int64_t groups = static_cast<int64_t>(num_cus()) * (16 / s.sl);
    const int64_t rpw = (n + groups - 1) / groups;
    s.rpw = rpw <= 8 ? static_cast<int>(rpw < 1 ? 1 : rpw) : 0;
    if (s.upw > 56 || units - (s.sl - 1) * s.upw < 4) s.rpw = 0;
    return s;
}

int gemv_q4k_split_rpw(int64_t n, int64_t k) {
    const int units = static_cast<int>(k / 64);
    return units > UNITS_MAX && units <= SPLIT_US ? split_shape(n, units).rpw : 0;
}

// Plain or residual-epilogue Q4_K GEMV, 4096 < k <= 16384, k % 256 == 0, at
// most 8 rows per wave; arguments validated by gemv_dispatch_fused.
int gemv_q4k_split(const void* w, const void* x, float* y, const float* resid, int64_t n, int64_t k,
                   hipStream_t st, bool x_half) {
    const int units = static_cast<int>(k / 64);
    const SplitShape sh = split_shape(n, units);
    if (sh.rpw == 0 || units <= UNITS_MAX || units > SPLIT_US || k % 256 != 0 || n > INT32_MAX) {
        set_error("vb_gemv: internal: Q4_K split-row kernel shape (n=%lld, k=%lld)", static_cast<long long>(n),
                  static_cast<long long>(k));
        return E_INVAL;
    }
    const uint32_t rb = static_cast<uint32_t>(row_bytes(TYPE_Q4_K, k));
    const int ni = static_cast<int>(n);
    if (x_half) {
        // fp16 x (the one-row GEMM): the default ring only
        if (sh.sl == 2)
            launch_split_rpw<2, 2, true>(sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
        else if (sh.sl == 4)
            launch_split_rpw<2, 4, true>(sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
        else
            launch_split_rpw<2, 8, true>(sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
        return check_launch("vb_gemm");
    }
    const int d = knobs().gemv_split_d;
    if (knobs().gemv_dma && d <= 2) {
        // the slices land in LDS by DMA (rows in flight: 2, or 1 with VB_GEMV_SPLIT="sl,1")
        const float* xf = static_cast<const float*>(x);
        if (sh.sl == 2)
            d == 1 ? launch_split_dma_rpw<1, 2>(sh.rpw, w, xf, y, resid, ni, units, sh.upw, rb, st)
                   : launch_split_dma_rpw<2, 2>(sh.rpw, w, xf, y, resid, ni, units, sh.upw, rb, st);
        else if (sh.sl == 4)
            d == 1 ? launch_split_dma_rpw<1, 4>(sh.rpw, w, xf, y, resid, ni, units, sh.upw, rb, st)
                   : launch_split_dma_rpw<2, 4>(sh.rpw, w, xf, y, resid, ni, units, sh.upw, rb, st);
        else
            d == 1 ? launch_split_dma_rpw<1, 8>(sh.rpw, w, xf, y, resid, ni, units, sh.upw, rb, st)
                   : launch_split_dma_rpw<2, 8>(sh.rpw, w, xf, y, resid, ni, units, sh.upw, rb, st);
        return check_launch("vb_gemv");
    }
    if (sh.sl == 2)
        launch_split_d<2>(d, sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
    else if (sh.sl == 4)
        launch_split_d<4>(d, sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
    else
        launch_split_d<8>(d, sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
    return check_launch("vb_gemv");
}

// Split-row shape for Q6_K / Q8_0: split_shape's, with Q6_K slices a multiple
// of 8 units (4-byte-aligned slice starts).
SplitShape split_shape_t(int32_t type, int64_t n, int units) {
    SplitShape s = split_shape(n, units);
    if (type == TYPE_Q6_K) {
        s.upw = ((units + s.sl - 1) / s.sl + 7) & ~7;
        if (s.upw > 56 || units - (s.sl - 1) * s.upw < 4) s.rpw = 0;
    }
    return s;
}

int gemv_split_rpw(int32_t type, int64_t n, int64_t k) {
    // Q6_K rows of a whole number of dwords (k % 512 == 0: an even super-block count)
    if (!((type == TYPE_Q6_K && k % 512 == 0) || (type == TYPE_Q8_0 && k % 256 == 0))) return 0;
    const int units = static_cast<int>(k / 64);
    return units > UNITS_MAX && units <= SPLIT_US && n <= INT32_MAX ? split_shape_t(type, n, units).rpw : 0;
}

// Plain or residual-epilogue Q6_K / Q8_0 GEMV, 4096 < k <= 16384, on the
// split-row kernel; arguments validated by gemv_dispatch_fused.
int gemv_split(int32_t type, const void* w, const void* x, float* y, const float* resid, int64_t n, int64_t k,
               hipStream_t st, bool x_half) {
    const int units = static_cast<int>(k / 64);
    const SplitShape sh = split_shape_t(type, n, units);
    if (gemv_split_rpw(type, n, k) == 0 || sh.rpw == 0) {
        set_error("vb_gemv: internal: split-row kernel shape (type %d, n=%lld, k=%lld)", type,
                  static_cast<long long>(n), static_cast<long long>(k));
        return E_INVAL;
    }
    const uint32_t rb = static_cast<uint32_t>(row_bytes(type, k));
    const int ni = static_cast<int>(n);
    // rows in flight (VB_GEMV_SPLIT): Q6_K 1, Q8_0 2 by default (on MI355X at
    // 4096 x 14336: Q6_K 10.7 us against 10.8 at 2 and 12.2 at 3; Q8_0 11.4
    // against 11.8 at 1); at most 3, 4 would spill registers at 8 rows per wave
    int d = knobs().gemv_split_d > 3 ? 3 : knobs().gemv_split_d;
    if (d == 0) d = type == TYPE_Q6_K ? 1 : 2;
    auto go = [&](auto type_c) {
        constexpr int TY = decltype(type_c)::value;
        if (x_half) {
            // fp16 x (the one-row GEMM): the default rows in flight only
            constexpr int D0 = TY == TYPE_Q6_K ? 1 : 2;
            if (sh.sl == 2)
                launch_tsplit_rpw<TY, D0, 2, true>(sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
            else if (sh.sl == 4)
                launch_tsplit_rpw<TY, D0, 4, true>(sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
            else
                launch_tsplit_rpw<TY, D0, 8, true>(sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
            return;
        }
        if (sh.sl == 2)
            launch_tsplit_d<TY, 2>(d, sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
        else if (sh.sl == 4)
            launch_tsplit_d<TY, 4>(d, sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
        else
            launch_tsplit_d<TY, 8>(d, sh.rpw, w, x, y, resid, ni, units, sh.upw, rb, st);
    };
    if (type == TYPE_Q6_K)
        go(std::integral_constant<int, TYPE_Q6_K>{});
    else
        go(std::integral_constant<int, TYPE_Q8_0>{});
    return check_launch(x_half ? "vb_gemm" : "vb_gemv");
}

// Neurons per wave of the pairs kernel: one 8-wave workgroup per CU when that
// covers n neurons at up to 8 per wave, else 0 (the caller takes the general
// kernel).
int gemv_q4k_pairs_npw(int64_t n) {
    const int64_t groups = static_cast<int64_t>(num_cus()) * 8;
    const int64_t npw = (n + groups - 1) / groups;
    return npw <= 8 ? static_cast<int>(npw < 1 ? 1 : npw) : 0;
}

// FFN block launch 1 for Q4_K gate/up with k <= 4096 (k % 256 == 0): y[p] =
// act(gate_p . n, up_p . n), p < n neurons; with `active`, the gathered
// form (y is the hidden vector of i_dim entries, above).  Arguments
// validated by the callers.
int gemv_q4k_pairs(const void* wg, const void* wu, const float* x, const float* norm_w, float eps, int kind,
                   float* y, int64_t n, int64_t k, hipStream_t st, const int32_t* active, const int32_t* n_dev,
                   int64_t i_dim) {
    const int npw = gemv_q4k_pairs_npw(n);
    const int units = static_cast<int>(k / 64);
    if (npw == 0 || units > UNITS_MAX || k % 256 != 0 || n > INT32_MAX || i_dim > INT32_MAX ||
        (active && i_dim * row_bytes(TYPE_Q4_K, k) >= (int64_t(1) << 32))) {
        set_error("vb_gemv: internal: Q4_K pairs kernel shape (n=%lld, k=%lld)", static_cast<long long>(n),
                  static_cast<long long>(k));
        return E_INVAL;
    }
    PairsArgs a{wg, wu, x, norm_w, eps, kind, y, static_cast<int>(n), units,
                static_cast<uint32_t>(row_bytes(TYPE_Q4_K, k)), active, n_dev, static_cast<int>(i_dim)};
    const int ring = knobs().gemv_ring;  // neurons in flight while computing (default 2)
    if (ring == 1)
        launch_pairs_npw<2>(npw, a, st);
    else if (ring >= 3)
        launch_pairs_npw<4>(npw, a, st);
    else
        launch_pairs_npw<3>(npw, a, st);
    return check_launch("vb_gemv");
}

}  // namespace vb
