// Q4_K GEMV (M = 1) on the int8 matrix cores: y[n] = sum_k W[n, k] x[k].
//
// Replaces gemv_dequant (cpp/src/dequant.cpp:739-780) for Q4_K weights (GGUF
// layout, cpp/src/dequant.cpp:258-301).  Same arithmetic as the v_dot4 path
// in gemv.hip -- activations as 16-bit fixed point split into two signed
// bytes, exact integer sums per 32-element sub-block, scales applied in
// fp32 -- but the integer sums come from v_mfma_i32_16x16x64_i8 instead of
// v_dot4_i32_i8, which cuts the VALU work per weight by about 2.5x (the M=1
// GEMV on gfx950 is VALU-bound with v_dot4: one wave-instruction retires 64
// lanes x 4 weights, the MFMA 16 x 16 x 64).
//
// MFMA mapping (16x16x64, lane l: row/col l % 16, k-block l / 16 of 16
// bytes; D: column l % 16, rows 4 * (l / 16) + 0..3):
//   B (64 x 16) = weights: column j = weight row j of a 16-row group; k-block
//     g = 8 qs bytes of chunk g (elements 64g..64g+63 of the super-block)
//     as 16 int8: the 8 low nibbles q (sub-block 2g) and the 8 high nibbles
//     as 16 * (q - 8) (sub-block 2g+1): one and / one and-xor (v_bitop3) per
//     4 bytes, no shifts; the offset and the factor 16 are folded into the
//     activation scales.  Four steps s = 0..3 walk the 32 qs bytes.
//   A (16 x 64) = activations: row 4g + v is nonzero only in k-block g and
//     holds variant v of the matching 16 activations: v = 0 / 1: high / low
//     byte of the sub-block 2g elements (zeros against the high nibbles),
//     v = 2 / 3: high / low byte of the sub-block 2g+1 elements.
//   D[4g + v][j] after the four steps = sum over the chunk of variant v x
//     weights: lane (g, j) holds exactly the four integer sums of (row j,
//     chunk g) and applies that row's sub-block scales -- every lane does
//     useful epilogue work.
//
// Geometry: a wave owns one group of 16 rows and a k-slice of nsbw
// super-blocks ("ks" waves per row group); its super-blocks stream through a
// ring of D register buffers.  Partial row sums meet in LDS and the
// workgroup adds the k-slices in a fixed order.
#include <cstdlib>
#include <type_traits>

#include "vb_common.hpp"
#include "vb_internal.hpp"

namespace vb {
namespace {

typedef int int4v __attribute__((ext_vector_type(4)));

constexpr int X16_MAX = 32512;  // 127 * 256: keeps the high byte a signed byte
constexpr int kMaxSB = 128;     // k <= 32768

// LDS layout (uint4 units), nsb = super-blocks per row:
//   xa[(sb * 4 + s) * 16 + 4g + v]  A operand of lane (g, 4g + v), step s
//   xa[nsb * 64 + 16 s]             zeros: A operand of the other lanes (the
//                                   same 256-byte step stride)
//   xs[(sb * 4 + g) * 2 + 0..1]     chunk 4sb+g: (s_A, s_B / 16, 8 s_B isum_B,
//                                   sum_A), (sum_B, 0, 0, 0)
//   red[ks][rows_wg]                partial row sums (floats)
// s = activation scale of a sub-block, sum = sum of its activations, isum =
// sum of its 16-bit codes.
__host__ __device__ constexpr int lds_zero_offset(int nsb) { return nsb * 64; }
__host__ __device__ constexpr int lds_xs_offset(int nsb) { return nsb * 64 + 64; }
__host__ __device__ constexpr int lds_red_offset(int nsb) { return nsb * 64 + 64 + nsb * 8; }

// Encode task t (8 activations): chunk c = t / 8, run r = (t / 4) & 1,
// step s = t & 3 -> x[64c + 32r + 8s, +8).  The four tasks of a run are
// adjacent lanes and combine max / sum with DPP quad shuffles.
__device__ __forceinline__ void load_task(const float* __restrict__ x, int ntasks, int t, float* v) {
    t = t < ntasks ? t : ntasks - 1;
    const float* p = x + static_cast<int64_t>(t) * 8;
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <int CTRL>
__device__ __forceinline__ float qdpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int qdpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ void encode_task(int t, const float* v, uint4* xa, float* xsf) {
    const int c = t >> 3, r = (t >> 2) & 1, s = t & 3;
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    // the 4 tasks of a run are lanes 4m..4m+3 of a quad
    amax = fmaxf(amax, qdpp<0xB1>(amax));  // quad_perm [1,0,3,2]
    amax = fmaxf(amax, qdpp<0x4E>(amax));  // quad_perm [2,3,0,1]
    sum += qdpp<0xB1>(sum);
    sum += qdpp<0x4E>(sum);
    const float inv = amax > 0.f ? static_cast<float>(X16_MAX) / amax : 0.f;
    uint32_t ph[2] = {0, 0}, pl[2] = {0, 0};
    int isum = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int q = static_cast<int>(rintf(v[i] * inv));
        q = q > X16_MAX ? X16_MAX : (q < -X16_MAX ? -X16_MAX : q);
        isum += q;
        const int lo = ((q + 128) & 255) - 128;
        const int hi = (q - lo) >> 8;
        ph[i >> 2] |= static_cast<uint32_t>(hi & 255) << (8 * (i & 3));
        pl[i >> 2] |= static_cast<uint32_t>(lo & 255) << (8 * (i & 3));
    }
    isum += qdpp_i<0xB1>(isum);
    isum += qdpp_i<0x4E>(isum);
    const int sb = c >> 2, cg = c & 3;
    uint4* slot = xa + (sb * 4 + s) * 16 + cg * 4 + 2 * r;
    slot[0] = r == 0 ? make_uint4(ph[0], ph[1], 0u, 0u) : make_uint4(0u, 0u, ph[0], ph[1]);
    slot[1] = r == 0 ? make_uint4(pl[0], pl[1], 0u, 0u) : make_uint4(0u, 0u, pl[0], pl[1]);
    if (s == 0) {
        const float sx = amax / static_cast<float>(X16_MAX);
        float* f = xsf + c * 8;
        if (r == 0) {
            f[0] = sx;
            f[3] = sum;
        } else {
            // high nibbles enter the MFMA as 16 * (q - 8):
            //   sum x16 * q = (sum x16 * 16 (q - 8)) / 16 + 8 * isum
            f[1] = sx * 0.0625f;
            f[2] = 8.0f * sx * static_cast<float>(isum);
            f[4] = sum;
            f[5] = 0.f;
            f[6] = 0.f;
            f[7] = 0.f;
        }
    }
}

struct SBUnit {
    uint4 hd, q0, q1;  // header, qs[32g, 32g+16), qs[32g+16, 32g+32)
};

constexpr int ROWS_PLAIN = 0;
constexpr int ROWS_PAIRS = 1;

template <int MODE>
__device__ __forceinline__ const uint8_t* row_ptr(const uint8_t* w, const uint8_t* w2,
                                                  const int32_t* gidx, int nsrc, int row, int64_t rb) {
    if constexpr (MODE == ROWS_PLAIN) {
        return w + static_cast<int64_t>(row) * rb;
    } else {
        int src = gidx[row >> 1];
        src = src < 0 ? 0 : (src >= nsrc ? nsrc - 1 : src);  // never read outside the tensor
        return ((row & 1) ? w2 : w) + static_cast<int64_t>(src) * rb;
    }
}

// Per-lane selectors of the 6-bit scale / min of sub-blocks 2g, 2g+1
// (get_scale_min_k4, cpp/src/dequant.cpp:258-266), with sh = 16 (g & 1):
//   g < 2:  sc = (s03 >> sh) & 0x3F3F,  m = (s47 >> sh) & 0x3F3F
//   g >= 2: sc = ((s8b >> sh) & 0x0F0F) | ((s03 >> (sh + 2)) & 0x3030)
//           m  = ((s8b >> (sh + 4)) & 0x0F0F) | ((s47 >> (sh + 2)) & 0x3030)
// (s03, s47, s8b = scales[0:4], [4:8], [8:12] as little-endian words), i.e.
//   sc = ((hi ? s8b : s03) >> sh) & m1 | (s03 >> (sh + 2)) & m2, and the same
// for m with s47 and shift sh (g < 2) or sh + 4.
struct ScaleSel {
    uint32_t sh, sh2, shm, m1, m2;
    bool hi;
};

__device__ __forceinline__ ScaleSel scale_sel(int g) {
    ScaleSel q;
    q.hi = g >= 2;
    q.sh = 16u * static_cast<uint32_t>(g & 1);
    q.sh2 = q.sh + 2u;
    q.shm = q.hi ? q.sh + 4u : q.sh;
    q.m1 = q.hi ? 0x0F0Fu : 0x3F3Fu;
    q.m2 = q.hi ? 0x3030u : 0u;
    return q;
}

// One row group x one super-block, lane (g = lane / 16, j = lane % 16).
// a_off: LDS byte offset of this lane's step-0 A operand (steps 256 B apart).
// f0 = (s_A, s_B / 16, 8 s_B isum_B, sum_A), sumB: the chunk's activation data.
__device__ __forceinline__ float sb_dot(const SBUnit& v, const uint8_t* xa_bytes, uint32_t a_off, float4 f0,
                                        float sumB, const ScaleSel& q) {
    const uint32_t qd[8] = {v.q0.x, v.q0.y, v.q0.z, v.q0.w, v.q1.x, v.q1.y, v.q1.z, v.q1.w};
    int4v acc = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const uint32_t a0 = qd[2 * s], a1 = qd[2 * s + 1];
        int4v b;
        b.x = static_cast<int>(a0 & 0x0F0F0F0Fu);
        b.y = static_cast<int>(a1 & 0x0F0F0F0Fu);
        b.z = static_cast<int>((a0 ^ 0x80808080u) & 0xF0F0F0F0u);  // 16 * (q - 8) as int8
        b.w = static_cast<int>((a1 ^ 0x80808080u) & 0xF0F0F0F0u);
        const uint4 av = *reinterpret_cast<const uint4*>(xa_bytes + a_off + 256 * s);
        const int4v a = {static_cast<int>(av.x), static_cast<int>(av.y), static_cast<int>(av.z),
                         static_cast<int>(av.w)};
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
    }
    const int SA = acc.x * 256 + acc.y;  // sum x16 q over sub-block 2g: |SA| < 2^24
    const int SB = acc.z * 256 + acc.w;  // sum x16 16 (q - 8) over sub-block 2g+1
    const uint32_t s03 = v.hd.y, s47 = v.hd.z, s8b = v.hd.w;
    const uint32_t SC = (((q.hi ? s8b : s03) >> q.sh) & q.m1) | ((s03 >> q.sh2) & q.m2);
    const uint32_t M = (((q.hi ? s8b : s47) >> q.shm) & q.m1) | ((s47 >> q.sh2) & q.m2);
    const float d = f16lo(v.hd.x), dmin = f16hi(v.hd.x);
    const float sc0 = static_cast<float>(SC & 0xFFu), sc1 = static_cast<float>((SC >> 8) & 0xFFu);
    const float m0 = static_cast<float>(M & 0xFFu), m1 = static_cast<float>((M >> 8) & 0xFFu);
    const float tA = f0.x * static_cast<float>(SA);
    const float tB = fmaf(f0.y, static_cast<float>(SB), f0.z);
    const float dot = fmaf(sc0, tA, sc1 * tB);
    const float mins = fmaf(m0, f0.w, m1 * sumB);
    return fmaf(d, dot, -dmin * mins);
}

// xt: encode tasks held in registers per thread (k <= 4096 * xt_regs with
// 512 threads); larger k loops.
constexpr int XT = 2;

// Weight staging.  The MFMA layout makes each lane group of a wave read 16
// different rows; loaded that way straight from HBM (16 rows per load
// instruction) the reads run at about two thirds of the row-contiguous
// pattern's rate.  So a wave loads its 16 rows x 4 super-blocks per step as
// row-contiguous 16-byte pieces (576 pieces, 9 per lane), stores them into a
// private LDS area (rows 592 bytes apart: the 16-lane column reads below are
// bank-conflict free) and reads the MFMA layout back from there.
constexpr int SB_STEP = 4;                          // super-blocks per step
constexpr int STAGE_ROW = SB_STEP * 144 + 16;       // bytes per staged row
constexpr int STAGE_BYTES = 16 * STAGE_ROW;         // per wave
constexpr int PIECES_PER_ROW = SB_STEP * 144 / 16;  // 36
constexpr int PPL = 16 * PIECES_PER_ROW / 64;       // pieces per lane: 9

__host__ __device__ constexpr size_t lds_stage_offset(int nsb, int ks, int rows_wg) {
    return ((static_cast<size_t>(lds_red_offset(nsb)) * 16 + static_cast<size_t>(ks) * rows_wg * 4) + 15) & ~size_t(15);
}

template <int D>
constexpr int mfma_max_threads() { return D <= 2 ? 512 : 256; }

template <int MODE, int D>
__global__ void __launch_bounds__(mfma_max_threads<D>()) gemv_q4k_mfma_kernel(
        const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, const int32_t* __restrict__ gidx,
        int nsrc, const float* __restrict__ x, float* __restrict__ y, int n, int64_t rb, int nsb, int nsbw,
        int ks, int* __restrict__ zbuf, int zn) {
    if (zn > 0 && blockIdx.x == 0) {
        for (int i = threadIdx.x; i < zn; i += blockDim.x) zbuf[i] = 0;
    }
    extern __shared__ uint4 lds[];
    uint4* xa = lds;
    float* xsf = reinterpret_cast<float*>(lds + lds_xs_offset(nsb));
    float* red = reinterpret_cast<float*>(lds + lds_red_offset(nsb));

    const int lane = threadIdx.x & 63;
    const int j = lane & 15, g = lane >> 4;
    // wave-uniform values (readfirstlane: integer division runs on the VALU)
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int rgs = __builtin_amdgcn_readfirstlane(static_cast<int>(blockDim.x >> 6) / ks);
    const int rgi = __builtin_amdgcn_readfirstlane(wave / ks);
    const int kw = wave - rgi * ks;
    const int rows_wg = rgs * 16;
    const int wg_row0 = static_cast<int>(blockIdx.x) * rows_wg;
    const int sb0 = kw * nsbw;
    int nsbk = nsb - sb0;  // super-blocks of this k-slice (the host avoids empty slices)
    nsbk = nsbk < nsbw ? nsbk : nsbw;
    nsbk = nsbk > 0 ? nsbk : 1;
    const int nsteps = (nsbk + SB_STEP - 1) / SB_STEP;
    const int nsteps_p = ((nsteps + D - 1) / D) * D;
    uint8_t* stage = reinterpret_cast<uint8_t*>(lds) + lds_stage_offset(nsb, ks, rows_wg) +
                     static_cast<size_t>(wave) * STAGE_BYTES;

    // pieces of this lane: p = 64 i + lane -> staged row p / 36, piece p % 36
    // (super-block (p % 36) / 9 of the step, 16-byte word (p % 36) % 9)
    const uint8_t* prow[PPL];
    int psb[PPL], pword[PPL], poff[PPL];
#pragma unroll
    for (int i = 0; i < PPL; i++) {
        const int p = 64 * i + lane, r = p / PIECES_PER_ROW, q = p - r * PIECES_PER_ROW;
        int row = wg_row0 + rgi * 16 + r;
        row = row < n ? row : n - 1;
        prow[i] = row_ptr<MODE>(w, w2, gidx, nsrc, row, rb);
        psb[i] = q / 9;
        pword[i] = 16 * (q - 9 * (q / 9));
        poff[i] = r * STAGE_ROW + 144 * psb[i] + pword[i];
    }
    // native vector type (HIP's uint4 struct copies become memcpys that keep
    // the array in scratch)
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 pv[D][PPL];
    int it = 0;
    // slots are compile-time constants (std::integral_constant) so pv stays
    // in registers
    auto issue = [&](auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value;
        const int t = it < nsteps ? it : nsteps - 1;
        const int last = sb0 + nsbk - 1;
#pragma unroll
        for (int i = 0; i < PPL; i++) {
            int sb = sb0 + SB_STEP * t + psb[i];
            sb = sb < last ? sb : last;
            pv[slot][i] = *reinterpret_cast<const u32x4*>(prow[i] + static_cast<int64_t>(sb) * 144 + pword[i]);
        }
        ++it;
    };

    // x first, then the first D steps of weights, then the encode.
    const int ntasks = nsb * 32;
    const bool x_in_regs = ntasks <= XT * static_cast<int>(blockDim.x);
    float xv[XT][8];
    if (x_in_regs) {
#pragma unroll
        for (int i = 0; i < XT; i++) load_task(x, ntasks, threadIdx.x + i * blockDim.x, xv[i]);
    }
    __builtin_amdgcn_sched_barrier(0);
    issue(std::integral_constant<int, 0>{});
    issue(std::integral_constant<int, 1>{});
    if constexpr (D == 4) {
        issue(std::integral_constant<int, 2>{});
        issue(std::integral_constant<int, 3>{});
    }
    __builtin_amdgcn_sched_barrier(0);
    // ntasks and blockDim are multiples of 32: every quad of tasks is complete.
    if (x_in_regs) {
#pragma unroll
        for (int i = 0; i < XT; i++) {
            const int t = threadIdx.x + i * blockDim.x;
            if (t < ntasks) encode_task(t, xv[i], xa, xsf);
        }
    } else {
        for (int t = threadIdx.x; t < ntasks; t += blockDim.x) {
            float tv[8];
            load_task(x, ntasks, t, tv);
            encode_task(t, tv, xa, xsf);
        }
    }
    if (threadIdx.x < 64) xa[lds_zero_offset(nsb) + threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();

    // A operand: lane (g, 4g + v) reads its variant, the others the zeros
    // (same 256-byte step stride).
    const bool a_live = (j >> 2) == g;
    const uint32_t a_lane = a_live ? 16u * j : 16u * lds_zero_offset(nsb);
    const uint32_t a_sbmask = a_live ? 0xFFFFFFFFu : 0u;
    const uint8_t* xa_bytes = reinterpret_cast<const uint8_t*>(xa);
    const ScaleSel q = scale_sel(g);
    const uint8_t* my = stage + j * STAGE_ROW;  // this lane's staged row
    float out = 0.f;

    int ct = 0;
    auto compute = [&](auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value;
        if (ct >= nsteps) return;  // padding step (uniform)
#pragma unroll
        for (int i = 0; i < PPL; i++) *reinterpret_cast<u32x4*>(stage + poff[i]) = pv[slot][i];
        const int nsb_here = nsbk - SB_STEP * ct < SB_STEP ? nsbk - SB_STEP * ct : SB_STEP;
#pragma unroll
        for (int t = 0; t < SB_STEP; t++) {
            if (t < nsb_here) {  // uniform
                const int sb = sb0 + SB_STEP * ct + t;
                SBUnit v;
                v.hd = *reinterpret_cast<const uint4*>(my + 144 * t);
                v.q0 = *reinterpret_cast<const uint4*>(my + 144 * t + 16 + 32 * g);
                v.q1 = *reinterpret_cast<const uint4*>(my + 144 * t + 32 + 32 * g);
                const uint32_t a_off = a_lane + ((static_cast<uint32_t>(sb) * 1024u) & a_sbmask);
                const float* f = xsf + (sb * 4 + g) * 8;
                const float4 f0 = *reinterpret_cast<const float4*>(f);
                out += sb_dot(v, xa_bytes, a_off, f0, f[4], q);
            }
        }
        ++ct;
    };

    // ring slots are literal constants (register arrays, no scratch)
    for (int s = 0; s + D < nsteps_p; s += D) {
        compute(std::integral_constant<int, 0>{});
        issue(std::integral_constant<int, 0>{});
        compute(std::integral_constant<int, 1>{});
        issue(std::integral_constant<int, 1>{});
        if constexpr (D == 4) {
            compute(std::integral_constant<int, 2>{});
            issue(std::integral_constant<int, 2>{});
            compute(std::integral_constant<int, 3>{});
            issue(std::integral_constant<int, 3>{});
        }
    }
    compute(std::integral_constant<int, 0>{});
    compute(std::integral_constant<int, 1>{});
    if constexpr (D == 4) {
        compute(std::integral_constant<int, 2>{});
        compute(std::integral_constant<int, 3>{});
    }

    // add the 4 chunk lanes of each row, then the k-slices (fixed order)
    out += __shfl_xor(out, 16, 64);
    out += __shfl_xor(out, 32, 64);
    if (lane < 16) red[kw * rows_wg + rgi * 16 + j] = out;
    __syncthreads();
    for (int i = threadIdx.x; i < rows_wg; i += blockDim.x) {
        float t = 0.f;
        for (int k = 0; k < ks; k++) t += red[k * rows_wg + i];
        if (wg_row0 + i < n) y[wg_row0 + i] = t;
    }
}

struct MfmaShape {
    int nsb, nsbw, ks, wpg, depth;
    int64_t grid;
    size_t lds;
};


size_t mfma_lds(int nsb, int ks, int wpg) {
    const int rows_wg = (wpg / ks) * 16;
    return lds_stage_offset(nsb, ks, rows_wg) + static_cast<size_t>(wpg) * STAGE_BYTES;
}

// Launch geometry: k-slices of nsbw super-blocks (a multiple of the 4 of a
// step), ks waves per 16-row group, wpg / ks row groups per workgroup.  The
// staging areas make LDS the occupancy limit.  Preferred: every workgroup
// resident at once, then more waves per CU, then fewer steps per wave.
// VB_GEMV_MFMA_CFG="wpg,ks" overrides (tuning sweeps).
MfmaShape mfma_shape(int64_t n, int nsb) {
    MfmaShape best{};
    int64_t best_key[3] = {0, 0, 0};
    bool have = false;
    const int64_t nrg = (n + 15) / 16;
    const int64_t cus = num_cus();
    auto consider = [&](int ks, int wpg) -> MfmaShape {
        const int nsbw = ((nsb + ks - 1) / ks + SB_STEP - 1) / SB_STEP * SB_STEP;
        const int steps = nsbw / SB_STEP;
        const int depth = steps <= 2 ? 2 : 4;
        const int64_t rows_wg = static_cast<int64_t>(wpg / ks) * 16;
        const size_t lds = mfma_lds(nsb, ks, wpg);
        return MfmaShape{nsb, nsbw, ks, wpg, depth, (nrg * 16 + rows_wg - 1) / rows_wg, lds};
    };
    for (int ks = 1; ks <= 8 && ks <= nsb; ks++) {
        for (int wpg = 8; wpg >= ks; wpg--) {
            if (wpg % ks) continue;
            const MfmaShape c = consider(ks, wpg);
            if ((ks - 1) * c.nsbw >= nsb) continue;  // an empty k-slice
            if (c.lds > 160 * 1024) continue;
            if (64 * wpg > (c.depth <= 2 ? 512 : 256)) continue;
            const int64_t per_lds = static_cast<int64_t>(160 * 1024 / c.lds);
            const int64_t per_waves = 8 / wpg;
            const int64_t res = per_lds < per_waves ? per_lds : per_waves;
            if (res < 1) continue;
            const int64_t rounds = (c.grid + cus * res - 1) / (cus * res);
            const int64_t wgs_cu = (c.grid + cus - 1) / cus;
            const int64_t waves_cu = (wgs_cu < res ? wgs_cu : res) * wpg;
            const int64_t key[3] = {rounds, -waves_cu, static_cast<int64_t>(c.nsbw)};
            bool better = !have;
            for (int t = 0; t < 3 && !better; t++) {
                if (key[t] < best_key[t]) better = true;
                else if (key[t] > best_key[t]) break;
            }
            if (better) {
                have = true;
                best = c;
                for (int t = 0; t < 3; t++) best_key[t] = key[t];
            }
        }
    }
    if (knobs().gemv_mfma_wpg > 0) {
        const int a = knobs().gemv_mfma_wpg, b = knobs().gemv_mfma_ks;
        if (b <= nsb && a >= b && a % b == 0 && a <= 8) {
            const MfmaShape c = consider(b, a);
            if ((b - 1) * c.nsbw < nsb && c.lds <= 160 * 1024 && 64 * a <= (c.depth <= 2 ? 512 : 256)) best = c;
        }
    }
    return best;
}

template <int MODE, int D>
void launch(const MfmaShape& s, const uint8_t* w, const uint8_t* w2, const int32_t* gidx, int nsrc,
            const float* x, float* y, int n, int64_t rb, int* zbuf, int zn, hipStream_t st) {
    gemv_q4k_mfma_kernel<MODE, D><<<dim3(static_cast<uint32_t>(s.grid)), dim3(64 * s.wpg), s.lds, st>>>(
        w, w2, gidx, nsrc, x, y, n, rb, s.nsb, s.nsbw, s.ks, zbuf, zn);
}

}  // namespace

// Caller (gemv_dispatch_src) has validated type, shapes and alignment
// (x 16-byte aligned, W 16-byte aligned, k % 256 == 0, n < 2^31).
int gemv_q4k_mfma(const void* w, const RowSrc& src, const float* x, float* y, int64_t n, int64_t k,
                  hipStream_t st) {
    const int nsb = static_cast<int>(k / 256);
    if (nsb > kMaxSB) {
        set_error("vb_gemv: k=%lld exceeds the supported maximum of %d for Q4_K", static_cast<long long>(k),
                  kMaxSB * 256);
        return E_UNSUPPORTED;
    }
    const MfmaShape s = mfma_shape(n, nsb);
    if (s.grid <= 0 || s.wpg == 0) {
        set_error("vb_gemv: no launch shape for n=%lld k=%lld", static_cast<long long>(n), static_cast<long long>(k));
        return E_UNSUPPORTED;
    }
    const int64_t rb = (k / 256) * 144;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const uint8_t* w2 = static_cast<const uint8_t*>(src.w2);
    const int ni = static_cast<int>(n), nsrc = static_cast<int>(src.nsrc);
    const bool pairs = src.gidx != nullptr;
#define VB_LAUNCH(D)                                                                                       \
    (pairs ? launch<ROWS_PAIRS, D>(s, wb, w2, src.gidx, nsrc, x, y, ni, rb, src.zbuf, src.zn, st)           \
           : launch<ROWS_PLAIN, D>(s, wb, w2, src.gidx, nsrc, x, y, ni, rb, src.zbuf, src.zn, st))
    switch (s.depth) {
    case 2: VB_LAUNCH(2); break;
    default: VB_LAUNCH(4); break;
    }
#undef VB_LAUNCH
    return check_launch("vb_gemv");
}

}  // namespace vb
