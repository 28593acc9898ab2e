// Dequant-fused GEMV, M = 1:  y[n] = sum_k W[n, k] x[k]  (GGUF layout).
//
// Replaces gemv_dequant (cpp/src/dequant.cpp:739-780), which decodes every
// weight to an fp32 scratch row and does a saxpy per row.  Here no weight is
// ever materialised: each lane owns a 64-element "unit" of a row and streams
// the packed bytes of that unit straight into integer dot products.
//
// Activation encoding.  Each lane loads the 64 fp32 activations of its unit
// once, splits them into runs (32 elements for Q4_K / Q8_0, 16 for Q6_K: the
// weight sub-block size) and encodes every run as 16-bit fixed point with a
// per-run fp32 scale:  x ~= s * x16,  |x16| <= 32512,  x16 = 256*xh + xl with
// xh, xl signed bytes.  A run's dot product with the integer weight codes q
// is then  s * (256 * sdot4(q, xh) + sdot4(q, xl))  -- exact integer
// arithmetic on v_dot4_i32_i8, about one VALU op per weight element.  The
// encoding error is |x - s*x16| <= s/2 = amax/65024 per element, which puts
// the GEMV rel-L2 error near 1e-5 (the fp32 bound is 1e-3).
//
// Unit -> bytes (row of k elements, units_per_row = k/64):
//   Q4_K  unit u: super-block u/4, chunk c = u%4: header (16 B: d, dmin,
//         scales) + qs[32c, 32c+32).  Low nibbles = run 0 = sub-block 2c,
//         high nibbles = run 1 = sub-block 2c+1 (cpp/src/dequant.cpp:278-299).
//   Q8_0  unit u: blocks 2u, 2u+1 = 68 bytes at 68u (4-byte aligned).
//   Q6_K  unit u: super-block u/4, c = u%4, h = c/2, l0 = 16*(c%2): the four
//         16-element runs t = 0..3 at elements 128h + 32t + l0 + [0, 16).
//         Bytes: ql[64h + l0 + [0,16)], ql[64h + 32 + l0 + [0,16)],
//         qh[32h + l0 + [0,16)], scales[8h + c%2 + 2t], d.
//
// Launch shape.  A wave covers 64 consecutive units of a row ("k-tile").
// Rows with more than one k-tile are split over `wpr` waves of the same
// workgroup (partial sums meet in LDS); a workgroup of `wpg` waves holds
// wpg/wpr row groups, each streaming R rows at a time so that every lane has
// R * (row bytes per unit) in flight before it computes.
#include <cstdlib>

#include "vb_common.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int X16_MAX = 32512;  // 127 * 256: keeps xh within a signed byte

struct XSlice {
    uint32_t h[16];  // high bytes of x16, 4 per dword, element order
    uint32_t l[16];  // low bytes (signed), same order
    float s[4];      // per-run scale
    float sum[4];    // per-run sum of the fp32 activations
    int isum[4];     // per-run sum of x16
};

// Encode 64 activations: 4 segments of 16 at x + seg*seg_stride.
template <int RUNLEN>
__device__ __forceinline__ void load_xslice(const float* __restrict__ x, int seg_stride, bool valid,
                                            XSlice& xs) {
    float v[64];
#pragma unroll
    for (int seg = 0; seg < 4; seg++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
            if (valid) f = *reinterpret_cast<const float4*>(x + seg * seg_stride + 4 * i);
            v[16 * seg + 4 * i + 0] = f.x;
            v[16 * seg + 4 * i + 1] = f.y;
            v[16 * seg + 4 * i + 2] = f.z;
            v[16 * seg + 4 * i + 3] = f.w;
        }
    }
    constexpr int NRUN = 64 / RUNLEN;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        xs.s[r] = 0.f;
        xs.sum[r] = 0.f;
        xs.isum[r] = 0;
    }
#pragma unroll
    for (int r = 0; r < NRUN; r++) {
        float amax = 0.f, sum = 0.f;
#pragma unroll
        for (int i = 0; i < RUNLEN; i++) {
            amax = fmaxf(amax, fabsf(v[r * RUNLEN + i]));
            sum += v[r * RUNLEN + i];
        }
        const float inv = amax > 0.f ? static_cast<float>(X16_MAX) / amax : 0.f;
        xs.s[r] = amax / static_cast<float>(X16_MAX);
        xs.sum[r] = sum;
        int isum = 0;
#pragma unroll
        for (int d = 0; d < RUNLEN / 4; d++) {
            uint32_t ph = 0, pl = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                int q = static_cast<int>(rintf(v[r * RUNLEN + 4 * d + b] * inv));
                q = q > X16_MAX ? X16_MAX : (q < -X16_MAX ? -X16_MAX : q);
                isum += q;
                const int lo = ((q + 128) & 255) - 128;
                const int hi = (q - lo) >> 8;
                ph |= static_cast<uint32_t>(hi & 255) << (8 * b);
                pl |= static_cast<uint32_t>(lo & 255) << (8 * b);
            }
            xs.h[r * (RUNLEN / 4) + d] = ph;
            xs.l[r * (RUNLEN / 4) + d] = pl;
        }
        xs.isum[r] = isum;
    }
}

// ---- per-type unit loaders and dot products -------------------------------

struct Q4KUnit { uint4 hd, qa, qb; };
struct Q8Unit { uint4 a, b, c, d; uint32_t e; };
struct Q6KUnit { uint4 la, lb, qh; uint32_t sc; uint32_t d; };

template <int TYPE> struct UnitOf;
template <> struct UnitOf<TYPE_Q4_K> { using T = Q4KUnit; };
template <> struct UnitOf<TYPE_Q8_0> { using T = Q8Unit; };
template <> struct UnitOf<TYPE_Q6_K> { using T = Q6KUnit; };

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, Q4KUnit& v) {
    const uint8_t* b = row + (u >> 2) * 144;
    const int c = u & 3;
    v.hd = *reinterpret_cast<const uint4*>(b);
    v.qa = *reinterpret_cast<const uint4*>(b + 16 + 32 * c);
    v.qb = *reinterpret_cast<const uint4*>(b + 32 + 32 * c);
}

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, Q8Unit& v) {
    const uint8_t* b = row + u * 68;
    v.a = ld_b128_a4(b);
    v.b = ld_b128_a4(b + 16);
    v.c = ld_b128_a4(b + 32);
    v.d = ld_b128_a4(b + 48);
    v.e = ld_b32(b + 64);
}

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, Q6KUnit& v) {
    const uint8_t* b = row + (u >> 2) * 210;
    const int c = u & 3, h = c >> 1, l0 = 16 * (c & 1);
    v.la = ld_b128_a2(b + 64 * h + l0);
    v.lb = ld_b128_a2(b + 64 * h + 32 + l0);
    v.qh = ld_b128_a2(b + 128 + 32 * h + l0);
    const uint8_t* s = b + 192 + 8 * h + (c & 1);
    v.sc = static_cast<uint32_t>(s[0]) | (static_cast<uint32_t>(s[2]) << 8) |
           (static_cast<uint32_t>(s[4]) << 16) | (static_cast<uint32_t>(s[6]) << 24);
    v.d = *reinterpret_cast<const uint16_t*>(b + 208);
}

__device__ __forceinline__ int run_dot(const uint32_t* q, const uint32_t* xh, const uint32_t* xl, int n) {
    int ah = 0, al = 0;
#pragma unroll
    for (int i = 0; i < n; i++) {
        ah = sdot4(q[i], xh[i], ah);
        al = sdot4(q[i], xl[i], al);
    }
    return ah * 256 + al;
}

__device__ __forceinline__ float unit_dot(const Q4KUnit& v, const XSlice& xs, int u) {
    const int c = u & 3;
    const uint32_t qd[8] = {v.qa.x, v.qa.y, v.qa.z, v.qa.w, v.qb.x, v.qb.y, v.qb.z, v.qb.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = qd[i] & 0x0F0F0F0Fu;
        hi[i] = (qd[i] >> 4) & 0x0F0F0F0Fu;
    }
    const int s0 = run_dot(lo, xs.h, xs.l, 8);
    const int s1 = run_dot(hi, xs.h + 8, xs.l + 8, 8);
    // 6-bit scales/mins of sub-blocks 2c and 2c+1, two bytes at a time.
    const uint32_t sh = 16u * static_cast<uint32_t>(c & 1);
    const uint32_t A = v.hd.y >> sh, B = v.hd.z >> sh, C = v.hd.w >> sh;
    uint32_t SC, M;
    if (c < 2) {
        SC = A & 0x3F3Fu;
        M = B & 0x3F3Fu;
    } else {
        SC = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u);
        M = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u);
    }
    const float d = f16lo(v.hd.x), dmin = f16hi(v.hd.x);
    const float sc0 = static_cast<float>(SC & 0xFFu), sc1 = static_cast<float>((SC >> 8) & 0xFFu);
    const float m0 = static_cast<float>(M & 0xFFu), m1 = static_cast<float>((M >> 8) & 0xFFu);
    const float dot = sc0 * (xs.s[0] * static_cast<float>(s0)) + sc1 * (xs.s[1] * static_cast<float>(s1));
    const float mins = m0 * xs.sum[0] + m1 * xs.sum[1];
    return d * dot - dmin * mins;
}

__device__ __forceinline__ float unit_dot(const Q8Unit& v, const XSlice& xs, int) {
    const uint32_t w[17] = {v.a.x, v.a.y, v.a.z, v.a.w, v.b.x, v.b.y, v.b.z, v.b.w,
                            v.c.x, v.c.y, v.c.z, v.c.w, v.d.x, v.d.y, v.d.z, v.d.w, v.e};
    uint32_t q0[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q0[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
    const int s0 = run_dot(q0, xs.h, xs.l, 8);
    const int s1 = run_dot(w + 9, xs.h + 8, xs.l + 8, 8);
    const float d0 = f16lo(w[0]), d1 = f16hi(w[8]);
    return d0 * (xs.s[0] * static_cast<float>(s0)) + d1 * (xs.s[1] * static_cast<float>(s1));
}

__device__ __forceinline__ float unit_dot(const Q6KUnit& v, const XSlice& xs, int) {
    const uint32_t la[4] = {v.la.x, v.la.y, v.la.z, v.la.w};
    const uint32_t lb[4] = {v.lb.x, v.lb.y, v.lb.z, v.lb.w};
    const uint32_t qh[4] = {v.qh.x, v.qh.y, v.qh.z, v.qh.w};
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t src = (t & 1) ? lb[i] : la[i];
            const uint32_t lo = (src >> (4 * (t >> 1))) & 0x0F0F0F0Fu;
            const uint32_t hb = (qh[i] >> (2 * t)) & 0x03030303u;
            q[i] = lo | (hb << 4);  // q6 + 32, in 0..63
        }
        const int s = run_dot(q, xs.h + 4 * t, xs.l + 4 * t, 4) - 32 * xs.isum[t];
        const float sc = static_cast<float>(static_cast<int8_t>((v.sc >> (8 * t)) & 0xFFu));
        acc += sc * (xs.s[t] * static_cast<float>(s));
    }
    return f16lo(v.d) * acc;
}

// x offset of unit u and the stride between its four 16-element segments.
template <int TYPE>
__device__ __forceinline__ int64_t unit_x_offset(int u, int& seg_stride) {
    if constexpr (TYPE == TYPE_Q6_K) {
        const int c = u & 3;
        seg_stride = 32;
        return static_cast<int64_t>(u >> 2) * 256 + 128 * (c >> 1) + 16 * (c & 1);
    } else {
        seg_stride = 16;
        return static_cast<int64_t>(u) * 64;
    }
}

template <int TYPE>
__device__ __forceinline__ void load_unit_x(const float* x, int u, bool valid, XSlice& xs) {
    int seg_stride;
    const int64_t off = unit_x_offset<TYPE>(u, seg_stride);
    load_xslice<TYPE == TYPE_Q6_K ? 16 : 32>(x + off, seg_stride, valid, xs);
}

template <int TYPE, int R>
__global__ void __launch_bounds__(512) gemv_q_kernel(const uint8_t* __restrict__ w,
                                                     const float* __restrict__ x,
                                                     float* __restrict__ y, int64_t n, int64_t rb,
                                                     int units, int n_ktiles, int wpr,
                                                     int rows_per_group) {
    using Unit = typename UnitOf<TYPE>::T;
    __shared__ float red[8][R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int groups = (blockDim.x >> 6) / wpr;
    const int g = wave / wpr, kw = wave - g * wpr;
    const int64_t row0 =
        (static_cast<int64_t>(blockIdx.x) * groups + g) * static_cast<int64_t>(rows_per_group);
    const bool one_tile = n_ktiles <= wpr;

    XSlice xs;
    if (one_tile) {
        const int u = kw * 64 + lane;
        load_unit_x<TYPE>(x, u, kw < n_ktiles && u < units, xs);
    }
    for (int rr = 0; rr < rows_per_group; rr += R) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;
        for (int kt = kw; kt < n_ktiles; kt += wpr) {
            const int u = kt * 64 + lane;
            const bool valid = u < units;
            if (!one_tile) load_unit_x<TYPE>(x, u, valid, xs);
            if (valid) {
                Unit v[R];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    int64_t row = row0 + rr + r;
                    row = row < n ? row : n - 1;
                    load_unit(w + row * rb, u, v[r]);
                }
#pragma unroll
                for (int r = 0; r < R; r++) acc[r] += unit_dot(v[r], xs, u);
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
        if (wpr == 1) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int64_t row = row0 + rr + r;
                    if (row < n) y[row] = acc[r];
                }
            }
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; r++) red[wave][r] = acc[r];
            }
            __syncthreads();
            if (kw == 0 && lane < R) {
                float s = 0.f;
                for (int j = 0; j < wpr; j++) s += red[wave + j][lane];
                const int64_t row = row0 + rr + lane;
                if (row < n) y[row] = s;
            }
            __syncthreads();
        }
    }
}

// F32 / F16 weights: plain fp32 dot products, one wave per R rows.
template <int TYPE, int R>
__global__ void __launch_bounds__(256) gemv_plain_kernel(const uint8_t* __restrict__ w,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int64_t n,
                                                         int64_t k) {
    const int lane = threadIdx.x & 63;
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (int64_t i = lane; i < k; i += 64) {
        const float xv = x[i];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int64_t row = row0 + r;
            row = row < n ? row : n - 1;
            float wv;
            if constexpr (TYPE == TYPE_F32)
                wv = reinterpret_cast<const float*>(w)[row * k + i];
            else
                wv = __half2float(reinterpret_cast<const __half*>(w)[row * k + i]);
            acc[r] += wv * xv;
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++)
            if (row0 + r < n) y[row0 + r] = acc[r];
    }
}

constexpr int GEMV_R = 4;

struct GemvShape {
    int units, n_ktiles, wpr, wpg, rows_per_group;
    int64_t grid;
};

// Launch geometry for n rows of `units` 64-element units.  VB_GEMV_CFG="wpg,nb"
// overrides the waves per workgroup and the R-row batches per row group (for
// tuning sweeps).
GemvShape gemv_shape(int64_t n, int units) {
    GemvShape s;
    s.units = units;
    s.n_ktiles = (units + 63) / 64;
    s.wpr = s.n_ktiles <= 1 ? 1 : (s.n_ktiles <= 2 ? 2 : 4);
    int wpg = 4, nb = 1;
    if (const char* cfg = std::getenv("VB_GEMV_CFG")) {
        int a = 0, b = 0;
        if (std::sscanf(cfg, "%d,%d", &a, &b) == 2 && a >= 1 && a <= 8 && b >= 1) {
            wpg = a;
            nb = b;
        }
    }
    if (wpg % s.wpr != 0) wpg = s.wpr * ((wpg + s.wpr - 1) / s.wpr);
    if (wpg > 8) wpg = 8;
    s.wpg = wpg;
    s.rows_per_group = GEMV_R * nb;
    const int64_t rows_per_wg = static_cast<int64_t>(wpg / s.wpr) * s.rows_per_group;
    s.grid = (n + rows_per_wg - 1) / rows_per_wg;
    return s;
}

template <int TYPE>
int launch_gemv_q(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t rb,
                  hipStream_t st) {
    const GemvShape s = gemv_shape(n, static_cast<int>(k / 64));
    gemv_q_kernel<TYPE, GEMV_R><<<dim3(static_cast<uint32_t>(s.grid)), dim3(64 * s.wpg), 0, st>>>(
        static_cast<const uint8_t*>(w), x, y, n, rb, s.units, s.n_ktiles, s.wpr, s.rows_per_group);
    return check_launch("vb_gemv");
}

}  // namespace

// Shared with the other translation units (sparse / moe).
int gemv_dispatch(const void* w, const float* x, float* y, int64_t n, int64_t k, int32_t type,
                  hipStream_t st) {
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
    if ((type == TYPE_Q4_K || type == TYPE_Q6_K || type == TYPE_Q8_0) && k % 64 != 0) {
        set_error("vb_gemv: k=%lld must be a multiple of 64 for type %d", static_cast<long long>(k), type);
        return E_UNSUPPORTED;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 4 != 0) {
        set_error("vb_gemv: x must be 16-byte and W 4-byte aligned");
        return E_INVAL;
    }
    if (type == TYPE_Q4_K && reinterpret_cast<uintptr_t>(w) % 16 != 0) {
        set_error("vb_gemv: Q4_K weights must be 16-byte aligned");
        return E_INVAL;
    }
    switch (type) {
    case TYPE_Q4_K: return launch_gemv_q<TYPE_Q4_K>(w, x, y, n, k, rb, st);
    case TYPE_Q6_K: return launch_gemv_q<TYPE_Q6_K>(w, x, y, n, k, rb, st);
    case TYPE_Q8_0: return launch_gemv_q<TYPE_Q8_0>(w, x, y, n, k, rb, st);
    case TYPE_F32:
    case TYPE_F16: {
        constexpr int R = 4;
        const int64_t grid = (n + 4 * R - 1) / (4 * R);
        if (type == TYPE_F32)
            gemv_plain_kernel<TYPE_F32, R><<<dim3(static_cast<uint32_t>(grid)), dim3(256), 0, st>>>(
                static_cast<const uint8_t*>(w), x, y, n, k);
        else
            gemv_plain_kernel<TYPE_F16, R><<<dim3(static_cast<uint32_t>(grid)), dim3(256), 0, st>>>(
                static_cast<const uint8_t*>(w), x, y, n, k);
        return check_launch("vb_gemv");
    }
    default:
        set_error("vb_gemv: unsupported type %d", type);
        return E_UNSUPPORTED;
    }
}

}  // namespace vb

extern "C" int vb_gemv(const void* w, const float* x, float* y, int64_t n, int64_t k,
                       int32_t ggml_type, void* stream) {
    return vb::gemv_dispatch(w, x, y, n, k, ggml_type, vb::as_stream(stream));
}
