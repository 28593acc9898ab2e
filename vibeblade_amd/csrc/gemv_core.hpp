// Device building blocks of the dequant-fused M = 1 kernels (gemv.hip, and
// the fused sparse FFN in sparse.hip): the activation encoding shared by a
// workgroup through LDS and the per-type unit loads and integer dot products.
//
// Activation encoding.  The workgroup encodes x once into LDS: the 64
// activations of every unit are split into runs (32 elements for Q4_K / Q8_0,
// 16 for Q6_K: the weight sub-block size) and every run becomes 16-bit fixed
// point with a per-run fp32 scale:  x ~= s * x16,  |x16| <= 32512,  x16 = 256*xh + xl with
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
//   Q5_K  unit u: as Q4_K (header shared by the quad, qs[32c, 32c+32) at 48)
//         plus the whole qh[32] at 16: bit 2c / 2c+1 of qh[l] is the fifth
//         bit of the low / high nibble of qs[32c + l].
//   Q2_K / Q3_K  unit u: super-block u/4, c = u%4, h = c/2, j0 = 2 (c%2):
//         four 16-element runs t, codes = bits 2 (j0 + t/2) of qs[32h + 16 (t%2)
//         + i], scales of sub-blocks 4c + t; Q3_K adds bit 4h + j of hmask[l]
//         as the third code bit (clear: minus 4).
//   Q4_0 / Q4_1 / Q5_0 / Q5_1  unit u: blocks 2u, 2u+1 (36 / 40 / 44 / 48
//         bytes from u * that, 4-byte aligned); element j < 16 of a block is
//         the low nibble of qs[j], j + 16 the high nibble; the fifth bit of
//         element e is bit e of the block's 32-bit qh.
#pragma once

#include "vb_common.hpp"

namespace vb {
namespace gemvc {

constexpr int X16_MAX = 32512;  // 127 * 256: keeps xh within a signed byte

struct XSlice {
    uint32_t h[16];  // high bytes of x16, 4 per dword, element order
    uint32_t l[16];  // low bytes (signed), same order
    float s[4];      // per-run scale
    float sum[4];    // per-run sum of the fp32 activations
    int isum[4];     // per-run sum of x16
};

// ---- per-type unit loaders and dot products -------------------------------

// Q4_K: each of the 4 lanes of a super-block loads one dword of the 16-byte
// header (d|dmin, scales[0:4], scales[4:8], scales[8:12]) and the quad shares
// them through DPP broadcasts, instead of 4 lanes fetching the same 16 bytes.
struct Q4KUnit { uint32_t hw; uint4 qa, qb; };
struct Q5KUnit { uint32_t hw; uint4 qa, qb, ha, hb; };
struct Q8Unit { uint4 a, b, c, d; uint32_t e; };
struct Q6KUnit { uint4 la, lb, qh; uint32_t sc; uint32_t d; };
// two 32-element blocks of NW dwords in all
template <int NW> struct LegacyUnit { uint32_t w[NW]; };
struct Q2KUnit { uint4 qa, qb; uint32_t sc, dd; };
struct Q3KUnit { uint4 qa, qb, ha, hb; uint32_t s0, s1, s2, d; };

template <int TYPE> struct UnitOf;
template <> struct UnitOf<TYPE_Q4_K> { using T = Q4KUnit; };
template <> struct UnitOf<TYPE_Q5_K> { using T = Q5KUnit; };
template <> struct UnitOf<TYPE_Q8_0> { using T = Q8Unit; };
template <> struct UnitOf<TYPE_Q6_K> { using T = Q6KUnit; };
template <> struct UnitOf<TYPE_Q2_K> { using T = Q2KUnit; };
template <> struct UnitOf<TYPE_Q3_K> { using T = Q3KUnit; };
template <> struct UnitOf<TYPE_Q4_0> { using T = LegacyUnit<9>; };
template <> struct UnitOf<TYPE_Q4_1> { using T = LegacyUnit<10>; };
template <> struct UnitOf<TYPE_Q5_0> { using T = LegacyUnit<11>; };
template <> struct UnitOf<TYPE_Q5_1> { using T = LegacyUnit<12>; };

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, Q4KUnit& v) {
    const uint8_t* b = row + (u >> 2) * 144;
    const int c = u & 3;
    v.hw = ld_b32(b + 4 * c);
    v.qa = *reinterpret_cast<const uint4*>(b + 16 + 32 * c);
    v.qb = *reinterpret_cast<const uint4*>(b + 32 + 32 * c);
}

// Value of v in lane I of this lane's quad (DPP quad_perm [I,I,I,I]).
template <int I>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), I * 0x55, 0xF, 0xF, false));
}

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, Q8Unit& v) {
    const uint8_t* b = row + u * 68;
    v.a = ld_b128_a4(b);
    v.b = ld_b128_a4(b + 16);
    v.c = ld_b128_a4(b + 32);
    v.d = ld_b128_a4(b + 48);
    v.e = ld_b32(b + 64);
}

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, Q5KUnit& v) {
    const uint8_t* b = row + (u >> 2) * 176;
    const int c = u & 3;
    v.hw = ld_b32(b + 4 * c);
    v.ha = *reinterpret_cast<const uint4*>(b + 16);
    v.hb = *reinterpret_cast<const uint4*>(b + 32);
    v.qa = *reinterpret_cast<const uint4*>(b + 48 + 32 * c);
    v.qb = *reinterpret_cast<const uint4*>(b + 64 + 32 * c);
}

template <int NW>
__device__ __forceinline__ void load_unit(const uint8_t* row, int u, LegacyUnit<NW>& v) {
    const uint8_t* b = row + static_cast<int64_t>(u) * (4 * NW);
#pragma unroll
    for (int i = 0; i + 4 <= NW; i += 4) {
        const uint4 t = ld_b128_a4(b + 4 * i);
        v.w[i] = t.x; v.w[i + 1] = t.y; v.w[i + 2] = t.z; v.w[i + 3] = t.w;
    }
#pragma unroll
    for (int i = NW / 4 * 4; i < NW; i++) v.w[i] = ld_b32(b + 4 * i);
}

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, Q2KUnit& v) {
    const uint8_t* b = row + (u >> 2) * 84;  // 4-byte aligned
    const int c = u & 3;
    v.qa = ld_b128_a4(b + 16 + 32 * (c >> 1));
    v.qb = ld_b128_a4(b + 32 + 32 * (c >> 1));
    v.sc = ld_b32(b + 4 * c);
    v.dd = ld_b32(b + 80);
}

__device__ __forceinline__ uint32_t ld_b32_a2(const uint8_t* p) {
    return static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(p)) |
           (static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(p + 2)) << 16);
}

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, Q3KUnit& v) {
    const uint8_t* b = row + (u >> 2) * 110;  // 2-byte aligned
    const int c = u & 3;
    v.qa = ld_b128_a2(b + 32 + 32 * (c >> 1));
    v.qb = ld_b128_a2(b + 48 + 32 * (c >> 1));
    v.ha = ld_b128_a2(b);
    v.hb = ld_b128_a2(b + 16);
    v.s0 = ld_b32_a2(b + 96);
    v.s1 = ld_b32_a2(b + 100);
    v.s2 = ld_b32_a2(b + 104);
    v.d = *reinterpret_cast<const uint16_t*>(b + 108);
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

// Lane-constant selectors of the 6-bit scale / min of sub-blocks 2c, 2c+1
// (c = the lane's chunk; get_scale_min_k4, cpp/src/dequant.cpp:258-266),
// with sh = 16 (c & 1) and A, B, C = scales[0:4], [4:8], [8:12]:
//   c < 2:  sc = (A >> sh) & 0x3F3F,  m = (B >> sh) & 0x3F3F
//   c >= 2: sc = ((C >> sh) & 0x0F0F) | ((A >> (sh + 2)) & 0x3030)
//           m  = ((C >> (sh + 4)) & 0x0F0F) | ((B >> (sh + 2)) & 0x3030)
struct Q4KSel {
    uint32_t sh, sh2, shm, m1, m2;
    bool hi;
};

template <int TYPE>
__device__ __forceinline__ auto make_unit_sel(int u) {
    if constexpr (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K) {
        const int c = u & 3;
        Q4KSel q;
        q.hi = c >= 2;
        q.sh = 16u * static_cast<uint32_t>(c & 1);
        q.sh2 = q.sh + 2u;
        q.shm = q.hi ? q.sh + 4u : q.sh;
        q.m1 = q.hi ? 0x0F0Fu : 0x3F3Fu;
        q.m2 = q.hi ? 0x3030u : 0u;
        return q;
    } else {
        return u;
    }
}

// High nibbles enter the dot products as (q ^ 0x80) & 0xF0 = 16 (q - 8), a
// signed byte, with one v_bitop3 per 4 bytes instead of a shift and a mask:
//   sum x16 q = (sum x16 16 (q - 8) + 128 isum) / 16   (exact; isum = sum x16)
__device__ __forceinline__ float unit_dot(const Q4KUnit& v, const XSlice& xs, const Q4KSel& q) {
    const uint32_t qd[8] = {v.qa.x, v.qa.y, v.qa.z, v.qa.w, v.qb.x, v.qb.y, v.qb.z, v.qb.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = qd[i] & 0x0F0F0F0Fu;
        hi[i] = (qd[i] ^ 0x80808080u) & 0xF0F0F0F0u;
    }
    const int s0 = run_dot(lo, xs.h, xs.l, 8);
    const int s1 = (run_dot(hi, xs.h + 8, xs.l + 8, 8) + 128 * xs.isum[1]) >> 4;
    // The quad's lanes hold units c = 0..3 of the same super-block and share
    // its 16-byte header through DPP broadcasts.
    const uint32_t hx = quad_bcast<0>(v.hw);
    const uint32_t A = quad_bcast<1>(v.hw), B = quad_bcast<2>(v.hw), C = quad_bcast<3>(v.hw);
    const uint32_t SC = (((q.hi ? C : A) >> q.sh) & q.m1) | ((A >> q.sh2) & q.m2);
    const uint32_t M = (((q.hi ? C : B) >> q.shm) & q.m1) | ((B >> q.sh2) & q.m2);
    const float d = f16lo(hx), dmin = f16hi(hx);
    const float sc0 = static_cast<float>(SC & 0xFFu), sc1 = static_cast<float>((SC >> 8) & 0xFFu);
    const float m0 = static_cast<float>(M & 0xFFu), m1 = static_cast<float>((M >> 8) & 0xFFu);
    const float dot = sc0 * (xs.s[0] * static_cast<float>(s0)) + sc1 * (xs.s[1] * static_cast<float>(s1));
    const float mins = m0 * xs.sum[0] + m1 * xs.sum[1];
    return d * dot - dmin * mins;
}

// Q5_K: the Q4_K selectors; q5 = nibble | fifth bit << 4 (0..31) enters
// the dot products directly.
__device__ __forceinline__ float unit_dot(const Q5KUnit& v, const XSlice& xs, const Q4KSel& q) {
    const uint32_t qd[8] = {v.qa.x, v.qa.y, v.qa.z, v.qa.w, v.qb.x, v.qb.y, v.qb.z, v.qb.w};
    const uint32_t hd[8] = {v.ha.x, v.ha.y, v.ha.z, v.ha.w, v.hb.x, v.hb.y, v.hb.z, v.hb.w};
    const uint32_t c2 = 2u * ((q.sh >> 4) + (q.hi ? 2u : 0u));  // 2c for chunk c = u % 4
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = (qd[i] & 0x0F0F0F0Fu) | (((hd[i] >> c2) & 0x01010101u) << 4);
        hi[i] = ((qd[i] >> 4) & 0x0F0F0F0Fu) | (((hd[i] >> (c2 + 1)) & 0x01010101u) << 4);
    }
    const int s0 = run_dot(lo, xs.h, xs.l, 8);
    const int s1 = run_dot(hi, xs.h + 8, xs.l + 8, 8);
    const uint32_t hx = quad_bcast<0>(v.hw);
    const uint32_t A = quad_bcast<1>(v.hw), B = quad_bcast<2>(v.hw), C = quad_bcast<3>(v.hw);
    const uint32_t SC = (((q.hi ? C : A) >> q.sh) & q.m1) | ((A >> q.sh2) & q.m2);
    const uint32_t M = (((q.hi ? C : B) >> q.shm) & q.m1) | ((B >> q.sh2) & q.m2);
    const float d = f16lo(hx), dmin = f16hi(hx);
    const float sc0 = static_cast<float>(SC & 0xFFu), sc1 = static_cast<float>((SC >> 8) & 0xFFu);
    const float m0 = static_cast<float>(M & 0xFFu), m1 = static_cast<float>((M >> 8) & 0xFFu);
    const float dot = sc0 * (xs.s[0] * static_cast<float>(s0)) + sc1 * (xs.s[1] * static_cast<float>(s1));
    const float mins = m0 * xs.sum[0] + m1 * xs.sum[1];
    return d * dot - dmin * mins;
}

// Q2_K: sum over the four 16-element runs of d sc_t s_t Σ x16 q2 - dmin m_t Σ x.
__device__ __forceinline__ float unit_dot(const Q2KUnit& v, const XSlice& xs, int u) {
    const uint32_t qd[8] = {v.qa.x, v.qa.y, v.qa.z, v.qa.w, v.qb.x, v.qb.y, v.qb.z, v.qb.w};
    const int j0 = 2 * (u & 1);
    float acc = 0.f, accm = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int sh = 2 * (j0 + t / 2);
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = (qd[4 * (t & 1) + i] >> sh) & 0x03030303u;
        const int sdot = run_dot(q, xs.h + 4 * t, xs.l + 4 * t, 4);
        const uint32_t sm = (v.sc >> (8 * t)) & 0xFFu;
        acc += static_cast<float>(sm & 0xFu) * (xs.s[t] * static_cast<float>(sdot));
        accm += static_cast<float>(sm >> 4) * xs.sum[t];
    }
    return f16lo(v.dd) * acc - f16hi(v.dd) * accm;
}

// Q3_K: codes q2 | hbit << 2 (0..7), minus 4 through the run's x16 sum; the
// 6-bit scale of sub-block 4c + t: low 4 bits from byte 4c + t (c < 2) or the
// high nibble of byte 4(c - 2) + t, high 2 bits from bits 2c of byte 8 + t.
__device__ __forceinline__ float unit_dot(const Q3KUnit& v, const XSlice& xs, int u) {
    const uint32_t qd[8] = {v.qa.x, v.qa.y, v.qa.z, v.qa.w, v.qb.x, v.qb.y, v.qb.z, v.qb.w};
    const uint32_t hd[8] = {v.ha.x, v.ha.y, v.ha.z, v.ha.w, v.hb.x, v.hb.y, v.hb.z, v.hb.w};
    const int c = u & 3, h = c >> 1, j0 = 2 * (c & 1);
    const uint32_t lowsrc = (c & 1) ? v.s1 : v.s0;
    const int lowsh = c >= 2 ? 4 : 0;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int j = j0 + t / 2;
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int w = 16 * (t & 1) / 4 + i;  // dword of bytes l = 16 (t%2) + 4i ..
            q[i] = ((qd[w] >> (2 * j)) & 0x03030303u) | (((hd[w] >> (4 * h + j)) & 0x01010101u) << 2);
        }
        const int sdot = run_dot(q, xs.h + 4 * t, xs.l + 4 * t, 4) - 4 * xs.isum[t];
        const int lo = static_cast<int>((lowsrc >> (8 * t + lowsh)) & 0xFu);
        const int hi = static_cast<int>((v.s2 >> (8 * t + 2 * c)) & 3u);
        acc += static_cast<float>((lo | (hi << 4)) - 32) * (xs.s[t] * static_cast<float>(sdot));
    }
    return f16lo(v.d) * acc;
}

// Fifth bits b (4 consecutive elements, bits 0..3) moved to bit 4 of each byte.
__device__ __forceinline__ uint32_t bits_to_bytes4(uint32_t b) {
    return ((b & 1u) | ((b & 2u) << 7) | ((b & 4u) << 14) | ((b & 8u) << 21)) << 4;
}

// The 32-element block types.  Block r (r = 0, 1) of the unit is run r:
// 16 code bytes -> low nibbles = elements 0..15, high = 16..31, each with
// its fifth bit from qh.  Σ x·y = d·s·(Σ x16·q - off·isum) + m·Σx.
template <int TYPE, int NW>
__device__ __forceinline__ float legacy_dot(const LegacyUnit<NW>& v, const XSlice& xs) {
    constexpr bool HAS_M = TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_1;
    constexpr bool HAS_H = TYPE == TYPE_Q5_0 || TYPE == TYPE_Q5_1;
    constexpr int BB = 2 * NW;                     // block bytes
    constexpr int QH = HAS_M ? 4 : 2;              // qh offset in a block
    constexpr int QS = QH + (HAS_H ? 4 : 0);       // qs offset
    constexpr int OFF = HAS_M ? 0 : (HAS_H ? 16 : 8);
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int base = r * BB;  // byte offset of the block in the unit
        auto byte_word = [&](int off) -> uint32_t {  // 4 bytes from any 2-byte offset
            const int o = base + off;
            if (o % 4 == 0) return v.w[o / 4];
            return __builtin_amdgcn_alignbyte(v.w[o / 4 + 1], v.w[o / 4], 2);
        };
        const uint32_t hdr = byte_word(0);  // d (low half), m (high half, when present)
        const float d = (base % 4 == 0) ? f16lo(v.w[base / 4]) : f16hi(v.w[base / 4]);
        const float m = HAS_M ? f16hi(hdr) : 0.f;
        const uint32_t qh = HAS_H ? byte_word(QH) : 0u;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = byte_word(QS + 4 * i);
            lo[i] = w & 0x0F0F0F0Fu;
            hi[i] = (w >> 4) & 0x0F0F0F0Fu;
            if constexpr (HAS_H) {
                lo[i] |= bits_to_bytes4((qh >> (4 * i)) & 0xFu);
                hi[i] |= bits_to_bytes4((qh >> (16 + 4 * i)) & 0xFu);
            }
        }
        int sdot = run_dot(lo, xs.h + 8 * r, xs.l + 8 * r, 4) + run_dot(hi, xs.h + 8 * r + 4, xs.l + 8 * r + 4, 4);
        if constexpr (OFF != 0) sdot -= OFF * xs.isum[r];
        acc += d * (xs.s[r] * static_cast<float>(sdot));
        if constexpr (HAS_M) acc += m * xs.sum[r];
    }
    return acc;
}

__device__ __forceinline__ float unit_dot(const LegacyUnit<9>& v, const XSlice& xs, int) {
    return legacy_dot<TYPE_Q4_0>(v, xs);
}
__device__ __forceinline__ float unit_dot(const LegacyUnit<10>& v, const XSlice& xs, int) {
    return legacy_dot<TYPE_Q4_1>(v, xs);
}
__device__ __forceinline__ float unit_dot(const LegacyUnit<11>& v, const XSlice& xs, int) {
    return legacy_dot<TYPE_Q5_0>(v, xs);
}
__device__ __forceinline__ float unit_dot(const LegacyUnit<12>& v, const XSlice& xs, int) {
    return legacy_dot<TYPE_Q5_1>(v, xs);
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

// ---- shared activation encoding (LDS) -------------------------------------
//
// The encoded slice of unit u lives in LDS as 11 uint4 "quads" at
// xq[q * slots + u]: quads 0-3 = h[0..15], 4-7 = l[0..15], 8 = s[0..3],
// 9 = sum[0..3], 10 = isum[0..3].  A wave's lanes read consecutive units, so
// their ds_read_b128 loads are bank-conflict free.  `slots` (a multiple of 8)
// covers every unit index a lane may read, idle lanes included; units past
// the row are encoded as zeros.
constexpr int XQ_QUADS = 11;
constexpr int kMaxSlots = 520;      // LDS encoding up to k = 32768 (+ idle lanes)
constexpr int kMaxRedFloats = 8192;  // per-row partial sums kept in LDS

// All threads of the workgroup encode the activations of every slot: one
// task = 8 consecutive elements of a unit; the 2 (Q6_K) or 4 tasks of a run
// sit on adjacent lanes and combine their max / sums with shuffles.  Loading
// is split from encoding so the caller can put the weight loads in between:
// loads return in issue order, so x must be requested first or its encode
// would wait for the weights.
constexpr int XT_MAX = 2;  // tasks per thread held in registers

struct XTasks {
    float v[XT_MAX][8];
};

template <int TYPE>
__device__ __forceinline__ int64_t task_x_offset(int u, int p) {
    if constexpr (TYPE == TYPE_Q6_K) {
        int seg_stride;
        return unit_x_offset<TYPE>(u, seg_stride) + (p >> 1) * 32 + 8 * (p & 1);
    } else {
        return static_cast<int64_t>(u) * 64 + 8 * p;
    }
}

// Loads are branch-free (clamped address; the value is masked later, in
// encode_x_task): a load under a branch makes the compiler's wait-count
// merge fall back to vmcnt(0), and masking here would wait for the load.
template <int TYPE>
__device__ __forceinline__ void load_x_task(const float* __restrict__ x, int units, int task, float* v) {
    const int u = task >> 3, p = task & 7;
    const int64_t off = task_x_offset<TYPE>(u < units ? u : units - 1, p);
    const float4 a = *reinterpret_cast<const float4*>(x + off);
    const float4 b = *reinterpret_cast<const float4*>(x + off + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Value of v in lane i ^ 1 (M = 1) or i ^ 2 (M = 2) of this lane's quad
// (DPP quad_perm): the run reductions stay in registers, no LDS round trip.
template <int M>
__device__ __forceinline__ float quad_xor(float v) {
    constexpr int CTRL = M == 1 ? 0xB1 : 0x4E;  // [1,0,3,2] / [2,3,0,1]
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int M>
__device__ __forceinline__ int quad_xor(int v) {
    constexpr int CTRL = M == 1 ? 0xB1 : 0x4E;
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// `store` false: the task only takes part in the run reductions of its
// neighbours (every lane of the wave must run them); nothing is written.
template <int TYPE>
__device__ __forceinline__ void encode_x_task(int task, int units, int slots, const float* vin, uint4* xq,
                                              bool store = true) {
    constexpr int RUNLEN = (TYPE == TYPE_Q6_K || TYPE == TYPE_Q2_K || TYPE == TYPE_Q3_K) ? 16 : 32;
    constexpr int TPR = RUNLEN / 8;
    static_assert(TPR == 2 || TPR == 4, "runs of 2 or 4 tasks (one quad)");
    const int u = task >> 3, p = task & 7;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = u < units ? vin[i] : 0.f;
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    amax = fmaxf(amax, quad_xor<1>(amax));
    sum += quad_xor<1>(sum);
    if constexpr (TPR == 4) {
        amax = fmaxf(amax, quad_xor<2>(amax));
        sum += quad_xor<2>(sum);
    }
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
    isum += quad_xor<1>(isum);
    if constexpr (TPR == 4) isum += quad_xor<2>(isum);
    if (!store) return;
    uint4* base = xq + u;
    reinterpret_cast<uint2*>(&base[(p >> 1) * slots])[p & 1] = make_uint2(ph[0], ph[1]);
    reinterpret_cast<uint2*>(&base[(4 + (p >> 1)) * slots])[p & 1] = make_uint2(pl[0], pl[1]);
    if (p % TPR == 0) {
        const int r = p / TPR;
        reinterpret_cast<float*>(&base[8 * slots])[r] = amax / static_cast<float>(X16_MAX);
        reinterpret_cast<float*>(&base[9 * slots])[r] = sum;
        reinterpret_cast<int*>(&base[10 * slots])[r] = isum;
    }
}

// Register path: at most XT_MAX tasks per thread.  The task count (8 per
// slot, slots a multiple of 8) and the thread count are multiples of 64, so
// each wave's shuffles see all 64 lanes active.  No branch around a task's
// encode (threads past the task count redo the last task and store
// nothing): an encode under a branch makes the compiler wait for every load
// in flight, the weight loads issued after x included.
template <int TYPE>
__device__ __forceinline__ void prefetch_x(const float* __restrict__ x, int units, int slots, XTasks& t) {
    const int ntasks = slots * 8;
#pragma unroll
    for (int i = 0; i < XT_MAX; i++) {
        const int task = threadIdx.x + i * blockDim.x;
        load_x_task<TYPE>(x, units, task < ntasks ? task : ntasks - 1, t.v[i]);
    }
}

template <int TYPE>
__device__ __forceinline__ void encode_x_regs(int units, int slots, const XTasks& t, uint4* xq) {
    const int ntasks = slots * 8;
#pragma unroll
    for (int i = 0; i < XT_MAX; i++) {
        const int task = threadIdx.x + i * blockDim.x;
        encode_x_task<TYPE>(task < ntasks ? task : ntasks - 1, units, slots, t.v[i], xq, task < ntasks);
    }
}

// Loop path for more tasks than fit in registers.
template <int TYPE>
__device__ void encode_x_loop(const float* __restrict__ x, int units, int slots, uint4* xq) {
    const int ntasks = slots * 8;
    for (int task = threadIdx.x; task < ntasks; task += blockDim.x) {
        float v[8];
        load_x_task<TYPE>(x, units, task, v);
        encode_x_task<TYPE>(task, units, slots, v, xq);
    }
}

// ---- RMSNorm folded into the encode ----------------------------------------
//
// x -> x * rinv * w with rinv = 1 / sqrt(sum(x^2) / k + eps) (the reference's
// rms_norm, cpp/src/fast_model.cpp:61-71).  The workgroup reduces sum(x^2)
// itself: the register path from the tasks it already holds (each element of
// x sits in exactly one valid task), the loop path with a pass over x.

// Sum of one float per thread over the workgroup, in a fixed order (wave
// sums, then waves 0, 1, ... in turn), so every thread and every workgroup
// gets the same value.  red: one float per wave of LDS, free until the
// barrier that follows the caller's next use of it.
__device__ __forceinline__ float wg_sum_fixed(float v, float* red) {
    const float t = wave_sum_dpp(v);
    const int nw = static_cast<int>(blockDim.x >> 6);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

__device__ __forceinline__ float rms_inv(float sumsq, int k, float eps) {
    return 1.0f / sqrtf(sumsq / static_cast<float>(k) + eps);
}

// Register path: this thread's share of sum(x^2) over its valid tasks.
__device__ __forceinline__ float sumsq_tasks(int units, int slots, const XTasks& t) {
    const int ntasks = slots * 8;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < XT_MAX; i++) {
        const int task = threadIdx.x + i * blockDim.x;
        if (task < ntasks && (task >> 3) < units) {
#pragma unroll
            for (int j = 0; j < 8; j++) s += t.v[i][j] * t.v[i][j];
        }
    }
    return s;
}

// Register path: t = t * rinv * w, w the norm weights of the same tasks.
__device__ __forceinline__ void scale_tasks(XTasks& t, const XTasks& w, float rinv) {
#pragma unroll
    for (int i = 0; i < XT_MAX; i++) {
#pragma unroll
        for (int j = 0; j < 8; j++) t.v[i][j] = t.v[i][j] * rinv * w.v[i][j];
    }
}

// Loop path: this thread's share of sum(x^2) over x[0, k) (k a multiple of 4,
// x 16-byte aligned).
__device__ __forceinline__ float sumsq_loop(const float* __restrict__ x, int k) {
    float s = 0.f;
    for (int i = 4 * static_cast<int>(threadIdx.x); i < k; i += 4 * static_cast<int>(blockDim.x)) {
        const float4 a = *reinterpret_cast<const float4*>(x + i);
        s += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    return s;
}

template <int TYPE>
__device__ void encode_x_loop_norm(const float* __restrict__ x, const float* __restrict__ nw, float rinv,
                                   int units, int slots, uint4* xq) {
    const int ntasks = slots * 8;
    for (int task = threadIdx.x; task < ntasks; task += blockDim.x) {
        float v[8], w[8];
        load_x_task<TYPE>(x, units, task, v);
        load_x_task<TYPE>(nw, units, task, w);
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = v[j] * rinv * w[j];
        encode_x_task<TYPE>(task, units, slots, v, xq);
    }
}

__device__ __forceinline__ void read_xslice(const uint4* xq, int slots, int u, XSlice& xs) {
    const uint4* q = xq + u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 h = q[i * slots], l = q[(4 + i) * slots];
        xs.h[4 * i] = h.x; xs.h[4 * i + 1] = h.y; xs.h[4 * i + 2] = h.z; xs.h[4 * i + 3] = h.w;
        xs.l[4 * i] = l.x; xs.l[4 * i + 1] = l.y; xs.l[4 * i + 2] = l.z; xs.l[4 * i + 3] = l.w;
    }
    const uint4 s = q[8 * slots], sm = q[9 * slots], is = q[10 * slots];
    xs.s[0] = __uint_as_float(s.x); xs.s[1] = __uint_as_float(s.y);
    xs.s[2] = __uint_as_float(s.z); xs.s[3] = __uint_as_float(s.w);
    xs.sum[0] = __uint_as_float(sm.x); xs.sum[1] = __uint_as_float(sm.y);
    xs.sum[2] = __uint_as_float(sm.z); xs.sum[3] = __uint_as_float(sm.w);
    xs.isum[0] = static_cast<int>(is.x); xs.isum[1] = static_cast<int>(is.y);
    xs.isum[2] = static_cast<int>(is.z); xs.isum[3] = static_cast<int>(is.w);
}


}  // namespace gemvc
}  // namespace vb
