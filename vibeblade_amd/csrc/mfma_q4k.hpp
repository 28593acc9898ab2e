// Building blocks for the Q4_K x fp16 MFMA kernels (gemm.hip, moe.hip).
//
// Instruction: v_mfma_f32_16x16x32_f16 (gfx950), D[16x16] += A[16x32] B[32x16]
// with fp32 accumulation.  Operand layout for lane l (0..63):
//   A: row i = l % 16, k = 8 * (l / 16) + 0..7  (8 halves, 4 VGPRs)
//   B: col j = l % 16, k = 8 * (l / 16) + 0..7
//   D: col j = l % 16, rows i = 4 * (l / 16) + 0..3 (4 floats)
// The k order inside a lane's 8 halves is irrelevant to the product as long
// as A and B agree, so both use the order sigma = (0, 2, 1, 3, 4, 6, 5, 7):
// it lets the weight nibbles of a byte pair land in one half2 with one
// mask-and-or (see q4k_bfrags).
//
// Q4_K B fragments.  A 32-element MFMA k-step is exactly one Q4_K sub-block.
// Lane group g = l / 16 loads the 8 bytes qs[32c + 8g, +8) of chunk c; their
// low nibbles are elements 8g..8g+7 of sub-block 2c, their high nibbles the
// same elements of sub-block 2c+1, so one 8-byte load feeds two k-steps.  A
// nibble q becomes the half 1024 + q by or-ing in 0x6400 (exact), then
// w = (h - 1024) * (d*sc) - dmin*m with packed fp16 ops: the weight is
// rounded once to fp16 (rel. error <= 2^-11).
#pragma once

#include "vb_common.hpp"

namespace vb {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

union Frag {
    half8_t h;
    uint32_t u[4];
};

__device__ __forceinline__ float4_t mfma16x16x32(const Frag& a, const Frag& b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, b.h, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t h2bits(half2_t v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ half2_t bits2h(uint32_t v) { return __builtin_bit_cast(half2_t, v); }

// Apply sigma to 8 consecutive halves held as 4 dwords (x01, x23, x45, x67).
__device__ __forceinline__ void sigma_permute(uint32_t x01, uint32_t x23, uint32_t x45, uint32_t x67,
                                              uint32_t* o) {
    o[0] = __builtin_amdgcn_perm(x23, x01, 0x05040100u);  // (x0, x2)
    o[1] = __builtin_amdgcn_perm(x23, x01, 0x07060302u);  // (x1, x3)
    o[2] = __builtin_amdgcn_perm(x67, x45, 0x05040100u);  // (x4, x6)
    o[3] = __builtin_amdgcn_perm(x67, x45, 0x07060302u);  // (x5, x7)
}

// 8 fp32 -> 8 fp16 (round to nearest even), sigma order.
__device__ __forceinline__ void f32x8_to_frag(const float4& a, const float4& b, uint32_t* o) {
    auto pk = [](float lo, float hi) {
        const uint32_t l = __half_as_ushort(__float2half_rn(lo));
        const uint32_t h = __half_as_ushort(__float2half_rn(hi));
        return l | (h << 16);
    };
    o[0] = pk(a.x, a.z);
    o[1] = pk(a.y, a.w);
    o[2] = pk(b.x, b.z);
    o[3] = pk(b.y, b.w);
}

// 8 fp32 -> 8 fp16 (round to nearest even), natural order.
__device__ __forceinline__ void f32x8_to_frag_nat(const float4& a, const float4& b, uint32_t* o) {
    auto pk = [](float lo, float hi) {
        const uint32_t l = __half_as_ushort(__float2half_rn(lo));
        const uint32_t h = __half_as_ushort(__float2half_rn(hi));
        return l | (h << 16);
    };
    o[0] = pk(a.x, a.y);
    o[1] = pk(a.z, a.w);
    o[2] = pk(b.x, b.y);
    o[3] = pk(b.z, b.w);
}

// Per-row scale pair of Q4_K sub-blocks 2c and 2c+1 as fp16 half2 splats:
// ds[i] = d * sc_(2c+i), nm[i] = -(dmin * m_(2c+i)).  hd = the 16-byte block
// header (d, dmin, scales[12]); c is uniform across the wave.
__device__ __forceinline__ void q4k_chunk_scales(const uint4& hd, int c, half2_t* ds, half2_t* nm) {
    const uint32_t sh = 16u * static_cast<uint32_t>(c & 1);
    const uint32_t A = hd.y >> sh, B = hd.z >> sh, C = hd.w >> sh;
    uint32_t SC, M;
    if (c < 2) {
        SC = A & 0x3F3Fu;
        M = B & 0x3F3Fu;
    } else {
        SC = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u);
        M = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u);
    }
    const float d = f16lo(hd.x), dmin = f16hi(hd.x);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const _Float16 s = static_cast<_Float16>(d * static_cast<float>((SC >> (8 * i)) & 0xFFu));
        const _Float16 m = static_cast<_Float16>(-(dmin * static_cast<float>((M >> (8 * i)) & 0xFFu)));
        ds[i] = half2_t{s, s};
        nm[i] = half2_t{m, m};
    }
}

// Same values for a chunk index c that varies between waves: selects
// instead of a branch, so a loop that calls it stays one basic block (the
// scheduler can then interleave its VALU work with the MFMAs around it).
__device__ __forceinline__ void q4k_chunk_scales_sel(const uint4& hd, int c, half2_t* ds, half2_t* nm) {
    const uint32_t sh = 16u * static_cast<uint32_t>(c & 1);
    const uint32_t A = hd.y >> sh, B = hd.z >> sh, C = hd.w >> sh;
    const uint32_t lo = c < 2 ? 0xFFFFFFFFu : 0u;
    const uint32_t SC = (lo & A & 0x3F3Fu) | (~lo & ((C & 0x0F0Fu) | ((A >> 2) & 0x3030u)));
    const uint32_t M = (lo & B & 0x3F3Fu) | (~lo & (((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u)));
    const float d = f16lo(hd.x), dmin = f16hi(hd.x);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const _Float16 s = static_cast<_Float16>(d * static_cast<float>((SC >> (8 * i)) & 0xFFu));
        const _Float16 m = static_cast<_Float16>(-(dmin * static_cast<float>((M >> (8 * i)) & 0xFFu)));
        ds[i] = half2_t{s, s};
        nm[i] = half2_t{m, m};
    }
}

// Natural-k-order variant: dword i of a fragment holds elements (2i, 2i+1).
// v_perm spreads bytes (b0, b1) of a qs dword into the two halves first, so
// the activation operand needs no reordering (X can be staged as is).
__device__ __forceinline__ void q4k_bfrags_nat(uint32_t q0, uint32_t q1, const half2_t* ds, const half2_t* nm,
                                               Frag& lo, Frag& hi) {
    const half2_t k1024 = half2_t{static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    const uint32_t src[4] = {__builtin_amdgcn_perm(0u, q0, 0x0C010C00u), __builtin_amdgcn_perm(0u, q0, 0x0C030C02u),
                             __builtin_amdgcn_perm(0u, q1, 0x0C010C00u), __builtin_amdgcn_perm(0u, q1, 0x0C030C02u)};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const half2_t a = bits2h((src[i] & 0x000F000Fu) | 0x64006400u) - k1024;
        const half2_t b = bits2h(((src[i] >> 4) & 0x000F000Fu) | 0x64006400u) - k1024;
        lo.u[i] = h2bits(__builtin_elementwise_fma(a, ds[0], nm[0]));
        hi.u[i] = h2bits(__builtin_elementwise_fma(b, ds[1], nm[1]));
    }
}

// Natural k order through the scaled fp8 -> fp16 conversion: a byte holding
// a nibble q (0..15) is the OCP e4m3 code of q * 2^-9 exactly (codes 0..7
// are the subnormals q/8 * 2^-6, codes 8..15 the first binade (1 + (q-8)/8)
// * 2^-6), and v_cvt_scalef32_pk_f16_fp8 multiplies by the power of two in
// its f32 scale, so scale 2^9 gives q as fp16 exactly, two per instruction.
// One mask takes the four low nibbles of a word, a shift and a mask the four
// high ones.  The fma then rounds q * d * sc - dmin * m once, as in
// q4k_bfrags_nat: same results.
__device__ __forceinline__ void q4k_bfrags_cvt(uint32_t q0, uint32_t q1, const half2_t* ds, const half2_t* nm,
                                               Frag& lo, Frag& hi) {
    const uint32_t l0 = q0 & 0x0F0F0F0Fu, l1 = q1 & 0x0F0F0F0Fu;
    const uint32_t h0 = (q0 >> 4) & 0x0F0F0F0Fu, h1 = (q1 >> 4) & 0x0F0F0F0Fu;
    const half2_t a[4] = {__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l0, 512.0f, false),
                          __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l0, 512.0f, true),
                          __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l1, 512.0f, false),
                          __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l1, 512.0f, true)};
    const half2_t b[4] = {__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h0, 512.0f, false),
                          __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h0, 512.0f, true),
                          __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h1, 512.0f, false),
                          __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h1, 512.0f, true)};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        lo.u[i] = h2bits(__builtin_elementwise_fma(a[i], ds[0], nm[0]));
        hi.u[i] = h2bits(__builtin_elementwise_fma(b[i], ds[1], nm[1]));
    }
}

// Dequantize the two B fragments (sub-blocks 2c, 2c+1) of one lane from its
// 8 qs bytes (q0 = bytes 0-3, q1 = bytes 4-7), sigma order.
__device__ __forceinline__ void q4k_bfrags(uint32_t q0, uint32_t q1, const half2_t* ds,
                                           const half2_t* nm, Frag& lo, Frag& hi) {
    const half2_t k1024 = half2_t{static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    const uint32_t src[4] = {q0, q0 >> 8, q1, q1 >> 8};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const half2_t a = bits2h((src[i] & 0x000F000Fu) | 0x64006400u) - k1024;
        const half2_t b = bits2h(((src[i] >> 4) & 0x000F000Fu) | 0x64006400u) - k1024;
        lo.u[i] = h2bits(__builtin_elementwise_fma(a, ds[0], nm[0]));
        hi.u[i] = h2bits(__builtin_elementwise_fma(b, ds[1], nm[1]));
    }
}

// ---- 2-byte-aligned GGUF rows (Q6_K, Q8_0): 12-byte reads from a field's
// dword, realigned with v_alignbyte.  The buffer resource spans the tensor
// rounded up to whole dwords, so the dword past a field's end is either
// mapped tensor memory or outside the range (reads zero).
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

__device__ __forceinline__ u32x3 ld96(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b96(r, static_cast<int>(off), 0, 0);
}
__device__ __forceinline__ uint32_t ld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0);
}
// bytes [sh, sh + 8) of the 12 loaded bytes (sh = 0 or 2)
__device__ __forceinline__ void realign(const u32x3& v, uint32_t sh, uint32_t& x, uint32_t& y) {
    x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
}

// Constants of the Q6_K / Q8_0 decoders in VGPRs: gfx9 VOP3 takes no
// literal and one scalar operand at most.
struct KqConsts {
    uint32_t m0f, m30, h64, x80;
};
__device__ __forceinline__ KqConsts kq_consts() {
    KqConsts c;
    asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(c.m0f));
    asm volatile("v_mov_b32 %0, 0x00300030" : "=v"(c.m30));
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(c.h64));
    asm volatile("v_mov_b32 %0, 0x64806480" : "=v"(c.x80));
    return c;
}

// Q5_K codes to B-fragment dwords: chunk c of a super-block (elements 64 c ..
// 64 c + 63), 8 elements of each of its sub-blocks 2 c (lo) and 2 c + 1 (hi).
// q0, q1: the 8 qs bytes (low nibbles: sub-block 2 c, high: 2 c + 1); h0, h1:
// the qh bytes of the same element positions (bit 2 c, bit 2 c + 1).  Four
// codes per dword operation: a rotation moves each byte's qh bit to bit 4 of
// the same byte, the nibbles fill bits 0-3, v_perm with the 0x64 bytes of
// kc.h64 spreads bytes (0, 1) and (2, 3) into fp16 halves 1024 + q5 (exact);
// then (h - 1024) d sc - dmin m with one rounding.
__device__ __forceinline__ void q5k_frags(uint32_t q0, uint32_t q1, uint32_t h0, uint32_t h1, uint32_t c,
                                          const half2_t* ds, const half2_t* nm, const KqConsts& kc, Frag& lo,
                                          Frag& hi) {
    const half2_t k1024 = half2_t{static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    const uint32_t rl = (28u + 2u * c) & 31u, rh = (29u + 2u * c) & 31u;
    const uint32_t qd[2] = {q0, q1}, hd[2] = {h0, h1};
#pragma unroll
    for (int d = 0; d < 2; d++) {
        const uint32_t a = (__builtin_amdgcn_alignbit(hd[d], hd[d], rl) & 0x10101010u) | (qd[d] & 0x0F0F0F0Fu);
        const uint32_t b =
            (__builtin_amdgcn_alignbit(hd[d], hd[d], rh) & 0x10101010u) | ((qd[d] >> 4) & 0x0F0F0F0Fu);
        lo.u[2 * d] = h2bits(__builtin_elementwise_fma(bits2h(__builtin_amdgcn_perm(kc.h64, a, 0x07010500u)) - k1024,
                                                       ds[0], nm[0]));
        lo.u[2 * d + 1] = h2bits(__builtin_elementwise_fma(
            bits2h(__builtin_amdgcn_perm(kc.h64, a, 0x07030502u)) - k1024, ds[0], nm[0]));
        hi.u[2 * d] = h2bits(__builtin_elementwise_fma(bits2h(__builtin_amdgcn_perm(kc.h64, b, 0x07010500u)) - k1024,
                                                       ds[1], nm[1]));
        hi.u[2 * d + 1] = h2bits(__builtin_elementwise_fma(
            bits2h(__builtin_amdgcn_perm(kc.h64, b, 0x07030502u)) - k1024, ds[1], nm[1]));
    }
}

// ---- 32-element block types (GGUF Q4_0, Q4_1, Q5_0, Q5_1): fp16 d @0, fp16
// m @2 (Q4_1, Q5_1), then qh (Q5_0 @2, Q5_1 @4: bit e is the fifth bit of
// element e), then qs[16] (element e < 16: low nibble of qs[e], element
// 16 + e: high nibble).  w = d (q - kBias) or d q + m.
template <int TYPE> struct B32;
template <> struct B32<TYPE_Q4_0> {
    static constexpr uint32_t kBytes = 18, kQs = 2, kQh = 0;
    static constexpr bool kMin = false, kHigh = false;
    static constexpr int kBias = 8;
};
template <> struct B32<TYPE_Q4_1> {
    static constexpr uint32_t kBytes = 20, kQs = 4, kQh = 0;
    static constexpr bool kMin = true, kHigh = false;
    static constexpr int kBias = 0;
};
template <> struct B32<TYPE_Q5_0> {
    static constexpr uint32_t kBytes = 22, kQs = 6, kQh = 2;
    static constexpr bool kMin = false, kHigh = true;
    static constexpr int kBias = 16;
};
template <> struct B32<TYPE_Q5_1> {
    static constexpr uint32_t kBytes = 24, kQs = 8, kQh = 4;
    static constexpr bool kMin = true, kHigh = true;
    static constexpr int kBias = 0;
};

// Codes [8 e, 8 e + 8) of one block as a B fragment (dword i: elements 2 i,
// 2 i + 1): q0, q1 the qs bytes [8 (e % 2), +8), nibble nib = e / 2; qhb =
// byte e of qh; d = {d, d}; nb = {m, m} (Q4_1, Q5_1) or {-kBias d, ..}
// (Q4_0: exact, a power-of-two multiple of d).  4-bit codes become fp16
// through the scaled fp8 conversion (a byte n < 16 is the e4m3 code of n
// 2^-9), 5-bit codes through v_perm into halves 1024 + q (the qh bits spread
// to bit 4 of each byte by a multiply: no two shifted copies overlap); each
// weight is rounded to fp16 once.
template <int TYPE>
__device__ __forceinline__ void b32_frag(uint32_t q0, uint32_t q1, uint32_t nib, uint32_t qhb, half2_t d,
                                         half2_t nb, const KqConsts& kc, Frag& f) {
    using B = B32<TYPE>;
    const uint32_t v[2] = {(q0 >> (4u * nib)) & 0x0F0F0F0Fu, (q1 >> (4u * nib)) & 0x0F0F0F0Fu};
#pragma unroll
    for (int dd = 0; dd < 2; dd++) {
        if constexpr (!B::kHigh) {
            const half2_t n01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v[dd], 512.0f, false);
            const half2_t n23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v[dd], 512.0f, true);
            f.u[2 * dd] = h2bits(__builtin_elementwise_fma(n01, d, nb));
            f.u[2 * dd + 1] = h2bits(__builtin_elementwise_fma(n23, d, nb));
        } else {
            const uint32_t hb = (((qhb >> (4u * dd)) & 0xFu) * 0x00204081u) & 0x01010101u;
            const uint32_t a = v[dd] | (hb << 4);
            const half2_t h01 = bits2h(__builtin_amdgcn_perm(kc.h64, a, 0x07010500u));
            const half2_t h23 = bits2h(__builtin_amdgcn_perm(kc.h64, a, 0x07030502u));
            if constexpr (B::kMin) {
                const half2_t k1024 = half2_t{static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
                f.u[2 * dd] = h2bits(__builtin_elementwise_fma(h01 - k1024, d, nb));
                f.u[2 * dd + 1] = h2bits(__builtin_elementwise_fma(h23 - k1024, d, nb));
            } else {
                const _Float16 kb = static_cast<_Float16>(1024.0f + B::kBias);
                const half2_t kbb = half2_t{kb, kb};
                f.u[2 * dd] = h2bits((h01 - kbb) * d);
                f.u[2 * dd + 1] = h2bits((h23 - kbb) * d);
            }
        }
    }
}

// d and nb of b32_frag from the block's first dword (bytes 0-3 of the block)
template <int TYPE>
__device__ __forceinline__ void b32_scales(uint32_t w0, half2_t& d, half2_t& nb) {
    using B = B32<TYPE>;
    const uint32_t d16 = w0 & 0xFFFFu;
    d = bits2h(d16 | (d16 << 16));
    if constexpr (B::kMin) {
        const uint32_t m16 = w0 >> 16;
        nb = bits2h(m16 | (m16 << 16));
    } else {
        const _Float16 kb = static_cast<_Float16>(-static_cast<float>(B::kBias));
        nb = d * half2_t{kb, kb};
    }
}

// Codes [8 e, 8 e + 8) of a 32-element block from the six dwords that start
// at the block's address rounded down to 4 (sh = that address % 4, 0 or 2).
template <int TYPE>
__device__ __forceinline__ void b32_block_frag(const uint32_t* w, uint32_t sh, int e, const KqConsts& kc, Frag& f) {
    using B = B32<TYPE>;
    // block bytes [4 i, 4 i + 4); of b[5] only bytes 20, 21 are used (the
    // end of a 22-byte block, or a 24-byte block read aligned)
    uint32_t b[6];
#pragma unroll
    for (int i = 0; i < 5; i++) b[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
    b[5] = __builtin_amdgcn_alignbyte(w[5], w[5], sh);
    half2_t d, nb;
    b32_scales<TYPE>(b[0], d, nb);
    // dword k of a field at block byte o (o even): bytes [o + 4 k, +4)
    auto field = [&](uint32_t o, int k) -> uint32_t {
        const int i = static_cast<int>(o >> 2) + k;
        return (o & 3u) == 0 ? b[i] : __builtin_amdgcn_alignbyte(b[i + 1], b[i], 2u);
    };
    const uint32_t qo = B::kQs + 8u * static_cast<uint32_t>(e & 1);
    const uint32_t qh = B::kHigh ? field(B::kQh, 0) : 0u;
    b32_frag<TYPE>(field(qo, 0), field(qo, 1), static_cast<uint32_t>(e >> 1), (qh >> (8 * e)) & 0xFFu, d, nb, kc,
                   f);
}

// Q6_K codes to B-fragment dwords, 8 elements of each of two runs: l0 / l1
// the ql bytes of the runs (nibble p of each), qh their common qh bytes
// (bits 4 p, 4 p + 1 for the first run, 4 p + 2, 4 p + 3 for the second).
// Four codes per dword operation: rotating a qh dword right by 28 + 4 p (30
// + 4 p) moves each byte's two bits to bits 4, 5 of the same byte, the
// nibbles fill bits 0-3, and v_perm with the 0x64 bytes of kc.h64 spreads
// bytes (0, 1) and (2, 3) into fp16 halves 1024 + q (exact); then (h - 1056)
// x scale rounds each weight once.
__device__ __forceinline__ void q6k_frags(const uint32_t* l0, const uint32_t* l1, const uint32_t* qh, uint32_t p,
                                          half2_t ds0, half2_t ds1, const KqConsts& kc, Frag& lo, Frag& hi) {
    const half2_t k1056 = half2_t{static_cast<_Float16>(1056.0f), static_cast<_Float16>(1056.0f)};
    const uint32_t sx = 4u * p;
    const uint32_t rl = (28u + sx) & 31u, rh = (30u + sx) & 31u;
#pragma unroll
    for (int d = 0; d < 2; d++) {
        const uint32_t a =
            (__builtin_amdgcn_alignbit(qh[d], qh[d], rl) & 0x30303030u) | ((l0[d] >> sx) & 0x0F0F0F0Fu);
        const uint32_t b =
            (__builtin_amdgcn_alignbit(qh[d], qh[d], rh) & 0x30303030u) | ((l1[d] >> sx) & 0x0F0F0F0Fu);
        lo.u[2 * d] = h2bits((bits2h(__builtin_amdgcn_perm(kc.h64, a, 0x07010500u)) - k1056) * ds0);
        lo.u[2 * d + 1] = h2bits((bits2h(__builtin_amdgcn_perm(kc.h64, a, 0x07030502u)) - k1056) * ds0);
        hi.u[2 * d] = h2bits((bits2h(__builtin_amdgcn_perm(kc.h64, b, 0x07010500u)) - k1056) * ds1);
        hi.u[2 * d + 1] = h2bits((bits2h(__builtin_amdgcn_perm(kc.h64, b, 0x07030502u)) - k1056) * ds1);
    }
}

}  // namespace vb
