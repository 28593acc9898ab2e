// Block decode (vb_dequant_rows) and block encode (vb_quantize_rows).
//
// Decode formulas (GGUF standard; the Q4_K one is identical to
// cpp/src/dequant.cpp:258-301):
//   Q8_0: y = q * d
//   Q4_K: y = (d * sc_j) * nib - (dmin * m_j), sub-block j = e / 32
//   Q5_K: as Q4_K with q5 = nib + 16 * (bit 2c or 2c+1 of qh[l]), c = e / 64
//   Q6_K: y = (d * sc_s) * (q6 - 32),          sub-block s = e / 16
//   Q4_0: y = (q - 8) * d;  Q4_1: y = d * q + m   (q: element j < 16 in the
//         low nibble of qs[j], element j + 16 in its high nibble)
//   Q5_0: y = (q5 - 16) * d;  Q5_1: y = d * q5 + m (fifth bit of element e:
//         bit e of the 32-bit qh)
//   Q2_K: y = (d * sc_s) * q2 - (dmin * m_s), s = e / 16, q2 = bits 2j of
//         qs[32h + l] for e = 128h + 32j + l
//   Q3_K: y = (d * (sc6_s - 32)) * (q2 + 4 * hbit - 4), hbit = bit 4h + j of
//         hmask[l]
//   BF16: the 16 bits above 16 zero bits
// Every product here is exact in fp32 (at most 23 significant bits), so the
// only rounding is the final add or subtraction, and the result is
// bit-identical to any CPU evaluation of the same formula.
#include "vb_common.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// Q4_K sub-block scale/min (the 6-bit packing of cpp/src/dequant.cpp:258-266).
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t* s, float& sc, float& m) {
    if (j < 4) {
        sc = static_cast<float>(s[j] & 63);
        m = static_cast<float>(s[j + 4] & 63);
    } else {
        sc = static_cast<float>((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        m = static_cast<float>((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

// Four 4-bit codes (bytes of n4, low nibbles) and their fifth bits (bits 0..3
// of h4) as four ints.
__device__ __forceinline__ void nib4(uint32_t n4, uint32_t h4, int (&q)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = static_cast<int>(((n4 >> (8 * i)) & 0xF) | (((h4 >> i) & 1u) << 4));
}

// Elements e0 .. e0+3 of the row at rp (e0 a multiple of 4).
template <int TYPE>
__device__ __forceinline__ float4 decode4(const uint8_t* __restrict__ rp, int64_t e0) {
    float4 y;
    if constexpr (TYPE == TYPE_Q4_0 || TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_0 || TYPE == TYPE_Q5_1) {
        constexpr int BB = static_cast<int>(block_bytes(TYPE));
        constexpr bool HAS_M = TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_1;
        constexpr bool HAS_H = TYPE == TYPE_Q5_0 || TYPE == TYPE_Q5_1;
        const uint8_t* b = rp + (e0 / 32) * BB;
        const int i0 = static_cast<int>(e0 % 32);  // 4 elements in one half
        const float d = f16lo(ld_u16(b));
        const float m = HAS_M ? f16lo(ld_u16(b + 2)) : 0.f;
        const int qh_off = HAS_M ? 4 : 2, qs_off = qh_off + (HAS_H ? 4 : 0);
        const uint32_t qh = HAS_H ? (ld_u16(b + qh_off) | (ld_u16(b + qh_off + 2) << 16)) : 0u;
        const int j = i0 & 15;
        const uint32_t bytes = ld_u16(b + qs_off + j) | (ld_u16(b + qs_off + j + 2) << 16);
        const uint32_t n4 = i0 < 16 ? bytes : bytes >> 4;
        int q[4];
        nib4(n4, qh >> i0, q);
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if constexpr (HAS_M)
                v[i] = d * static_cast<float>(q[i]) + m;
            else
                v[i] = static_cast<float>(q[i] - (HAS_H ? 16 : 8)) * d;
        }
        return make_float4(v[0], v[1], v[2], v[3]);
    }
    if constexpr (TYPE == TYPE_Q4_K) {
        const uint8_t* b = rp + (e0 / 256) * 144;
        const int wi = static_cast<int>(e0 % 256);
        const int c = wi / 64, l = wi % 32, hi = (wi % 64) / 32;
        const uint32_t hd = ld_b32(b);
        const float d = f16lo(hd), dmin = f16hi(hd);
        float sc, m;
        q4k_scale_min(2 * c + hi, b + 4, sc, m);
        const float d1 = d * sc, m1 = dmin * m;
        const uint32_t q = ld_b32(b + 16 + 32 * c + l) >> (4 * hi);
        y.x = d1 * static_cast<float>(q & 0xF) - m1;
        y.y = d1 * static_cast<float>((q >> 8) & 0xF) - m1;
        y.z = d1 * static_cast<float>((q >> 16) & 0xF) - m1;
        y.w = d1 * static_cast<float>((q >> 24) & 0xF) - m1;
    } else if constexpr (TYPE == TYPE_Q5_K) {
        const uint8_t* b = rp + (e0 / 256) * 176;
        const int wi = static_cast<int>(e0 % 256);
        const int c = wi / 64, l = wi % 32, hi = (wi % 64) / 32;
        const uint32_t hd = ld_b32(b);
        const float d = f16lo(hd), dmin = f16hi(hd);
        float sc, m;
        q4k_scale_min(2 * c + hi, b + 4, sc, m);
        const float d1 = d * sc, m1 = dmin * m;
        const uint32_t q = ld_b32(b + 48 + 32 * c + l) >> (4 * hi);
        const uint32_t h = ld_b32(b + 16 + l) >> (2 * c + hi);  // bit 0 of each byte
        y.x = d1 * static_cast<float>((q & 0xF) | ((h & 1u) << 4)) - m1;
        y.y = d1 * static_cast<float>(((q >> 8) & 0xF) | (((h >> 8) & 1u) << 4)) - m1;
        y.z = d1 * static_cast<float>(((q >> 16) & 0xF) | (((h >> 16) & 1u) << 4)) - m1;
        y.w = d1 * static_cast<float>(((q >> 24) & 0xF) | (((h >> 24) & 1u) << 4)) - m1;
    } else if constexpr (TYPE == TYPE_Q2_K || TYPE == TYPE_Q3_K) {
        const uint8_t* b = rp + (e0 / 256) * block_bytes(TYPE);
        const int wi = static_cast<int>(e0 % 256);
        const int h = wi / 128, j = (wi % 128) / 32, l = wi % 32, s = wi / 16;
        float v[4];
        if constexpr (TYPE == TYPE_Q2_K) {
            const uint32_t q = (ld_u16(b + 16 + 32 * h + l) | (ld_u16(b + 18 + 32 * h + l) << 16)) >> (2 * j);
            const uint32_t sm = b[s];
            const float dd = f16lo(ld_u16(b + 80)), dm = f16lo(ld_u16(b + 82));
            const float d1 = dd * static_cast<float>(sm & 0xF), m1 = dm * static_cast<float>(sm >> 4);
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = d1 * static_cast<float>((q >> (8 * i)) & 3) - m1;
        } else {
            const uint32_t q = (ld_u16(b + 32 + 32 * h + l) | (ld_u16(b + 34 + 32 * h + l) << 16)) >> (2 * j);
            const uint32_t hb = (ld_u16(b + l) | (ld_u16(b + l + 2) << 16)) >> (4 * h + j);
            const uint8_t* sc = b + 96;
            const int lo = s < 8 ? (sc[s] & 0xF) : (sc[s - 8] >> 4);
            const int hi = (sc[8 + s % 4] >> (2 * (s / 4))) & 3;
            const float d1 = f16lo(ld_u16(b + 108)) * static_cast<float>((lo | (hi << 4)) - 32);
#pragma unroll
            for (int i = 0; i < 4; i++)
                v[i] = d1 * static_cast<float>(static_cast<int>((q >> (8 * i)) & 3) + 4 * static_cast<int>((hb >> (8 * i)) & 1) - 4);
        }
        return make_float4(v[0], v[1], v[2], v[3]);
    } else if constexpr (TYPE == TYPE_Q6_K) {
        const uint8_t* b = rp + (e0 / 256) * 210;
        const int wi = static_cast<int>(e0 % 256);
        const int h = wi / 128, r = wi % 128, t = r / 32, l = r % 32;
        const uint8_t* ql = b + 64 * h + l + 32 * (t & 1);
        const uint8_t* qh = b + 128 + 32 * h + l;
        const uint32_t lo = (ld_u16(ql) | (ld_u16(ql + 2) << 16)) >> (4 * (t >> 1));
        const uint32_t hb = (ld_u16(qh) | (ld_u16(qh + 2) << 16)) >> (2 * t);
        const float d = f16lo(ld_u16(b + 208));
        const float ds = d * static_cast<float>(static_cast<int8_t>(b[192 + 8 * h + l / 16 + 2 * t]));
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = static_cast<int>(((lo >> (8 * i)) & 0xF) | (((hb >> (8 * i)) & 3) << 4)) - 32;
            v[i] = ds * static_cast<float>(q);
        }
        y = make_float4(v[0], v[1], v[2], v[3]);
    } else if constexpr (TYPE == TYPE_Q8_0) {
        const uint8_t* b = rp + (e0 / 32) * 34;
        const int i0 = static_cast<int>(e0 % 32);
        const float d = f16lo(ld_u16(b));
        const uint32_t q = ld_u16(b + 2 + i0) | (ld_u16(b + 4 + i0) << 16);
        y.x = static_cast<float>(static_cast<int8_t>(q & 0xff)) * d;
        y.y = static_cast<float>(static_cast<int8_t>((q >> 8) & 0xff)) * d;
        y.z = static_cast<float>(static_cast<int8_t>((q >> 16) & 0xff)) * d;
        y.w = static_cast<float>(static_cast<int8_t>(q >> 24)) * d;
    }
    return y;
}

// One thread decodes 4 consecutive elements (e0 .. e0+3) of one row.
template <int TYPE>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ w,
                                                      float* __restrict__ out, int64_t n_groups,
                                                      int64_t k, int64_t rb) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    const int64_t gpr = k / 4;
    const int64_t row = g / gpr;
    const int64_t e0 = (g - row * gpr) * 4;
    *reinterpret_cast<float4*>(out + row * k + e0) = decode4<TYPE>(w + row * rb, e0);
}

// Row gather: out row t = decoded row ids[t] of w (zeros for ids outside
// [0, n_src)).  Block types: 4 elements per thread; F32 / F16: 1.
template <int TYPE>
__global__ void __launch_bounds__(256) gather_rows_kernel(const uint8_t* __restrict__ w,
                                                          const int32_t* __restrict__ ids, int64_t n_src,
                                                          float* __restrict__ out, int64_t n_items, int64_t k,
                                                          int64_t rb) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= n_items) return;
    constexpr int64_t PER = (TYPE == TYPE_F32 || TYPE == TYPE_F16 || TYPE == TYPE_BF16) ? 1 : 4;
    const int64_t ipr = k / PER;
    const int64_t t = g / ipr;
    const int64_t e0 = (g - t * ipr) * PER;
    const int32_t id = ids[t];
    const bool ok = id >= 0 && id < n_src;
    const uint8_t* rp = w + (ok ? static_cast<int64_t>(id) : 0) * rb;
    if constexpr (PER == 1) {
        float v;
        if constexpr (TYPE == TYPE_F32)
            v = reinterpret_cast<const float*>(rp)[e0];
        else if constexpr (TYPE == TYPE_BF16)
            v = __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(rp)[e0]) << 16);
        else
            v = __half2float(reinterpret_cast<const __half*>(rp)[e0]);
        out[t * k + e0] = ok ? v : 0.f;
    } else {
        const float4 y = decode4<TYPE>(rp, e0);
        *reinterpret_cast<float4*>(out + t * k + e0) = ok ? y : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// F32 / F16: one thread per element (any k).
template <int TYPE>
__global__ void __launch_bounds__(256) dequant_plain_kernel(const uint8_t* __restrict__ w,
                                                            float* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if constexpr (TYPE == TYPE_F32)
        out[i] = reinterpret_cast<const float*>(w)[i];
    else if constexpr (TYPE == TYPE_BF16)
        out[i] = __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(w)[i]) << 16);
    else
        out[i] = __half2float(reinterpret_cast<const __half*>(w)[i]);
}

// The same decode with each value rounded once to fp16 (round to nearest
// even): the weight operand of the batched kernels for the types that have
// no fused decoder (gemm.hip).  Four elements a thread; plain types take
// the fp32 / bf16 value as is before the rounding.
template <int TYPE>
__global__ void __launch_bounds__(256) dequant_f16_kernel(const uint8_t* __restrict__ w, _Float16* __restrict__ out,
                                                          int64_t n_groups, int64_t k, int64_t rb) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    const int64_t gpr = k / 4;
    const int64_t row = g / gpr;
    const int64_t e0 = (g - row * gpr) * 4;
    float4 y;
    if constexpr (TYPE == TYPE_F32) {
        y = *reinterpret_cast<const float4*>(w + row * rb + e0 * 4);
    } else if constexpr (TYPE == TYPE_BF16) {
        const uint2 v = *reinterpret_cast<const uint2*>(w + row * rb + e0 * 2);
        y = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y << 16),
                        __uint_as_float(v.y & 0xFFFF0000u));
    } else {
        y = decode4<TYPE>(w + row * rb, e0);
    }
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 h = {static_cast<_Float16>(y.x), static_cast<_Float16>(y.y), static_cast<_Float16>(y.z),
                  static_cast<_Float16>(y.w)};
    *reinterpret_cast<h4*>(out + row * k + e0) = h;
}

// ---- quantizers (one thread per block) ------------------------------------

__device__ __forceinline__ void st_u16(uint8_t* p, uint16_t v) {
    p[0] = static_cast<uint8_t>(v);
    p[1] = static_cast<uint8_t>(v >> 8);
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

__device__ void quant_q8_0_block(const float* x, uint8_t* b) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    const float d = amax / 127.0f;
    st_u16(b, f32_to_f16_rne(d));
    for (int i = 0; i < 32; i++) {
        const float v = d > 0.f ? roundf(x[i] / d) : 0.f;
        b[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(clampf(v, -127.f, 127.f)));
    }
}

__device__ void quant_q4_k_block(const float* x, uint8_t* b) {
    float scale[8], mneg[8];
    float max_scale = 0.f, max_mneg = 0.f;
    for (int j = 0; j < 8; j++) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int l = 1; l < 32; l++) {
            lo = fminf(lo, x[32 * j + l]);
            hi = fmaxf(hi, x[32 * j + l]);
        }
        lo = fminf(lo, 0.f);
        scale[j] = (hi - lo) / 15.0f;
        mneg[j] = -lo;
        max_scale = fmaxf(max_scale, scale[j]);
        max_mneg = fmaxf(max_mneg, mneg[j]);
    }
    const uint16_t dh = f32_to_f16_rne(max_scale / 63.0f);
    const uint16_t dmh = f32_to_f16_rne(max_mneg / 63.0f);
    const float df = __half2float(__ushort_as_half(dh));
    const float dmf = __half2float(__ushort_as_half(dmh));
    uint8_t sc[8], mm[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = static_cast<uint8_t>(clampf(df > 0.f ? roundf(scale[j] / df) : 0.f, 0.f, 63.f));
        mm[j] = static_cast<uint8_t>(clampf(dmf > 0.f ? roundf(mneg[j] / dmf) : 0.f, 0.f, 63.f));
    }
    st_u16(b, dh);
    st_u16(b + 2, dmh);
    for (int j = 0; j < 4; j++) {
        b[4 + j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        b[8 + j] = static_cast<uint8_t>((mm[j] & 63) | ((mm[j + 4] >> 4) << 6));
        b[12 + j] = static_cast<uint8_t>((sc[j + 4] & 0xF) | ((mm[j + 4] & 0xF) << 4));
    }
    for (int c = 0; c < 4; c++) {
        const float es0 = df * static_cast<float>(sc[2 * c]);
        const float em0 = dmf * static_cast<float>(mm[2 * c]);
        const float es1 = df * static_cast<float>(sc[2 * c + 1]);
        const float em1 = dmf * static_cast<float>(mm[2 * c + 1]);
        for (int l = 0; l < 32; l++) {
            const float v0 = es0 > 0.f ? roundf((x[64 * c + l] + em0) / es0) : 0.f;
            const float v1 = es1 > 0.f ? roundf((x[64 * c + 32 + l] + em1) / es1) : 0.f;
            const uint32_t n0 = static_cast<uint32_t>(clampf(v0, 0.f, 15.f));
            const uint32_t n1 = static_cast<uint32_t>(clampf(v1, 0.f, 15.f));
            b[16 + 32 * c + l] = static_cast<uint8_t>(n0 | (n1 << 4));
        }
    }
}

__device__ void quant_q6_k_block(const float* x, uint8_t* b) {
    float s16[16];
    float max_s = 0.f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.f;
        for (int l = 0; l < 16; l++) amax = fmaxf(amax, fabsf(x[16 * j + l]));
        s16[j] = amax / 31.0f;
        max_s = fmaxf(max_s, s16[j]);
    }
    const uint16_t dh = f32_to_f16_rne(max_s / 127.0f);
    const float df = __half2float(__ushort_as_half(dh));
    for (int i = 0; i < 192; i++) b[i] = 0;
    for (int j = 0; j < 16; j++) {
        const float scv = clampf(df > 0.f ? roundf(s16[j] / df) : 0.f, -128.f, 127.f);
        const int8_t sc = static_cast<int8_t>(scv);
        const int h = j / 8, t = (j % 8) / 2, half = j % 2;
        b[192 + 8 * h + half + 2 * t] = static_cast<uint8_t>(sc);
        const float es = df * static_cast<float>(sc);
        for (int l16 = 0; l16 < 16; l16++) {
            const int e = 16 * j + l16;
            const float v = es > 0.f ? roundf(x[e] / es) : 0.f;
            const uint32_t q = static_cast<uint32_t>(static_cast<int>(clampf(v, -32.f, 31.f)) + 32);
            const int r = e % 128, l = r % 32;
            b[64 * h + l + 32 * (t & 1)] |= static_cast<uint8_t>((q & 0xF) << (4 * (t >> 1)));
            b[128 + 32 * h + l] |= static_cast<uint8_t>((q >> 4) << (2 * t));
        }
    }
    st_u16(b + 208, dh);
}

template <int TYPE>
__global__ void __launch_bounds__(64) quantize_kernel(const float* __restrict__ src,
                                                      uint8_t* __restrict__ w, int64_t n_blocks) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    constexpr int64_t BE = block_elems(TYPE), BB = block_bytes(TYPE);
    const float* x = src + i * BE;
    uint8_t* b = w + i * BB;
    if constexpr (TYPE == TYPE_Q8_0) quant_q8_0_block(x, b);
    else if constexpr (TYPE == TYPE_Q4_K) quant_q4_k_block(x, b);
    else if constexpr (TYPE == TYPE_Q6_K) quant_q6_k_block(x, b);
    else if constexpr (TYPE == TYPE_F32) *reinterpret_cast<float*>(b) = x[0];
    else st_u16(b, f32_to_f16_rne(x[0]));
}

template <int TYPE>
int launch_quantize(const float* src, void* w, int64_t n_blocks, hipStream_t st) {
    const int64_t grid = (n_blocks + 63) / 64;
    quantize_kernel<TYPE><<<dim3(static_cast<uint32_t>(grid)), dim3(64), 0, st>>>(
        src, static_cast<uint8_t*>(w), n_blocks);
    return check_launch("vb_quantize_rows");
}

}  // namespace

// n_rows x k of W (any decodable type but F16) as row-major fp16 at out
// (16-byte aligned, k % 4 == 0); the caller has checked the type and k.
int dequant_rows_f16(const void* w, _Float16* out, int64_t n_rows, int64_t k, int32_t type, hipStream_t st) {
    const int64_t rb = row_bytes(type, k);
    const int64_t n_groups = n_rows * (k / 4);
    const int64_t grid = (n_groups + 255) / 256;
    if (rb < 0 || k % 4 != 0 || grid > 0x7fffffff) {
        set_error("vb_gemm: cannot decode %lld x %lld of type %d to fp16", static_cast<long long>(n_rows),
                  static_cast<long long>(k), type);
        return E_INVAL;
    }
    if (n_rows == 0) return OK;
    const dim3 g(static_cast<uint32_t>(grid)), b(256);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (type) {
    case TYPE_F32: dequant_f16_kernel<TYPE_F32><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_BF16: dequant_f16_kernel<TYPE_BF16><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q4_K: dequant_f16_kernel<TYPE_Q4_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q6_K: dequant_f16_kernel<TYPE_Q6_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q8_0: dequant_f16_kernel<TYPE_Q8_0><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q5_K: dequant_f16_kernel<TYPE_Q5_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q2_K: dequant_f16_kernel<TYPE_Q2_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q3_K: dequant_f16_kernel<TYPE_Q3_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q4_0: dequant_f16_kernel<TYPE_Q4_0><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q4_1: dequant_f16_kernel<TYPE_Q4_1><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q5_0: dequant_f16_kernel<TYPE_Q5_0><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q5_1: dequant_f16_kernel<TYPE_Q5_1><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    default: set_error("vb_gemm: no fp16 decode for type %d", type); return E_UNSUPPORTED;
    }
    return check_launch("vb_gemm");
}

}  // namespace vb

using namespace vb;

extern "C" int vb_dequant_rows(const void* w, float* out, int64_t n_rows, int64_t k,
                               int32_t ggml_type, void* stream) {
    const int64_t rb = row_bytes(ggml_type, k);
    if (rb < 0) {
        set_error("vb_dequant_rows: unsupported type %d or k=%lld not a whole number of blocks",
                  ggml_type, static_cast<long long>(k));
        return E_INVAL;
    }
    if (n_rows < 0 || (n_rows > 0 && (!w || !out))) {
        set_error("vb_dequant_rows: bad arguments (n_rows=%lld)", static_cast<long long>(n_rows));
        return E_INVAL;
    }
    if (n_rows == 0) return OK;
    hipStream_t st = as_stream(stream);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (ggml_type == TYPE_F32 || ggml_type == TYPE_F16 || ggml_type == TYPE_BF16) {
        const int64_t n = n_rows * k;
        const int64_t grid = (n + 255) / 256;
        if (grid > 0x7fffffff) {
            set_error("vb_dequant_rows: tensor too large for one launch");
            return E_INVAL;
        }
        const dim3 g(static_cast<uint32_t>(grid)), b(256);
        if (ggml_type == TYPE_F32)
            dequant_plain_kernel<TYPE_F32><<<g, b, 0, st>>>(wb, out, n);
        else if (ggml_type == TYPE_BF16)
            dequant_plain_kernel<TYPE_BF16><<<g, b, 0, st>>>(wb, out, n);
        else
            dequant_plain_kernel<TYPE_F16><<<g, b, 0, st>>>(wb, out, n);
        return check_launch("vb_dequant_rows");
    }
    const int64_t n_groups = n_rows * (k / 4);
    const int64_t grid = (n_groups + 255) / 256;
    if (grid > 0x7fffffff) {
        set_error("vb_dequant_rows: tensor too large for one launch");
        return E_INVAL;
    }
    const dim3 g(static_cast<uint32_t>(grid)), b(256);
    switch (ggml_type) {
    case TYPE_Q4_K: dequant_kernel<TYPE_Q4_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q6_K: dequant_kernel<TYPE_Q6_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q8_0: dequant_kernel<TYPE_Q8_0><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q5_K: dequant_kernel<TYPE_Q5_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q2_K: dequant_kernel<TYPE_Q2_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q3_K: dequant_kernel<TYPE_Q3_K><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q4_0: dequant_kernel<TYPE_Q4_0><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q4_1: dequant_kernel<TYPE_Q4_1><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q5_0: dequant_kernel<TYPE_Q5_0><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    case TYPE_Q5_1: dequant_kernel<TYPE_Q5_1><<<g, b, 0, st>>>(wb, out, n_groups, k, rb); break;
    default: set_error("vb_dequant_rows: unsupported type %d", ggml_type); return E_UNSUPPORTED;
    }
    return check_launch("vb_dequant_rows");
}

extern "C" int vb_quantize_rows(const float* src, void* w, int64_t n_rows, int64_t k,
                                int32_t ggml_type, void* stream) {
    const int64_t rb = row_bytes(ggml_type, k);
    if (rb < 0) {
        set_error("vb_quantize_rows: unsupported type %d or k=%lld not a whole number of blocks",
                  ggml_type, static_cast<long long>(k));
        return E_INVAL;
    }
    if (n_rows < 0 || (n_rows > 0 && (!w || !src))) {
        set_error("vb_quantize_rows: bad arguments");
        return E_INVAL;
    }
    if (n_rows == 0) return OK;
    const int64_t n_blocks = n_rows * (k / block_elems(ggml_type));
    if ((n_blocks + 63) / 64 > 0x7fffffff) {
        set_error("vb_quantize_rows: tensor too large for one launch");
        return E_INVAL;
    }
    hipStream_t st = as_stream(stream);
    switch (ggml_type) {
    case TYPE_Q8_0: return launch_quantize<TYPE_Q8_0>(src, w, n_blocks, st);
    case TYPE_Q4_K: return launch_quantize<TYPE_Q4_K>(src, w, n_blocks, st);
    case TYPE_Q6_K: return launch_quantize<TYPE_Q6_K>(src, w, n_blocks, st);
    case TYPE_F32: return launch_quantize<TYPE_F32>(src, w, n_blocks, st);
    case TYPE_F16: return launch_quantize<TYPE_F16>(src, w, n_blocks, st);
    default: set_error("vb_quantize_rows: unsupported type %d", ggml_type); return E_UNSUPPORTED;
    }
}

extern "C" int vb_embed_rows(const void* table, int32_t ggml_type, int64_t n_vocab, int64_t k,
                             const int32_t* tokens, int64_t n_tokens, float* out, void* stream) {
    const int64_t rb = row_bytes(ggml_type, k);
    if (rb < 0) {
        set_error("vb_embed_rows: unsupported type %d or k=%lld not a whole number of blocks", ggml_type,
                  static_cast<long long>(k));
        return E_INVAL;
    }
    if (n_tokens < 0 || n_vocab <= 0 || (n_tokens > 0 && (!table || !tokens || !out))) {
        set_error("vb_embed_rows: bad arguments (n_vocab=%lld, n_tokens=%lld)", static_cast<long long>(n_vocab),
                  static_cast<long long>(n_tokens));
        return E_INVAL;
    }
    if (n_tokens == 0) return OK;
    const bool plain = ggml_type == TYPE_F32 || ggml_type == TYPE_F16 || ggml_type == TYPE_BF16;
    if (!plain && reinterpret_cast<uintptr_t>(out) % 16 != 0) {
        set_error("vb_embed_rows: out must be 16-byte aligned for block types");
        return E_INVAL;
    }
    const int64_t n_items = n_tokens * (plain ? k : k / 4);
    const int64_t grid = (n_items + 255) / 256;
    if (grid > 0x7fffffff) {
        set_error("vb_embed_rows: too many rows for one launch");
        return E_INVAL;
    }
    hipStream_t st = as_stream(stream);
    const uint8_t* wb = static_cast<const uint8_t*>(table);
    const dim3 g(static_cast<uint32_t>(grid)), b(256);
    switch (ggml_type) {
    case TYPE_Q4_K: gather_rows_kernel<TYPE_Q4_K><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q6_K: gather_rows_kernel<TYPE_Q6_K><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q8_0: gather_rows_kernel<TYPE_Q8_0><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_F32: gather_rows_kernel<TYPE_F32><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_F16: gather_rows_kernel<TYPE_F16><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_BF16: gather_rows_kernel<TYPE_BF16><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q5_K: gather_rows_kernel<TYPE_Q5_K><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q2_K: gather_rows_kernel<TYPE_Q2_K><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q3_K: gather_rows_kernel<TYPE_Q3_K><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q4_0: gather_rows_kernel<TYPE_Q4_0><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q4_1: gather_rows_kernel<TYPE_Q4_1><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q5_0: gather_rows_kernel<TYPE_Q5_0><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    case TYPE_Q5_1: gather_rows_kernel<TYPE_Q5_1><<<g, b, 0, st>>>(wb, tokens, n_vocab, out, n_items, k, rb); break;
    default: set_error("vb_embed_rows: unsupported type %d", ggml_type); return E_UNSUPPORTED;
    }
    return check_launch("vb_embed_rows");
}
