/*
 * CPU oracle for the GGUF quantized-matmul path.  TEST INFRASTRUCTURE ONLY:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library; the product (vibeblade_amd) never does.
 *
 * Plain C restatement of the reference algorithms:
 *   - fp16 -> fp32 exactly as cpp/src/fp16_compat.cpp:13-35
 *   - Q4_K decode as cpp/src/dequant.cpp:258-301 (get_scale_min_k4 + decode),
 *     which is the GGUF (ggml) standard layout
 *   - Q8_0 decode with the GGUF layout: fp16 d at bytes 0-1, int8 qs at 2-33,
 *     as vibeblade/loader.py:129-133 and cpp/src/cuda_kernels.cu:718-735
 *     (cpp/src/dequant.cpp:99-112 reads a 4-byte float there instead; that
 *     variant is ORC_TYPE_Q8_0_VBREF below, kept for timing parity only)
 *   - Q6_K decode with the GGUF standard gather; the literal reference gather
 *     of cpp/src/dequant.cpp:359-402 is ORC_TYPE_Q6_K_VBREF
 *   - gemv_kn: the reference's gemv_dequant loop (cpp/src/dequant.cpp:739-780):
 *     W stored as K rows of N elements, out = x . W, per-row decode into a
 *     scratch row then saxpy.  Single threaded like gemv_dequant_mt
 *     (cpp/src/dequant.cpp:783-792).  This is the CPU timing baseline.
 *   - gemv / gemm in the GGUF orientation y[n] = sum_k W[n,k] x[k]
 *     (rows = outputs, blocks along K), accumulated in double.
 *   - quantizers for Q8_0 / Q4_K / Q6_K.  The reference has none; these are
 *     deterministic and only need to produce valid blocks.
 *   - Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q5_K / BF16 decode with the GGUF layouts.
 *     The reference's own decoders for the 32-element types
 *     (cpp/src/dequant.cpp:23-94) interleave the nibbles (element 2j = low
 *     nibble of byte j), and its Q5_K (:307-353) reads qh bits 7 / 3 and
 *     advances qh by 32 bytes per 64-element group, past the 32 bytes of qh.
 *     GGUF files hold elements 0..15 in the low nibbles and 16..31 in the
 *     high nibbles of qs[0..15], and Q5_K group g takes bits 2g / 2g+1 of
 *     qh[l]; these decoders follow the files.
 *   - Q2_K / Q3_K decode with the GGUF layouts.  The reference's decoders
 *     (cpp/src/dequant.cpp:128-149, :157-219) take other code bytes, add dmin
 *     instead of subtracting dmin * min (Q2_K), and unpack the Q3_K scales and
 *     hmask bits differently.  GGUF: element e = 128 h + 32 j + l takes bits
 *     2j, 2j+1 of qs[32 h + l] and the scale of sub-block e / 16; Q3_K adds
 *     bit 4h + j of hmask[l] as the code's third bit (clear: minus 4), with
 *     6-bit scales (low 4 bits: byte i or the high nibble of byte i - 8;
 *     high 2 bits: bits 2 (i / 4) of byte 8 + i % 4) minus 32.
 *
 * Parity pins (tests/test_oracle.py): Q4_K and Q6_K_VBREF against golden
 * vectors produced by the compiled reference dequant.cpp; Q6_K against the
 * layout-invariant known answers of tests/test_kquants.py:134-175 plus
 * single-position index-map blocks; Q8_0 against closed forms (d=1 gives q,
 * d=0 gives 0) and loader.py semantics; Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q5_K /
 * Q2_K / Q3_K against ggml's published dequantize_row_* loop forms on random
 * blocks; gemv against brute force on blocks whose decoded values are known
 * integers.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum {
    ORC_TYPE_F32 = 0,
    ORC_TYPE_F16 = 1,
    ORC_TYPE_Q4_0 = 2,
    ORC_TYPE_Q4_1 = 3,
    ORC_TYPE_Q5_0 = 6,
    ORC_TYPE_Q5_1 = 7,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q2_K = 10,
    ORC_TYPE_Q3_K = 11,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q5_K = 13,
    ORC_TYPE_Q6_K = 14,
    ORC_TYPE_BF16 = 30,
    /* test-only: the reference's own (non-GGUF) gathers */
    ORC_TYPE_Q6_K_VBREF = 1014,
    ORC_TYPE_Q8_0_VBREF = 1008,
};

int64_t orc_block_elems(int type) {
    switch (type) {
    case ORC_TYPE_F32: case ORC_TYPE_F16: case ORC_TYPE_BF16: return 1;
    case ORC_TYPE_Q8_0: case ORC_TYPE_Q8_0_VBREF: case ORC_TYPE_Q4_0: case ORC_TYPE_Q4_1:
    case ORC_TYPE_Q5_0: case ORC_TYPE_Q5_1: return 32;
    case ORC_TYPE_Q2_K: case ORC_TYPE_Q3_K:
    case ORC_TYPE_Q4_K: case ORC_TYPE_Q5_K: case ORC_TYPE_Q6_K: case ORC_TYPE_Q6_K_VBREF: return 256;
    default: return -1;
    }
}

int64_t orc_block_bytes(int type) {
    switch (type) {
    case ORC_TYPE_F32: return 4;
    case ORC_TYPE_F16: case ORC_TYPE_BF16: return 2;
    case ORC_TYPE_Q4_0: return 18;
    case ORC_TYPE_Q4_1: return 20;
    case ORC_TYPE_Q5_0: return 22;
    case ORC_TYPE_Q5_1: return 24;
    case ORC_TYPE_Q8_0: case ORC_TYPE_Q8_0_VBREF: return 34;
    case ORC_TYPE_Q2_K: return 84;
    case ORC_TYPE_Q3_K: return 110;
    case ORC_TYPE_Q4_K: return 144;
    case ORC_TYPE_Q5_K: return 176;
    case ORC_TYPE_Q6_K: case ORC_TYPE_Q6_K_VBREF: return 210;
    default: return -1;
    }
}

int64_t orc_row_bytes(int type, int64_t k) {
    int64_t be = orc_block_elems(type), bb = orc_block_bytes(type);
    if (be <= 0 || k % be != 0) return -1;
    return (k / be) * bb;
}

/* fp16 -> fp32, exact including subnormals, inf and NaN
 * (cpp/src/fp16_compat.cpp:13-35). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t ex = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign << 31;
        } else {
            /* normalise the subnormal: value = man * 2^-24 */
            int e = -14;
            while (!(man & 0x400u)) { man <<= 1; e--; }
            man &= 0x3ffu;
            bits = (sign << 31) | ((uint32_t)(e + 127) << 23) | (man << 13);
        }
    } else if (ex == 31) {
        bits = (sign << 31) | 0x7f800000u | (man << 13);
    } else {
        bits = (sign << 31) | ((ex - 15u + 127u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* fp32 -> fp16 with round-to-nearest-even (used by the quantizers only). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* result is subnormal (or zero) in fp16 */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        int shift = (int)(126 - e); /* value = m * 2^(e-150); want units of 2^-24 */
        /* units of 2^-24: m * 2^(e-150+24) = m >> (126-e) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void wr_u16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* 6-bit scale/min of sub-block j (cpp/src/dequant.cpp:258-266). */
void orc_q4k_scale_min(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* ---- single-block decoders ------------------------------------------- */

static void dec_q8_0(const uint8_t* b, float* y) {
    float d = orc_f16_to_f32(rd_u16(b));
    const int8_t* q = (const int8_t*)(b + 2);
    for (int i = 0; i < 32; i++) y[i] = (float)q[i] * d;
}

static void dec_q8_0_vbref(const uint8_t* b, float* y) {
    /* cpp/src/dequant.cpp:99-112: 4-byte float at [0,4), qs at [4,36) */
    float d;
    memcpy(&d, b, 4);
    const int8_t* q = (const int8_t*)(b + 4);
    for (int i = 0; i < 32; i++) y[i] = (float)q[i] * d;
}

static void dec_q4_k(const uint8_t* b, float* y) {
    float d = orc_f16_to_f32(rd_u16(b));
    float dmin = orc_f16_to_f32(rd_u16(b + 2));
    const uint8_t* sc = b + 4;
    const uint8_t* qs = b + 16;
    for (int c = 0; c < 4; c++) {
        uint8_t s0, m0, s1, m1;
        orc_q4k_scale_min(2 * c, sc, &s0, &m0);
        orc_q4k_scale_min(2 * c + 1, sc, &s1, &m1);
        float d0 = d * (float)s0, mm0 = dmin * (float)m0;
        float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            y[64 * c + l] = d0 * (float)(qs[32 * c + l] & 0xF) - mm0;
            y[64 * c + 32 + l] = d1 * (float)(qs[32 * c + l] >> 4) - mm1;
        }
    }
}

/* 32-element GGUF blocks: element j (j < 16) = low nibble of qs[j], element
 * j + 16 = high nibble; the fifth bit of element e is bit e of qh (LE). */
static void dec_q4_0(const uint8_t* b, float* y) {
    float d = orc_f16_to_f32(rd_u16(b));
    const uint8_t* qs = b + 2;
    for (int j = 0; j < 16; j++) {
        y[j] = (float)((qs[j] & 0xF) - 8) * d;
        y[j + 16] = (float)((qs[j] >> 4) - 8) * d;
    }
}

static void dec_q4_1(const uint8_t* b, float* y) {
    float d = orc_f16_to_f32(rd_u16(b)), m = orc_f16_to_f32(rd_u16(b + 2));
    const uint8_t* qs = b + 4;
    for (int j = 0; j < 16; j++) {
        y[j] = d * (float)(qs[j] & 0xF) + m;
        y[j + 16] = d * (float)(qs[j] >> 4) + m;
    }
}

static uint32_t rd_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

static void dec_q5_0(const uint8_t* b, float* y) {
    float d = orc_f16_to_f32(rd_u16(b));
    uint32_t qh = rd_u32(b + 2);
    const uint8_t* qs = b + 6;
    for (int j = 0; j < 16; j++) {
        int q0 = (qs[j] & 0xF) | (int)(((qh >> j) & 1) << 4);
        int q1 = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
        y[j] = (float)(q0 - 16) * d;
        y[j + 16] = (float)(q1 - 16) * d;
    }
}

static void dec_q5_1(const uint8_t* b, float* y) {
    float d = orc_f16_to_f32(rd_u16(b)), m = orc_f16_to_f32(rd_u16(b + 2));
    uint32_t qh = rd_u32(b + 4);
    const uint8_t* qs = b + 8;
    for (int j = 0; j < 16; j++) {
        int q0 = (qs[j] & 0xF) | (int)(((qh >> j) & 1) << 4);
        int q1 = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
        y[j] = d * (float)q0 + m;
        y[j + 16] = d * (float)q1 + m;
    }
}

/* Q5_K: Q4_K's header and scale packing, qh[32] at 16, qs[128] at 48; group
 * c (elements 64c .. 64c + 63) adds bit 2c (low nibbles) / 2c+1 (high) of
 * qh[l] as the fifth bit. */
static void dec_q5_k(const uint8_t* b, float* y) {
    float d = orc_f16_to_f32(rd_u16(b));
    float dmin = orc_f16_to_f32(rd_u16(b + 2));
    const uint8_t* sc = b + 4;
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int c = 0; c < 4; c++) {
        uint8_t s0, m0, s1, m1;
        orc_q4k_scale_min(2 * c, sc, &s0, &m0);
        orc_q4k_scale_min(2 * c + 1, sc, &s1, &m1);
        float d0 = d * (float)s0, mm0 = dmin * (float)m0;
        float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            int q0 = (qs[32 * c + l] & 0xF) | (((qh[l] >> (2 * c)) & 1) << 4);
            int q1 = (qs[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4);
            y[64 * c + l] = d0 * (float)q0 - mm0;
            y[64 * c + 32 + l] = d1 * (float)q1 - mm1;
        }
    }
}

/* Q2_K: scales[16] at 0 (low nibble scale, high nibble min, per 16
 * elements), qs[64] at 16, d at 80, dmin at 82. */
static void dec_q2_k(const uint8_t* b, float* y) {
    const uint8_t* sc = b;
    const uint8_t* qs = b + 16;
    float d = orc_f16_to_f32(rd_u16(b + 80)), dmin = orc_f16_to_f32(rd_u16(b + 82));
    for (int e = 0; e < 256; e++) {
        int h = e / 128, j = (e % 128) / 32, l = e % 32;
        int q = (qs[32 * h + l] >> (2 * j)) & 3;
        uint8_t s = sc[e / 16];
        y[e] = d * (float)(s & 0xF) * (float)q - dmin * (float)(s >> 4);
    }
}

/* Q3_K: hmask[32] at 0, qs[64] at 32, scales[12] at 96, d at 108. */
static int q3k_scale(const uint8_t* sc, int i) {
    int lo = i < 8 ? (sc[i] & 0xF) : (sc[i - 8] >> 4);
    int hi = (sc[8 + i % 4] >> (2 * (i / 4))) & 3;
    return (lo | (hi << 4)) - 32;
}

static void dec_q3_k(const uint8_t* b, float* y) {
    const uint8_t* hm = b;
    const uint8_t* qs = b + 32;
    const uint8_t* sc = b + 96;
    float d = orc_f16_to_f32(rd_u16(b + 108));
    for (int e = 0; e < 256; e++) {
        int h = e / 128, j = (e % 128) / 32, l = e % 32;
        int q = ((qs[32 * h + l] >> (2 * j)) & 3) - (((hm[l] >> (4 * h + j)) & 1) ? 0 : 4);
        y[e] = d * (float)q3k_scale(sc, e / 16) * (float)q;
    }
}

static void dec_q6_k(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    float d = orc_f16_to_f32(rd_u16(b + 208));
    for (int e = 0; e < 256; e++) {
        int h = e / 128, r = e % 128, t = r / 32, l = r % 32;
        int lo = (ql[64 * h + l + 32 * (t & 1)] >> (4 * (t >> 1))) & 0xF;
        int hi = (qh[32 * h + l] >> (2 * t)) & 3;
        int q = (lo | (hi << 4)) - 32;
        y[e] = d * (float)sc[8 * h + l / 16 + 2 * t] * (float)q;
    }
}

static void dec_q6_k_vbref(const uint8_t* b, float* y) {
    /* cpp/src/dequant.cpp:379-400: sequential nibbles, LSB-first qh pairs */
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    float d = orc_f16_to_f32(rd_u16(b + 208));
    for (int e = 0; e < 256; e++) {
        int lo = (ql[e / 2] >> (4 * (e & 1))) & 0xF;
        int hi = (qh[e / 4] >> (2 * (e & 3))) & 3;
        int q = (lo | (hi << 4)) - 32;
        y[e] = d * (float)sc[e / 16] * (float)q;
    }
}

/* Decode one row of k elements.  Returns 0 or -1 (bad type / k). */
int orc_dequant_row(const void* row, float* out, int64_t k, int type) {
    const uint8_t* p = (const uint8_t*)row;
    int64_t be = orc_block_elems(type), bb = orc_block_bytes(type);
    if (be <= 0 || k % be != 0) return -1;
    int64_t nb = k / be;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t* b = p + i * bb;
        float* y = out + i * be;
        switch (type) {
        case ORC_TYPE_F32: memcpy(y, b, 4); break;
        case ORC_TYPE_F16: y[0] = orc_f16_to_f32(rd_u16(b)); break;
        case ORC_TYPE_BF16: {
            uint32_t u = (uint32_t)rd_u16(b) << 16;
            memcpy(y, &u, 4);
            break;
        }
        case ORC_TYPE_Q4_0: dec_q4_0(b, y); break;
        case ORC_TYPE_Q4_1: dec_q4_1(b, y); break;
        case ORC_TYPE_Q5_0: dec_q5_0(b, y); break;
        case ORC_TYPE_Q5_1: dec_q5_1(b, y); break;
        case ORC_TYPE_Q5_K: dec_q5_k(b, y); break;
        case ORC_TYPE_Q2_K: dec_q2_k(b, y); break;
        case ORC_TYPE_Q3_K: dec_q3_k(b, y); break;
        case ORC_TYPE_Q8_0: dec_q8_0(b, y); break;
        case ORC_TYPE_Q8_0_VBREF: dec_q8_0_vbref(b, y); break;
        case ORC_TYPE_Q4_K: dec_q4_k(b, y); break;
        case ORC_TYPE_Q6_K: dec_q6_k(b, y); break;
        case ORC_TYPE_Q6_K_VBREF: dec_q6_k_vbref(b, y); break;
        default: return -1;
        }
    }
    return 0;
}

int orc_dequant_rows(const void* w, float* out, int64_t n_rows, int64_t k, int type) {
    int64_t rb = orc_row_bytes(type, k);
    if (rb < 0) return -1;
    for (int64_t r = 0; r < n_rows; r++)
        if (orc_dequant_row((const uint8_t*)w + r * rb, out + r * k, k, type)) return -1;
    return 0;
}

/* ---- quantizers -------------------------------------------------------- */

static float rnd(float v) { return roundf(v); } /* ties away from zero */

static void quant_q8_0(const float* x, uint8_t* b) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
    float d = amax / 127.0f;
    wr_u16(b, orc_f32_to_f16(d));
    int8_t* q = (int8_t*)(b + 2);
    for (int i = 0; i < 32; i++) {
        float v = d > 0.f ? rnd(x[i] / d) : 0.f;
        if (v > 127.f) v = 127.f;
        if (v < -127.f) v = -127.f;
        q[i] = (int8_t)v;
    }
}

static void quant_q4_k(const float* x, uint8_t* b) {
    float scale[8], mneg[8];
    float max_scale = 0.f, max_mneg = 0.f;
    for (int j = 0; j < 8; j++) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int l = 1; l < 32; l++) {
            float v = x[32 * j + l];
            if (v < lo) lo = v;
            if (v > hi) hi = v;
        }
        if (lo > 0.f) lo = 0.f;
        scale[j] = (hi - lo) / 15.0f;
        mneg[j] = -lo;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (mneg[j] > max_mneg) max_mneg = mneg[j];
    }
    float d = max_scale / 63.0f, dmin = max_mneg / 63.0f;
    uint16_t dh = orc_f32_to_f16(d), dmh = orc_f32_to_f16(dmin);
    float df = orc_f16_to_f32(dh), dmf = orc_f16_to_f32(dmh);
    uint8_t sc[8], mm[8];
    for (int j = 0; j < 8; j++) {
        float s = df > 0.f ? rnd(scale[j] / df) : 0.f;
        float m = dmf > 0.f ? rnd(mneg[j] / dmf) : 0.f;
        sc[j] = (uint8_t)(s > 63.f ? 63.f : (s < 0.f ? 0.f : s));
        mm[j] = (uint8_t)(m > 63.f ? 63.f : (m < 0.f ? 0.f : m));
    }
    wr_u16(b, dh);
    wr_u16(b + 2, dmh);
    uint8_t* s = b + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mm[j] & 63) | ((mm[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mm[j + 4] & 0xF) << 4));
    }
    uint8_t* qs = b + 16;
    uint8_t nib[256];
    for (int j = 0; j < 8; j++) {
        float es = df * (float)sc[j];
        float em = dmf * (float)mm[j];
        for (int l = 0; l < 32; l++) {
            float v = es > 0.f ? rnd((x[32 * j + l] + em) / es) : 0.f;
            if (v > 15.f) v = 15.f;
            if (v < 0.f) v = 0.f;
            nib[32 * j + l] = (uint8_t)v;
        }
    }
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++)
            qs[32 * c + l] = (uint8_t)(nib[64 * c + l] | (nib[64 * c + 32 + l] << 4));
}

static void quant_q6_k(const float* x, uint8_t* b) {
    float s16[16];
    float max_s = 0.f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.f;
        for (int l = 0; l < 16; l++) { float a = fabsf(x[16 * j + l]); if (a > amax) amax = a; }
        s16[j] = amax / 31.0f;
        if (s16[j] > max_s) max_s = s16[j];
    }
    float d = max_s / 127.0f;
    uint16_t dh = orc_f32_to_f16(d);
    float df = orc_f16_to_f32(dh);
    int8_t sc[16];
    for (int j = 0; j < 16; j++) {
        float v = df > 0.f ? rnd(s16[j] / df) : 0.f;
        if (v > 127.f) v = 127.f;
        sc[j] = (int8_t)v;
    }
    uint8_t q6[256];
    for (int j = 0; j < 16; j++) {
        float es = df * (float)sc[j];
        for (int l = 0; l < 16; l++) {
            float v = es > 0.f ? rnd(x[16 * j + l] / es) : 0.f;
            if (v > 31.f) v = 31.f;
            if (v < -32.f) v = -32.f;
            q6[16 * j + l] = (uint8_t)((int)v + 32);
        }
    }
    memset(b, 0, 210);
    uint8_t* ql = b;
    uint8_t* qh = b + 128;
    /* GGUF standard layout, inverse of dec_q6_k */
    for (int e = 0; e < 256; e++) {
        int h = e / 128, r = e % 128, t = r / 32, l = r % 32;
        ql[64 * h + l + 32 * (t & 1)] |= (uint8_t)((q6[e] & 0xF) << (4 * (t >> 1)));
        qh[32 * h + l] |= (uint8_t)((q6[e] >> 4) << (2 * t));
    }
    /* scales: element e uses scales[8h + l/16 + 2t]; sub-block j = e/16 maps
     * to that index (h = j/8, t = (j%8)/2, l/16 = j%2). */
    for (int j = 0; j < 16; j++) {
        int h = j / 8, t = (j % 8) / 2, half = j % 2;
        ((int8_t*)(b + 192))[8 * h + half + 2 * t] = sc[j];
    }
    wr_u16(b + 208, dh);
}

int orc_quantize_rows(const float* src, void* dst, int64_t n_rows, int64_t k, int type) {
    int64_t be = orc_block_elems(type), bb = orc_block_bytes(type);
    if (be <= 0 || k % be != 0) return -1;
    if (type != ORC_TYPE_Q8_0 && type != ORC_TYPE_Q4_K && type != ORC_TYPE_Q6_K &&
        type != ORC_TYPE_F32 && type != ORC_TYPE_F16)
        return -1;
    int64_t nb = k / be;
    uint8_t* out = (uint8_t*)dst;
    for (int64_t r = 0; r < n_rows; r++) {
        for (int64_t i = 0; i < nb; i++) {
            const float* x = src + r * k + i * be;
            uint8_t* b = out + (r * nb + i) * bb;
            switch (type) {
            case ORC_TYPE_F32: memcpy(b, x, 4); break;
            case ORC_TYPE_F16: wr_u16(b, orc_f32_to_f16(x[0])); break;
            case ORC_TYPE_Q8_0: quant_q8_0(x, b); break;
            case ORC_TYPE_Q4_K: quant_q4_k(x, b); break;
            case ORC_TYPE_Q6_K: quant_q6_k(x, b); break;
            }
        }
    }
    return 0;
}

/* ---- matrix products in the GGUF orientation ---------------------------- */

/* y[n] = sum_k W[n,k] x[k], W = n rows of k elements; double accumulation. */
int orc_gemv(const void* w, const float* x, float* y, int64_t n, int64_t k, int type) {
    int64_t rb = orc_row_bytes(type, k);
    if (rb < 0) return -1;
    float* row = (float*)malloc((size_t)k * sizeof(float));
    if (!row) return -1;
    for (int64_t r = 0; r < n; r++) {
        orc_dequant_row((const uint8_t*)w + r * rb, row, k, type);
        double acc = 0.0;
        for (int64_t i = 0; i < k; i++) acc += (double)row[i] * (double)x[i];
        y[r] = (float)acc;
    }
    free(row);
    return 0;
}

/* Y[m, n] = sum_k X[m,k] W[n,k]; X fp32 row-major (m x k). */
int orc_gemm(const void* w, const float* x, float* y, int64_t m, int64_t n, int64_t k, int type) {
    int64_t rb = orc_row_bytes(type, k);
    if (rb < 0) return -1;
    float* row = (float*)malloc((size_t)k * sizeof(float));
    if (!row) return -1;
    for (int64_t r = 0; r < n; r++) {
        orc_dequant_row((const uint8_t*)w + r * rb, row, k, type);
        for (int64_t t = 0; t < m; t++) {
            const float* xt = x + t * k;
            double acc = 0.0;
            for (int64_t i = 0; i < k; i++) acc += (double)row[i] * (double)xt[i];
            y[t * n + r] = (float)acc;
        }
    }
    free(row);
    return 0;
}

/* ---- the reference's CPU GEMV loop, restated (timing baseline) ---------- */

/* out[n] = sum_k x[k] W[k][n]; W = K rows of N elements (blocks along N).
 * Same loop as cpp/src/dequant.cpp:767-779: zero out, then for each of the K
 * rows decode it into scratch (N floats) and saxpy with x[k]. */
int orc_gemv_kn(const float* x, const void* w, float* out, int64_t K, int64_t N, int type,
                float* scratch) {
    int64_t rb = orc_row_bytes(type, N);
    if (rb < 0) return -1;
    for (int64_t i = 0; i < N; i++) out[i] = 0.0f;
    const uint8_t* p = (const uint8_t*)w;
    for (int64_t kk = 0; kk < K; kk++) {
        orc_dequant_row(p + kk * rb, scratch, N, type);
        float xk = x[kk];
        for (int64_t i = 0; i < N; i++) out[i] += xk * scratch[i];
    }
    return 0;
}
