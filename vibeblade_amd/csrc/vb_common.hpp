// Shared definitions for the gfx950 GGUF quantized-matmul library (libvbhip).
//
// GGUF block geometry follows cpp/include/ggml_types.h:11-71 (type ids,
// elements and bytes per block) with the on-disk layouts of the GGUF standard:
//   Q8_0  34 B / 32 elem : fp16 d, int8 qs[32]
//   Q4_K 144 B / 256 elem: fp16 d, fp16 dmin, u8 scales[12], u8 qs[128]
//   Q6_K 210 B / 256 elem: u8 ql[128], u8 qh[64], i8 scales[16], fp16 d
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>
#include <cstdio>
#include <string>

namespace vb {

enum : int32_t {
    TYPE_F32 = 0,
    TYPE_F16 = 1,
    TYPE_Q4_0 = 2,
    TYPE_Q4_1 = 3,
    TYPE_Q5_0 = 6,
    TYPE_Q5_1 = 7,
    TYPE_Q8_0 = 8,
    TYPE_Q2_K = 10,
    TYPE_Q3_K = 11,
    TYPE_Q4_K = 12,
    TYPE_Q5_K = 13,
    TYPE_Q6_K = 14,
    TYPE_BF16 = 30,
};

enum : int32_t {
    OK = 0,
    E_INVAL = -1,        // bad argument (shape, null pointer, bad enum)
    E_UNSUPPORTED = -2,  // type / variant not implemented
    E_HIP = -3,          // HIP runtime error
    E_NOMEM = -4,        // workspace too small
};

__host__ __device__ constexpr int64_t block_elems(int32_t t) {
    return t == TYPE_F32 || t == TYPE_F16 || t == TYPE_BF16 ? 1
         : (t == TYPE_Q8_0 || t == TYPE_Q4_0 || t == TYPE_Q4_1 || t == TYPE_Q5_0 || t == TYPE_Q5_1) ? 32
         : (t == TYPE_Q2_K || t == TYPE_Q3_K || t == TYPE_Q4_K || t == TYPE_Q5_K || t == TYPE_Q6_K) ? 256 : -1;
}

__host__ __device__ constexpr int64_t block_bytes(int32_t t) {
    return t == TYPE_F32 ? 4 : (t == TYPE_F16 || t == TYPE_BF16) ? 2 : t == TYPE_Q4_0 ? 18 : t == TYPE_Q4_1 ? 20
         : t == TYPE_Q5_0 ? 22 : t == TYPE_Q5_1 ? 24 : t == TYPE_Q8_0 ? 34 : t == TYPE_Q2_K ? 84
         : t == TYPE_Q3_K ? 110 : t == TYPE_Q4_K ? 144
         : t == TYPE_Q5_K ? 176 : t == TYPE_Q6_K ? 210 : -1;
}

// Block-quantized types with dequant-fused GEMV kernels (gemv.hip).
__host__ __device__ constexpr bool is_block_type(int32_t t) {
    return t == TYPE_Q4_0 || t == TYPE_Q4_1 || t == TYPE_Q5_0 || t == TYPE_Q5_1 || t == TYPE_Q8_0 ||
           t == TYPE_Q2_K || t == TYPE_Q3_K || t == TYPE_Q4_K || t == TYPE_Q5_K || t == TYPE_Q6_K;
}

// Bytes of one row of k elements; -1 when the type is unknown or k is not a
// whole number of blocks.
inline int64_t row_bytes(int32_t t, int64_t k) {
    const int64_t be = block_elems(t), bb = block_bytes(t);
    if (be <= 0 || k <= 0 || k % be != 0) return -1;
    return (k / be) * bb;
}

// Thread-local error text behind vb_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const char* last_error();

// Returns E_HIP (with the message recorded) when the previous launch failed.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- device helpers ------------------------------------------------------

// Exact fp16 -> fp32 (v_cvt_f32_f16 is exact for every input, subnormals
// included).
__device__ __forceinline__ float f16lo(uint32_t w) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(w & 0xffffu)));
}
__device__ __forceinline__ float f16hi(uint32_t w) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(w >> 16)));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Buffer loads: a wave-uniform resource (base, size) plus a 32-bit per-lane
// offset and a uniform offset; no 64-bit address arithmetic per lane.
// Resource word 3 = 0x00020000 (raw untyped access on gfx9).  A load that
// reaches past the resource's size reads zeros; callers keep every load
// inside the tensor anyway.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}

__device__ __forceinline__ u32x4 buf_ld128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// 16 bytes from a 4-byte-aligned address (one global_load_dwordx4).
__device__ __forceinline__ uint4 ld_b128_a4(const uint8_t* p) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t ld_b32(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}

// 16 bytes from a 2-byte-aligned address p.  Reads the dwords covering
// [p & ~3, (p & ~3) + 20): the caller guarantees that window is in bounds.
__device__ __forceinline__ uint4 ld_b128_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t* q = reinterpret_cast<const uint8_t*>(a & ~uintptr_t(3));
    const uint32_t sh = static_cast<uint32_t>(a & 3u);
    const uint4 w = ld_b128_a4(q);
    const uint32_t w4 = ld_b32(q + 16);
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(w.y, w.x, sh);
    r.y = __builtin_amdgcn_alignbyte(w.z, w.y, sh);
    r.z = __builtin_amdgcn_alignbyte(w.w, w.z, sh);
    r.w = __builtin_amdgcn_alignbyte(w4, w.w, sh);
    return r;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// old = 0 (the identity of the add that follows) lets the compiler fold the
// move into v_add_f32_dpp.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// v from the DPP source lane in the rows of ROW_MASK, 0 in the other rows.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_rows_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes of a wave; the result is wave-uniform.  Quad
// butterflies and half-row / row mirrors give every lane its 16-lane row's
// sum; row_bcast:15 then adds row 0 into row 1 and row 2 into row 3, and
// row_bcast:31 adds lane 31 (rows 0 + 1) into rows 2 and 3, so lane 63 holds
// the total (DPP only, no LDS traffic).
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    v += dpp_rows_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
    v += dpp_rows_f<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Size of an active set: `bound` (known to the host), or the count the
// device wrote at *n_dev clamped to [0, bound].
__device__ __forceinline__ int active_count(int bound, const int32_t* n_dev) {
    if (!n_dev) return bound;
    const int c = *n_dev;
    return c < 0 ? 0 : (c > bound ? bound : c);
}

// Gated activations of an FFN neuron, act(g, u) with g = gate row . x and
// u = up row . x:
//   ACT_SILU       silu(g) * u = g / (1 + e^-g) * u
//                  (cpp/src/fast_model.cpp:75, :952; vibeblade/sparse.py:269-272)
//   ACT_RELU2      relu(g) * relu(u) (dReLU, ReLU after both projections)
//   ACT_GELU_TANH  gelu_tanh(g) * u, gelu_tanh(g) = 0.5 g (1 + tanh(z)),
//                  z = 0.7978845608 (g + 0.044715 g^3) (fast_model.cpp:944-948),
//                  evaluated as g / (1 + e^(-2z)), the same function.
constexpr int ACT_SILU = 0;
constexpr int ACT_RELU2 = 1;
constexpr int ACT_GELU_TANH = 2;

__device__ __forceinline__ float act_pair(float g, float u, int kind) {
    if (kind == ACT_SILU) return g / (1.0f + __expf(-g)) * u;
    if (kind == ACT_GELU_TANH) {
        const float z = 0.7978845608f * (g + 0.044715f * g * g * g);
        return g / (1.0f + __expf(-2.0f * z)) * u;
    }
    return fmaxf(g, 0.f) * fmaxf(u, 0.f);
}

// One expert's routed slots from the MoE routing lists: elist[eoff[e] ..
// eoff[e + 1]) with every slot in [0, nslots).  The prep kernel writes the
// lists; the clamps (range inside elist[0, nslots), slot values inside
// [0, nslots)) keep the expert kernels' plain loads and stores inside their
// buffers even if that memory was overwritten by a race with another stream.
struct SlotRange {
    const int32_t* list;
    int count;
    int nslots;
    __device__ __forceinline__ int operator[](int r) const {
        const int q = list[r];
        return static_cast<unsigned>(q) < static_cast<unsigned>(nslots) ? q : 0;
    }
};

__device__ __forceinline__ SlotRange expert_slots(const int32_t* __restrict__ eoff,
                                                  const int32_t* __restrict__ elist, int e, int nslots) {
    int64_t b = eoff[e];
    int64_t c = static_cast<int64_t>(eoff[e + 1]) - b;
    b = b < 0 ? 0 : (b > nslots ? nslots : b);
    c = c > nslots - b ? nslots - b : c;
    return SlotRange{elist + b, c < 0 ? 0 : static_cast<int>(c), nslots};
}

}  // namespace vb
