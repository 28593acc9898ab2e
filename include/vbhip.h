/*
 * libvbhip -- gfx950 (MI355X) GGUF quantized matmul: the C ABI.
 *
 * Every function returns an int status (0 = VB_OK, negative = error) unless
 * stated otherwise; vb_last_error() returns the thread-local text of the last
 * failure.  No C++ exception crosses this boundary.  All pointers passed to
 * the op functions are device pointers; `stream` is a hipStream_t (NULL =
 * the default stream).  Launches are asynchronous on `stream`.  There is no
 * global scratch state: functions that need temporaries take a caller-owned
 * workspace, so calls on different streams or threads are independent.
 *
 * Weights are GGUF tensors in the on-disk layout: n rows of k elements, each
 * row a sequence of blocks along k (rows = outputs).  Supported ggml types:
 * F32 (0), F16 (1), Q8_0 (8), Q4_K (12), Q6_K (14).
 */
#ifndef VBHIP_H
#define VBHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VB_ABI_VERSION 1

enum {
    VB_OK = 0,
    VB_E_INVAL = -1,
    VB_E_UNSUPPORTED = -2,
    VB_E_HIP = -3,
    VB_E_NOMEM = -4,
};

enum {
    VB_TYPE_F32 = 0,
    VB_TYPE_F16 = 1,
    VB_TYPE_Q8_0 = 8,
    VB_TYPE_Q4_K = 12,
    VB_TYPE_Q6_K = 14,
};

/* ---- runtime ------------------------------------------------------------
 * Replaces the reference's RAII DeviceBuffer alloc/upload/download and its
 * CUDA_CHECK error path (cpp/include/cuda_kernels.h:35-55,
 * cpp/src/cuda_kernels.cu:24-31). */

/* Text of the last error on this thread (never NULL). */
const char* vb_last_error(void);
/* VB_ABI_VERSION of the loaded library. */
int vb_version(void);
/* Bytes of one GGUF row of k elements, or -1 if k is not a whole number of
 * blocks or the type is unknown.  Same table as ggml_blck_size /
 * ggml_type_size / tensor_nbytes (cpp/include/ggml_types.h:30-71, :195-199). */
int64_t vb_row_bytes(int32_t ggml_type, int64_t k);
/* Select the device and check that it is a gfx950. */
int vb_init(int device);
int vb_malloc(void** ptr, size_t bytes);
int vb_free(void* ptr);
int vb_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int vb_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int vb_stream_create(void** stream);
int vb_stream_sync(void* stream);
int vb_stream_destroy(void* stream);

/* ---- block decode -------------------------------------------------------
 * out[r*k + i] = dequantized element i of row r, fp32, bit-exact with the
 * GGUF decode formulas.  Replaces dequantize_row(row, out, n, type)
 * (cpp/include/dequant.h:11, cpp/src/dequant.cpp:407-425) and the CUDA
 * dequant kernels (cpp/src/cuda_kernels.cu:718-838), batched over rows. */
int vb_dequant_rows(const void* w, float* out, int64_t n_rows, int64_t k,
                    int32_t ggml_type, void* stream);

/* ---- quantize (no reference counterpart: the reference has no
 * quantizer; this writes the same blocks as the CPU oracle's quantizer and
 * exists so callers can build GGUF tensors on the device) ---------------- */
int vb_quantize_rows(const float* src, void* w, int64_t n_rows, int64_t k,
                     int32_t ggml_type, void* stream);

/* ---- dequant-fused GEMV, M = 1 ------------------------------------------
 * y[n] = sum_k W[n, k] * x[k] with W in GGUF layout (n rows of k).
 * Replaces gemv_dequant / gemv_dequant_mt (cpp/include/dequant.h:27-47,
 * cpp/src/dequant.cpp:739-792) and cuda::gemv_dequant
 * (cpp/include/cuda_kernels.h:191-199).  Note the reference C++ names the
 * output dimension N and walks W as K rows of N; this entry takes the GGUF
 * orientation (rows = outputs), as real .gguf tensors are stored. */
int vb_gemv(const void* w, const float* x, float* y, int64_t n, int64_t k,
            int32_t ggml_type, void* stream);

/* ---- dequant-fused GEMM on MFMA, M >= 2 ---------------------------------
 * Y[m, n] = sum_k X[m, k] * W[n, k]; X row-major (m x k) in fp32
 * (x_dtype = 0) or fp16 (x_dtype = 1), Y fp32 row-major (m x n).  Products
 * run on v_mfma_f32_16x16x32_f16 with W dequantized to fp16 in registers and
 * fp32 accumulation.  variant: 0 = choose, 1 = skinny (m <= 16), 2 = tiled.
 * Replaces the reference's batched path, a per-token loop of gemv_dequant
 * (cpp/src/fast_model.cpp:644-669, :905-960), and cuda::gemm_f32
 * (cpp/include/cuda_kernels.h, cpp/src/cuda_kernels.cu:184-212).
 * Weight type: Q4_K. */
int vb_gemm(const void* w, const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n,
            int64_t k, int32_t ggml_type, int32_t variant, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VBHIP_H */
