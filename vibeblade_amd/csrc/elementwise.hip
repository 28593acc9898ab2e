// Elementwise and row-wise ops of the GPUBackend-compatible surface
// (vibeblade/gpu.py:100-198: drelu = max(x, 0), silu = x * sigmoid(x),
// rms_norm, softmax).
#include "vb_common.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

__global__ void __launch_bounds__(256) act_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n,
                                                  int kind) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    y[i] = kind == 0 ? v / (1.0f + __expf(-v)) : fmaxf(v, 0.f);
}

// One workgroup per row: y = x / sqrt(mean(x^2) + eps) * w.
__global__ void __launch_bounds__(256) rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       float* __restrict__ y, int64_t dim, float eps) {
    __shared__ float part[4];
    const float* xr = x + static_cast<int64_t>(blockIdx.x) * dim;
    float* yr = y + static_cast<int64_t>(blockIdx.x) * dim;
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) s += xr[i] * xr[i];
    s = wave_sum_dpp(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(dim) + eps);
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) yr[i] = xr[i] * inv * w[i];
}

// One workgroup per row: numerically stable softmax.
__global__ void __launch_bounds__(256) softmax_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    __shared__ float part[4];
    const float* xr = x + static_cast<int64_t>(blockIdx.x) * n;
    float* yr = y + static_cast<int64_t>(blockIdx.x) * n;
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, xr[i]);
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    __syncthreads();
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) s += __expf(xr[i] - m);
    s = wave_sum_dpp(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) yr[i] = __expf(xr[i] - m) / tot;
}

}  // namespace
}  // namespace vb

using namespace vb;

extern "C" int vb_rms_norm(const float* x, const float* w, float* y, int64_t rows, int64_t dim, float eps,
                           void* stream) {
    if (rows < 0 || dim <= 0 || rows > 0x7fffffff || (rows > 0 && (!x || !w || !y))) {
        set_error("vb_rms_norm: bad arguments");
        return E_INVAL;
    }
    if (rows == 0) return OK;
    rms_norm_kernel<<<dim3(static_cast<uint32_t>(rows)), dim3(256), 0, as_stream(stream)>>>(x, w, y, dim, eps);
    return check_launch("vb_rms_norm");
}

extern "C" int vb_softmax(const float* x, float* y, int64_t rows, int64_t n, void* stream) {
    if (rows < 0 || n <= 0 || rows > 0x7fffffff || (rows > 0 && (!x || !y))) {
        set_error("vb_softmax: bad arguments");
        return E_INVAL;
    }
    if (rows == 0) return OK;
    softmax_kernel<<<dim3(static_cast<uint32_t>(rows)), dim3(256), 0, as_stream(stream)>>>(x, y, n);
    return check_launch("vb_softmax");
}

extern "C" int vb_activation(const float* x, float* y, int64_t n, int32_t kind, void* stream) {
    if (n < 0 || (kind != 0 && kind != 1) || (n > 0 && (!x || !y))) {
        set_error("vb_activation: bad arguments");
        return E_INVAL;
    }
    if (n == 0) return OK;
    act_kernel<<<dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(x, y, n, kind);
    return check_launch("vb_activation");
}
