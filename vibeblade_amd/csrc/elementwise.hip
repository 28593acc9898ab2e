// Elementwise activations for the GPUBackend-compatible surface
// (vibeblade/gpu.py:100-124: drelu = max(x, 0), silu = x * sigmoid(x)).
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

}  // namespace
}  // namespace vb

using namespace vb;

extern "C" int vb_activation(const float* x, float* y, int64_t n, int32_t kind, void* stream) {
    if (n < 0 || (kind != 0 && kind != 1) || (n > 0 && (!x || !y))) {
        set_error("vb_activation: bad arguments");
        return E_INVAL;
    }
    if (n == 0) return OK;
    act_kernel<<<dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(x, y, n, kind);
    return check_launch("vb_activation");
}
