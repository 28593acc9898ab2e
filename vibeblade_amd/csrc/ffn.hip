// The FFN block of one token, fused around the dequant GEMVs:
//
//   y = x + W_down act(W_gate n, W_up n),   n = rms_norm(x, norm_w, eps)
//
// (the residual add is optional; without norm_w, n = x).  This is the dense
// FFN step of the reference's decoder layer, cpp/src/fast_model.cpp:837-975:
// RMSNorm (:838-840, rms_norm :61-71), gate and up GEMVs (:906-909),
// silu(g) * u (:949-953) or GeGLU (:943-948), the down GEMV (:957-958) and the
// residual add (:966-975), there as six passes over fp32 buffers.
//
// Here it is two launches when gate and up share a block-quantized type and
// down is block-quantized (GGUF Q4_K_M mixes Q4_K gate/up with Q4_K or Q6_K
// down):
//   1. the gate/up pair GEMV (gemv.hip, dense pairs): the workgroup
//      normalises x inside its activation encode and writes
//      h[p] = act(g_p, u_p) from the two dot products of neuron p;
//   2. the down GEMV over h, adding the residual as it writes y.
// The only intermediate in HBM is h (4 bytes per neuron).  Other type mixes
// run the same steps as separate launches (all on the GPU).
#include "vb_common.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

__global__ void __launch_bounds__(256) pair_act_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                       float* __restrict__ h, int64_t n, int kind) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) h[i] = act_pair(g[i], u[i], kind);
}

// y = a + b (y may be a or b)
__global__ void __launch_bounds__(256) add_kernel(const float* a, const float* b, float* y, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}

bool block_type(int32_t t) { return is_block_type(t); }

constexpr int64_t kAlign = 256;

int64_t up(int64_t b) { return (b + kAlign - 1) / kAlign * kAlign; }

// Workspace pieces (byte offsets): h, then for the unfused steps the
// normalised x, g, u and the down output.
struct FfnWs {
    int64_t h, xn, g, u, d, total;
};

FfnWs ffn_ws(int64_t hd, int64_t inter) {
    FfnWs w;
    w.h = 0;
    w.xn = up(inter * 4);
    w.g = w.xn + up(hd * 4);
    w.u = w.g + up(inter * 4);
    w.d = w.u + up(inter * 4);
    w.total = w.d + up(hd * 4);
    return w;
}

uint32_t blocks_of(int64_t n) { return static_cast<uint32_t>((n + 255) / 256); }

}  // namespace
}  // namespace vb

using namespace vb;

extern "C" {

int64_t vb_ffn_block_workspace(int64_t hd, int64_t inter) {
    if (hd <= 0 || inter <= 0) return -1;
    return ffn_ws(hd, inter).total;
}

int vb_ffn_block(const float* x, const float* norm_w, float eps, const void* w_gate, const void* w_up,
                 int32_t gate_up_type, const void* w_down, int32_t down_type, int64_t hd, int64_t inter,
                 int32_t act_kind, int32_t add_residual, float* y, void* workspace, size_t workspace_bytes,
                 void* stream) {
    if (!x || !w_gate || !w_up || !w_down || !y || !workspace || hd <= 0 || inter <= 0 ||
        (act_kind != ACT_SILU && act_kind != ACT_RELU2 && act_kind != ACT_GELU_TANH) ||
        !(eps >= 0.f)) {
        set_error("vb_ffn_block: bad arguments (hd=%lld, inter=%lld, act=%d)", static_cast<long long>(hd),
                  static_cast<long long>(inter), act_kind);
        return E_INVAL;
    }
    if (2 * inter > INT32_MAX) {
        set_error("vb_ffn_block: inter=%lld exceeds the supported maximum", static_cast<long long>(inter));
        return E_UNSUPPORTED;
    }
    const FfnWs ws = ffn_ws(hd, inter);
    if (static_cast<int64_t>(workspace_bytes) < ws.total || reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
        set_error("vb_ffn_block: workspace of %zu bytes (16-byte aligned) is below the %lld needed",
                  workspace_bytes, static_cast<long long>(ws.total));
        return E_INVAL;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || (norm_w && reinterpret_cast<uintptr_t>(norm_w) % 16 != 0)) {
        set_error("vb_ffn_block: x and norm_w must be 16-byte aligned");
        return E_INVAL;
    }
    hipStream_t st = as_stream(stream);
    uint8_t* base = static_cast<uint8_t*>(workspace);
    float* h = reinterpret_cast<float*>(base + ws.h);
    int rc;

    // h = act(W_gate n, W_up n)
    if (block_type(gate_up_type) && hd % 64 == 0) {
        RowSrc src;
        src.w2 = w_up;
        src.nsrc = inter;
        src.dense_pairs = true;
        GemvFuse fz;
        fz.norm_w = norm_w;
        fz.eps = eps;
        fz.act = act_kind;
        rc = gemv_dispatch_fused(w_gate, src, fz, x, h, 2 * inter, hd, gate_up_type, st);
        if (rc != OK) return rc;
    } else {
        const float* xn = x;
        if (norm_w) {
            float* xb = reinterpret_cast<float*>(base + ws.xn);
            rc = vb_rms_norm(x, norm_w, xb, 1, hd, eps, stream);
            if (rc != OK) return rc;
            xn = xb;
        }
        float* g = reinterpret_cast<float*>(base + ws.g);
        float* u = reinterpret_cast<float*>(base + ws.u);
        if ((rc = gemv_dispatch(w_gate, xn, g, inter, hd, gate_up_type, st)) != OK) return rc;
        if ((rc = gemv_dispatch(w_up, xn, u, inter, hd, gate_up_type, st)) != OK) return rc;
        pair_act_kernel<<<blocks_of(inter), 256, 0, st>>>(g, u, h, inter, act_kind);
        if ((rc = check_launch("vb_ffn_block")) != OK) return rc;
    }

    // y = x + W_down h
    if (block_type(down_type) && inter % 64 == 0) {
        GemvFuse fz;
        fz.resid = add_residual ? x : nullptr;
        return gemv_dispatch_fused(w_down, RowSrc{}, fz, h, y, hd, inter, down_type, st);
    }
    if (!add_residual) return gemv_dispatch(w_down, h, y, hd, inter, down_type, st);
    float* d = reinterpret_cast<float*>(base + ws.d);
    if ((rc = gemv_dispatch(w_down, h, d, hd, inter, down_type, st)) != OK) return rc;
    add_kernel<<<blocks_of(hd), 256, 0, st>>>(x, d, y, hd);
    return check_launch("vb_ffn_block");
}

}  // extern "C"
