// MoE expert-grouped FFN: route, group tokens per expert, SwiGLU experts,
// weighted combine.
//
// Reference semantics: per token, softmax over the router logits (clamped to
// +-50), top-k, renormalise the k weights (vibeblade/moe.py:184-206,
// cpp/src/fast_model.cpp:534-548), expert FFN down(silu(gate x) * up x)
// (vibeblade/moe_executor.py:331-344, cpp/src/fast_model.cpp:552-572), and
// y_t = sum_k w_tk * FFN_(e_tk)(x_t) (vibeblade/moe.py:457-482).  The
// reference's HotColdExecutor.dispatch routes only the first token of a batch
// (vibeblade/moe_executor.py:210-212); this routes every token.
//
// Three launches, no host round trip:
//   1. gate/up: grid (i/16, E).  Every workgroup recomputes the routing (T x E
//      logits, cheap), lists the (token, slot) pairs that chose its expert in
//      token order and, if any, computes the 16 gate and up rows of its tile
//      for those tokens on v_mfma_f32_16x16x32_f16 (X rows gathered, Q4_K
//      weights dequantized to fp16 in registers), 4 waves splitting k; the
//      epilogue writes silu(g) * u for every (slot, row) into hbuf.
//   2. down: grid (h/16, E), same routing, A rows = hbuf slots of the expert,
//      writes the expert output of every slot into obuf.
//   3. combine: y_t = sum_k w_tk * obuf[t*topk + k] in slot order (fixed
//      order, deterministic); also writes the routing (indices, weights).
// Each expert's weights are streamed once per 16 routed slots.
#include "mfma_q4k.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int MOE_MAX_EXPERTS = 64;
constexpr int MOE_MAX_TOPK = 8;
constexpr int MOE_MAX_SLOTS = 1024;  // tokens * topk

struct ExpertPtrs {
    const uint8_t* p[MOE_MAX_EXPERTS];
};

// Route token t: top-k of softmax(clamp(logits, -50, 50)), renormalised.
// Ties go to the lower expert id.
__device__ void route_token(const float* __restrict__ logits, int e_n, int topk, int* idx, float* w) {
    float mx = -INFINITY;
    for (int e = 0; e < e_n; e++) mx = fmaxf(mx, fminf(fmaxf(logits[e], -50.f), 50.f));
    float denom = 0.f;
    for (int e = 0; e < e_n; e++) denom += __expf(fminf(fmaxf(logits[e], -50.f), 50.f) - mx);
    for (int k = 0; k < topk; k++) {
        idx[k] = -1;
        w[k] = -1.f;
    }
    for (int e = 0; e < e_n; e++) {
        const float p = __expf(fminf(fmaxf(logits[e], -50.f), 50.f) - mx) / denom;
        int pos = topk;
        while (pos > 0 && p > w[pos - 1]) pos--;
        if (pos < topk) {
            for (int j = topk - 1; j > pos; j--) {
                w[j] = w[j - 1];
                idx[j] = idx[j - 1];
            }
            w[pos] = p;
            idx[pos] = e;
        }
    }
    float s = 0.f;
    for (int k = 0; k < topk; k++) s += w[k];
    s = s < 1e-12f ? 1.f : s;
    for (int k = 0; k < topk; k++) w[k] /= s;
}

// Slots (t*topk + k) routed to expert `e`, in slot order, into slots[];
// returns the count.  Uses the first T threads; all threads must call.
__device__ int expert_slots(const float* __restrict__ logits, int t_n, int e_n, int topk, int e,
                            int* slots, int* flags) {
    for (int t = threadIdx.x; t < t_n; t += blockDim.x) {
        int idx[MOE_MAX_TOPK];
        float w[MOE_MAX_TOPK];
        route_token(logits + static_cast<int64_t>(t) * e_n, e_n, topk, idx, w);
        for (int k = 0; k < topk; k++) flags[t * topk + k] = idx[k] == e ? 1 : 0;
    }
    __syncthreads();
    __shared__ int count;
    if (threadIdx.x == 0) {
        int c = 0;
        for (int s = 0; s < t_n * topk; s++)
            if (flags[s]) slots[c++] = s;
        count = c;
    }
    __syncthreads();
    return count;
}

// One 16-row tile of Q4_K weights times the gathered fp32 activation rows
// arow[0..nrow) (nrow <= 16), k split over the 4 waves.  NMAT = 1 or 2
// matrices over the same activations.  Returns the per-lane D fragments of
// the full-k sums in red (LDS, [4 waves][64 lanes] per matrix).
template <int NMAT, int WT>
__device__ void tile_mfma(const uint8_t* const* wrow, const float* const* arow, int nrow, int64_t k,
                          float4_t (*red)[4][64]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int nsb = static_cast<int>(k / 256);
    const int sb0 = (wave * nsb) / 4, sb1 = ((wave + 1) * nsb) / 4;
    const bool avalid = j < nrow;
    const float* ap = avalid ? arow[j] : arow[0];
    float4_t acc[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) acc[m] = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int sb = sb0; sb < sb1; sb++) {
        Frag a[8];
#pragma unroll
        for (int sub = 0; sub < 8; sub++) {
            const float* p = ap + static_cast<int64_t>(sb) * 256 + 32 * sub + 8 * g;
            const float4 lo4 = *reinterpret_cast<const float4*>(p);
            const float4 hi4 = *reinterpret_cast<const float4*>(p + 4);
            f32x8_to_frag(avalid ? lo4 : make_float4(0.f, 0.f, 0.f, 0.f),
                          avalid ? hi4 : make_float4(0.f, 0.f, 0.f, 0.f), a[sub].u);
        }
        if constexpr (WT == TYPE_Q4_K) {
            uint4 hd[NMAT];
            uint2 qs[NMAT][4];
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const uint8_t* b = wrow[m] + static_cast<int64_t>(sb) * 144;
                hd[m] = *reinterpret_cast<const uint4*>(b);
#pragma unroll
                for (int c = 0; c < 4; c++) qs[m][c] = *reinterpret_cast<const uint2*>(b + 16 + 32 * c + 8 * g);
            }
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    half2_t ds[2], nm[2];
                    q4k_chunk_scales(hd[m], c, ds, nm);
                    Frag lo, hi;
                    q4k_bfrags(qs[m][c].x, qs[m][c].y, ds, nm, lo, hi);
                    acc[m] = mfma16x16x32(a[2 * c], lo, acc[m]);
                    acc[m] = mfma16x16x32(a[2 * c + 1], hi, acc[m]);
                }
            }
        } else {  // F32 weights: row n, k = 256 sb + 32 sub + 8 g .. +8, rounded to fp16
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const float* wp = reinterpret_cast<const float*>(wrow[m]) + static_cast<int64_t>(sb) * 256 + 8 * g;
#pragma unroll
                for (int sub = 0; sub < 8; sub++) {
                    Frag b;
                    f32x8_to_frag(*reinterpret_cast<const float4*>(wp + 32 * sub),
                                  *reinterpret_cast<const float4*>(wp + 32 * sub + 4), b.u);
                    acc[m] = mfma16x16x32(a[sub], b, acc[m]);
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++) red[m][wave][lane] = acc[m];
    __syncthreads();
}

template <int WT>
__global__ void __launch_bounds__(256) moe_gate_up_kernel(ExpertPtrs wg, ExpertPtrs wu, const float* __restrict__ x,
                                                          const float* __restrict__ logits, int t_n, int e_n,
                                                          int topk, int64_t h, int64_t i_dim, int64_t rb,
                                                          float* __restrict__ hbuf) {
    __shared__ int slots[MOE_MAX_SLOTS], flags[MOE_MAX_SLOTS];
    __shared__ float4_t red[2][4][64];
    const int e = blockIdx.y;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    const int cnt = expert_slots(logits, t_n, e_n, topk, e, slots, flags);
    if (cnt == 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    int64_t n = n0 + j;
    n = n < i_dim ? n : i_dim - 1;
    const uint8_t* wrow[2] = {wg.p[e] + n * rb, wu.p[e] + n * rb};
    for (int m0 = 0; m0 < cnt; m0 += 16) {
        const int nrow = cnt - m0 < 16 ? cnt - m0 : 16;
        const float* arow[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int s = slots[m0 + (r < nrow ? r : 0)];
            arow[r] = x + static_cast<int64_t>(s / topk) * h;
        }
        tile_mfma<2, WT>(wrow, arow, nrow, h, red);
        if (wave == 0) {
            const float4_t gs = (red[0][0][lane] + red[0][1][lane]) + (red[0][2][lane] + red[0][3][lane]);
            const float4_t us = (red[1][0][lane] + red[1][1][lane]) + (red[1][2][lane] + red[1][3][lane]);
            const int64_t col = n0 + j;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * g + r;
                if (row < nrow && col < i_dim) {
                    const float gv = gs[r];
                    hbuf[static_cast<int64_t>(slots[m0 + row]) * i_dim + col] = gv / (1.0f + __expf(-gv)) * us[r];
                }
            }
        }
        __syncthreads();
    }
}

template <int WT>
__global__ void __launch_bounds__(256) moe_down_kernel(ExpertPtrs wd, const float* __restrict__ hbuf,
                                                       const float* __restrict__ logits, int t_n, int e_n,
                                                       int topk, int64_t h, int64_t i_dim, int64_t rb,
                                                       float* __restrict__ obuf) {
    __shared__ int slots[MOE_MAX_SLOTS], flags[MOE_MAX_SLOTS];
    __shared__ float4_t red[1][4][64];
    const int e = blockIdx.y;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    const int cnt = expert_slots(logits, t_n, e_n, topk, e, slots, flags);
    if (cnt == 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    int64_t n = n0 + j;
    n = n < h ? n : h - 1;
    const uint8_t* wrow[1] = {wd.p[e] + n * rb};
    for (int m0 = 0; m0 < cnt; m0 += 16) {
        const int nrow = cnt - m0 < 16 ? cnt - m0 : 16;
        const float* arow[16];
#pragma unroll
        for (int r = 0; r < 16; r++) arow[r] = hbuf + static_cast<int64_t>(slots[m0 + (r < nrow ? r : 0)]) * i_dim;
        tile_mfma<1, WT>(wrow, arow, nrow, i_dim, red);
        if (wave == 0) {
            const float4_t s = (red[0][0][lane] + red[0][1][lane]) + (red[0][2][lane] + red[0][3][lane]);
            const int64_t col = n0 + j;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * g + r;
                if (row < nrow && col < h) obuf[static_cast<int64_t>(slots[m0 + row]) * h + col] = s[r];
            }
        }
        __syncthreads();
    }
}

__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ obuf,
                                                          const float* __restrict__ logits, int e_n, int topk,
                                                          int64_t h, float* __restrict__ y,
                                                          int32_t* __restrict__ out_idx,
                                                          float* __restrict__ out_w) {
    const int t = blockIdx.x;
    __shared__ int sidx[MOE_MAX_TOPK];
    __shared__ float sw[MOE_MAX_TOPK];
    if (threadIdx.x == 0) {
        int idx[MOE_MAX_TOPK];
        float w[MOE_MAX_TOPK];
        route_token(logits + static_cast<int64_t>(t) * e_n, e_n, topk, idx, w);
        for (int k = 0; k < topk; k++) {
            sidx[k] = idx[k];
            sw[k] = w[k];
            if (out_idx) out_idx[t * topk + k] = idx[k];
            if (out_w) out_w[t * topk + k] = w[k];
        }
    }
    __syncthreads();
    for (int64_t o = threadIdx.x; o < h; o += blockDim.x) {
        float s = 0.f;
        for (int k = 0; k < topk; k++) s += sw[k] * obuf[(static_cast<int64_t>(t) * topk + k) * h + o];
        y[static_cast<int64_t>(t) * h + o] = s;
    }
}

struct MoeWs {
    size_t hbuf, obuf, total;
};

MoeWs moe_ws(int64_t t, int32_t topk, int64_t h, int64_t i) {
    MoeWs w;
    auto al = [](size_t b) { return (b + 255) & ~size_t(255); };
    w.hbuf = 0;
    w.obuf = al(static_cast<size_t>(t) * topk * i * sizeof(float));
    w.total = w.obuf + al(static_cast<size_t>(t) * topk * h * sizeof(float));
    return w;
}

}  // namespace
}  // namespace vb

using namespace vb;

extern "C" int64_t vb_moe_workspace(int32_t n_tokens, int32_t topk, int64_t h, int64_t i) {
    if (n_tokens < 0 || topk <= 0 || h <= 0 || i <= 0) return -1;
    return static_cast<int64_t>(moe_ws(n_tokens, topk, h, i).total);
}

extern "C" int vb_moe_grouped_ffn(const void* const* wg, const void* const* wu, const void* const* wd,
                                  int32_t n_exp, const float* x, int32_t n_tokens, const float* router_logits,
                                  int32_t topk, float* y, int32_t* out_idx, float* out_w, int64_t h,
                                  int64_t i, int32_t ggml_type, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    hipStream_t st = as_stream(stream);
    if (n_exp <= 0 || n_exp > MOE_MAX_EXPERTS || topk <= 0 || topk > MOE_MAX_TOPK || topk > n_exp ||
        n_tokens < 0 || static_cast<int64_t>(n_tokens) * topk > MOE_MAX_SLOTS || h <= 0 || i <= 0 || !wg ||
        !wu || !wd || (n_tokens > 0 && (!x || !router_logits || !y))) {
        set_error("vb_moe_grouped_ffn: bad arguments (n_exp<=%d, topk<=%d, tokens*topk<=%d)", MOE_MAX_EXPERTS,
                  MOE_MAX_TOPK, MOE_MAX_SLOTS);
        return E_INVAL;
    }
    if ((ggml_type != TYPE_Q4_K && ggml_type != TYPE_F32) || h % 256 != 0 || i % 256 != 0) {
        set_error("vb_moe_grouped_ffn: Q4_K or F32 experts with h, i multiples of 256 are supported");
        return E_UNSUPPORTED;
    }
    if (n_tokens == 0) return OK;
    if (reinterpret_cast<uintptr_t>(x) % 16) {
        set_error("vb_moe_grouped_ffn: x must be 16-byte aligned");
        return E_INVAL;
    }
    const MoeWs ws = moe_ws(n_tokens, topk, h, i);
    if (!workspace || workspace_bytes < ws.total) {
        set_error("vb_moe_grouped_ffn: workspace of %zu bytes needed", ws.total);
        return E_NOMEM;
    }
    ExpertPtrs pg{}, pu{}, pd{};
    for (int e = 0; e < n_exp; e++) {
        if (!wg[e] || !wu[e] || !wd[e] || reinterpret_cast<uintptr_t>(wg[e]) % 16 ||
            reinterpret_cast<uintptr_t>(wu[e]) % 16 || reinterpret_cast<uintptr_t>(wd[e]) % 16) {
            set_error("vb_moe_grouped_ffn: expert %d weights null or not 16-byte aligned", e);
            return E_INVAL;
        }
        pg.p[e] = static_cast<const uint8_t*>(wg[e]);
        pu.p[e] = static_cast<const uint8_t*>(wu[e]);
        pd.p[e] = static_cast<const uint8_t*>(wd[e]);
    }
    float* hbuf = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + ws.hbuf);
    float* obuf = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + ws.obuf);
    const dim3 gu_grid(static_cast<uint32_t>((i + 15) / 16), n_exp), dn_grid(static_cast<uint32_t>((h + 15) / 16), n_exp);
    if (ggml_type == TYPE_Q4_K)
        moe_gate_up_kernel<TYPE_Q4_K><<<gu_grid, dim3(256), 0, st>>>(pg, pu, x, router_logits, n_tokens, n_exp, topk,
                                                                     h, i, row_bytes(ggml_type, h), hbuf);
    else
        moe_gate_up_kernel<TYPE_F32><<<gu_grid, dim3(256), 0, st>>>(pg, pu, x, router_logits, n_tokens, n_exp, topk,
                                                                    h, i, row_bytes(ggml_type, h), hbuf);
    int rc = check_launch("vb_moe_grouped_ffn");
    if (rc != OK) return rc;
    if (ggml_type == TYPE_Q4_K)
        moe_down_kernel<TYPE_Q4_K><<<dn_grid, dim3(256), 0, st>>>(pd, hbuf, router_logits, n_tokens, n_exp, topk, h, i,
                                                                  row_bytes(ggml_type, i), obuf);
    else
        moe_down_kernel<TYPE_F32><<<dn_grid, dim3(256), 0, st>>>(pd, hbuf, router_logits, n_tokens, n_exp, topk, h, i,
                                                                 row_bytes(ggml_type, i), obuf);
    if ((rc = check_launch("vb_moe_grouped_ffn")) != OK) return rc;
    moe_combine_kernel<<<dim3(static_cast<uint32_t>(n_tokens)), dim3(256), 0, st>>>(obuf, router_logits, n_exp,
                                                                                  topk, h, y, out_idx, out_w);
    return check_launch("vb_moe_grouped_ffn");
}

namespace vb {
namespace {
__global__ void __launch_bounds__(256) moe_route_kernel(const float* __restrict__ logits, int t_n, int e_n, int topk,
                                                        int32_t* __restrict__ out_idx, float* __restrict__ out_w) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= t_n) return;
    int idx[MOE_MAX_TOPK];
    float w[MOE_MAX_TOPK];
    route_token(logits + static_cast<int64_t>(t) * e_n, e_n, topk, idx, w);
    for (int k = 0; k < topk; k++) {
        out_idx[t * topk + k] = idx[k];
        out_w[t * topk + k] = w[k];
    }
}
}  // namespace
}  // namespace vb

extern "C" int vb_moe_route(const float* router_logits, int32_t n_tokens, int32_t n_exp, int32_t topk,
                            int32_t* out_idx, float* out_w, void* stream) {
    if (n_exp <= 0 || n_exp > MOE_MAX_EXPERTS || topk <= 0 || topk > MOE_MAX_TOPK || topk > n_exp || n_tokens < 0 ||
        (n_tokens > 0 && (!router_logits || !out_idx || !out_w))) {
        set_error("vb_moe_route: bad arguments");
        return E_INVAL;
    }
    if (n_tokens == 0) return OK;
    moe_route_kernel<<<dim3(static_cast<uint32_t>((n_tokens + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(
        router_logits, n_tokens, n_exp, topk, out_idx, out_w);
    return check_launch("vb_moe_route");
}
