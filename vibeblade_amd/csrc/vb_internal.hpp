// Entry points shared between translation units of libvbhip (not exported).
#pragma once

#include "vb_common.hpp"

namespace vb {

// Launch-shape overrides for tuning sweeps, read from the environment once
// per process (vb_init reads them; so does the first op call without it):
//   VB_GEMV_RING=d, VB_GEMV_CFG="wpg,rpg"   GEMV ring depth / workgroup shape
//   VB_GEMV_Q4K_PATH=mfma|dot                 Q4_K GEMV on the int8-MFMA kernel, or on
//                                             the general v_dot4 kernel for every shape
//   VB_GEMV_Q6K_PATH=dot, VB_GEMV_Q8_PATH=dot  Q6_K / Q8_0 GEMV on the general kernel for every shape
//   VB_GEMV_MFMA_CFG="wpg,ks"                 that kernel's workgroup shape
//   VB_GEMM_NF=6|8                            tiled GEMM columns per workgroup
//   VB_GEMM_TILE="wm,wn,nf[,ks]"              tiled GEMM tile configuration (ks: K halves per
//                                             workgroup, 1 or 2)
//   VB_GEMM_SPLIT_MIN_M=m                     smallest M (up to 768) on the role-split GEMM (0: never)
//   VB_GEMM_ZSPLIT=z                          with VB_GEMM_TILE: K splits between workgroups (Q6_K / Q8_0,
//                                             fp16 X, M >= 384, N < 8192)
//   VB_GEMV_DMA=0                             short- and split-row Q4_K GEMV (fp32 x): register ring
//                                             instead of LDS DMA
//   VB_GEMV_SPLIT="sl,d"                      split-row Q4_K GEMV: slices per row (2, 4, 8), rows in flight (1-4)
//   VB_SPARSE_FUSED=0, VB_SPARSE_NPW=1|2      sparse FFN kernel choice (NPW: the row-split fused
//                                             kernel with 1 or 2 neurons per wave)
// Zero / false means "no override".
struct Knobs {
    int gemv_ring = 0;
    bool gemv_dma = true;  // short-row Q4_K GEMV: rows into LDS by DMA (VB_GEMV_DMA=0: register ring)
    int gemv_cfg_wpg = 0, gemv_cfg_rpg = 0;
    bool gemv_q4k_mfma = false;
    bool gemv_q4k_general = false;
    bool gemv_q6k_general = false;
    bool gemv_q8_general = false;
    int gemv_mfma_wpg = 0, gemv_mfma_ks = 0;
    int gemm_nf = 0;
    int gemm_tile_wm = 0, gemm_tile_wn = 0, gemm_tile_nf = 0, gemm_tile_ks = 1;
    int gemm_split_min_m = -1;  // smallest M on the role-split kernel (-1: default)
    int gemm_zsplit = 0;        // with VB_GEMM_TILE: K splits between workgroups (Q6_K / Q8_0)
    bool gemm_xr_kq = true;     // Q6_K / Q8_0 on the packed-X kernel where Q4_K takes it (VB_GEMM_XR_KQ=0: tiled)
    int gemv_split_sl = 0, gemv_split_d = 0;  // split-row Q4_K GEMV: slices per row, rows in flight
    bool sparse_fused = true;
    int sparse_npw = 0;
};
const Knobs& knobs();

// Compute units of the current device, from its properties (cached per
// device; 256 on MI355X).
int num_cus();

// Device address of the allocation-free sparse FFN's static scratch on the
// current device (sparse.hip; resolved once per device).
int sparse_scratch_ptr(void** out);

// Rows of a GEMV launch: plain (row r of w), or gathered gate/up pairs of a
// sparse FFN (row r = row gidx[r/2] of w for even r, of w2 for odd r).  zbuf
// / zn: an int buffer the launch clears (counters of a following kernel).
struct RowSrc {
    const void* w2 = nullptr;
    const int32_t* gidx = nullptr;
    int64_t nsrc = 0;  // rows of w / w2; gathered indices are clamped to [0, nsrc)
    int* zbuf = nullptr;
    int zn = 0;
    // dense gate/up pairs: row r = row r/2 of w (r even) or of w2 (r odd),
    // no index list (an FFN block: every neuron)
    bool dense_pairs = false;
    // gathered pairs: the number of pairs written by the device (a predicted
    // active set); n / 2 is then the host's bound and rows past 2 * count
    // are not computed
    const int32_t* n_dev = nullptr;
};

// Work fused into a block-quantized GEMV launch (Q4_K / Q6_K / Q8_0):
//  norm_w  RMSNorm prologue: x is replaced by x * (1 / sqrt(mean(x^2) + eps))
//          * norm_w inside the activation encode; every workgroup reduces
//          sum(x^2) over all of x itself, in a fixed order.
//  act     >= 0: pair epilogue.  Rows 2p and 2p+1 are the gate and up rows
//          of neuron p, and the launch writes y[p] = act_pair(dot(2p),
//          dot(2p+1), act) for p < n/2 instead of n dot products.
//  resid   y[r] = dot(r) + resid[r] (resid may be y itself).
struct GemvFuse {
    const float* norm_w = nullptr;
    float eps = 0.f;
    int act = -1;
    const float* resid = nullptr;
    bool any() const { return norm_w != nullptr || act >= 0 || resid != nullptr; }
};

int gemv_dispatch(const void* w, const float* x, float* y, int64_t n, int64_t k, int32_t type,
                  hipStream_t st);
int gemv_dispatch_src(const void* w, const RowSrc& src, const float* x, float* y, int64_t n, int64_t k,
                      int32_t type, hipStream_t st);
// gemv_dispatch_src with fused prologue / epilogue work; VB_E_UNSUPPORTED
// for types without it (F32 / F16) and for the int8-MFMA GEMV path.
int gemv_dispatch_fused(const void* w, const RowSrc& src, const GemvFuse& fz, const float* x, float* y,
                        int64_t n, int64_t k, int32_t type, hipStream_t st);
// Plain Q4_K GEMV for k <= 4096 at up to 8 rows per wave (gemv_q4k.hip);
// gemv_q4k_rpw(n) is its rows per wave, 0 when n is too large for it.
int gemv_q4k_rpw(int64_t n);
// x_half: x in fp16 (vb_gemm with one fp16 activation row).
int gemv_q4k_short(const void* w, const void* x, float* y, int64_t n, int64_t k, hipStream_t st,
                   bool x_half = false);
// Plain Q6_K (k = 2048 / 4096) and Q8_0 (k % 256 == 0, k <= 4096) GEMV on
// the short-row arithmetic (gemv_q4k.hip); gemv_short_rpw is its rows per
// wave, 0 for types and shapes it does not take.  x_half: x in fp16 (the
// one-row GEMM).
int gemv_short_rpw(int32_t type, int64_t n, int64_t k);
int gemv_short(int32_t type, const void* w, const void* x, float* y, int64_t n, int64_t k, hipStream_t st,
               bool x_half = false);
// Plain or residual-epilogue Q6_K (k % 512 == 0) / Q8_0 GEMV for 4096 < k <=
// 16384 on the split-row kernel with the short-row units (gemv_q4k.hip);
// gemv_split_rpw is 0 for types and shapes it does not take.
int gemv_split_rpw(int32_t type, int64_t n, int64_t k);
int gemv_split(int32_t type, const void* w, const void* x, float* y, const float* resid, int64_t n, int64_t k,
               hipStream_t st, bool x_half = false);
// Plain or residual-epilogue Q4_K GEMV for 4096 < k <= 16384, rows split over
// 2, 4 or 8 waves (gemv_q4k.hip); gemv_q4k_split_rpw is 0 for shapes it does not take.
int gemv_q4k_split_rpw(int64_t n, int64_t k);
// Q4_K gate/up pairs with the activation epilogue (and an optional RMSNorm of
// x) for k <= 4096 on the short-row arithmetic (gemv_q4k.hip): y[p] =
// act(gate_p . n, up_p . n) for p < n neurons; gemv_q4k_pairs_npw is 0 for
// neuron counts it does not take.  With `active` (sorted, unique): neuron p
// is row active[p] (p below the device count n_dev when given) and y is the
// whole hidden vector of i_dim entries, zeros off the active set.
int gemv_q4k_pairs_npw(int64_t n);
int gemv_q4k_pairs(const void* wg, const void* wu, const float* x, const float* norm_w, float eps, int kind,
                   float* y, int64_t n, int64_t k, hipStream_t st, const int32_t* active = nullptr,
                   const int32_t* n_dev = nullptr, int64_t i_dim = 0);
int gemv_q4k_split(const void* w, const void* x, float* y, const float* resid, int64_t n, int64_t k,
                   hipStream_t st, bool x_half = false);
// Q4_K M=1 GEMV on the int8 matrix cores (gemv_q4k_mfma.hip); arguments
// already validated by gemv_dispatch_src.
int gemv_q4k_mfma(const void* w, const RowSrc& src, const float* x, float* y, int64_t n, int64_t k,
                  hipStream_t st);
// M <= 32 Q4_K GEMM (gemm_skinny.hip); type, M, alignment already validated.
int gemm_q4k_skinny(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K,
                    hipStream_t st);
// Role-split Q4_K GEMM, fp16 X (gemm_split.hip); type, alignment and the
// 32-bit offset bounds already validated.
int gemm_q4k_split(const void* w, const void* X, float* Y, int64_t M, int64_t N, int64_t K, hipStream_t st);
// Q4_K / Q6_K / Q8_0 GEMM with the activation fragments loaded into
// registers from X packed in fragment order, fp16 X (gemm_xr.hip): a type
// gemm_xr_type takes, W and X 16-byte aligned, the 32-bit offset bounds,
// K % 256 == 0, M >= 256 and a 16-byte-aligned workspace of
// gemm_xr_workspace(M, N, K) bytes (the packed X, and the partial products
// of the K splits when the output tiles are fewer than the CUs).
bool gemm_xr_type(int32_t type);
int gemm_xr_ksplit(int64_t M, int64_t N, int64_t K);
// Y[0, total) = P[0, total) + P[total, 2 total) + ... (ks partial products,
// added in that order), fp32 (gemm_xr.hip).
int gemm_ksum(const float* P, float* Y, int64_t total, int ks, hipStream_t st);
// K splits of the tiled GEMM between workgroups for this shape (1: none; gemm.hip).
int tiled_zsplit(int type, int x_dtype, int64_t M, int64_t N, int64_t K);
int64_t gemm_xr_workspace(int64_t M, int64_t N, int64_t K);
// n_rows x k of W (a decodable type other than F16) as row-major fp16 at out,
// each value rounded once (dequant.hip; k % 4 == 0, out 16-byte aligned).
int dequant_rows_f16(const void* w, _Float16* out, int64_t n_rows, int64_t k, int32_t type, hipStream_t st);
// Weight types the batched GEMM runs through their fp16 decode (gemm.hip),
// and the workspace that decode needs (n x k x 2 bytes; 0 for F16).
bool gemm_other_type(int32_t type);
// Q4_0 / Q4_1 / Q5_0 / Q5_1, which the K-split and packed-X kernels decode
// themselves, and the largest M at which they take the K-split kernel by
// default (gemm.hip)
bool gemm_b32_type(int32_t type);
bool gemm_b32_high(int32_t type);  // Q5_0 / Q5_1
int64_t gemm_b32_kq_max_m(int64_t N);
int64_t gemm_other_workspace(int32_t type, int64_t N, int64_t K);
int gemm_xr(const void* w, const void* X, float* Y, int64_t M, int64_t N, int64_t K, int32_t type, void* ws,
            hipStream_t st);
// Q6_K / Q8_0 GEMM, every M (gemm_kq.hip); pointers, alignment, x_dtype and
// M, N > 0 already validated.
int gemm_kq(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K, int32_t type,
            hipStream_t st);
// ws / ws_bytes: the caller's workspace (may be null / 0: the kernels that
// need one are then not chosen, and variant 5 is refused).
// Expert-grouped K-split products of the MoE FFN (gemm_kq.hip) for the
// expert types other than Q4_K (and Q4_K where the caller asks): gate_up
// writes fp16 silu(W0 x) * (W1 x) into hout[slot][n] from rows slot / topk of
// the fp16 X; otherwise fout[slot][n] = W0 x from rows slot of X, or, with
// yacc (top-k <= 2), rw[slot] W0 x added atomically into the zeroed
// yacc[slot / topk][n].  eoff / elist: per-expert slot lists over nslots
// slots.
constexpr int MOE_KQ_MAX_EXPERTS = 64;
int moe_kq(int32_t type, bool gate_up, const void* const* w0, const void* const* w1, int n_exp, const void* X,
           int64_t xbytes, int topk, const int32_t* eoff, const int32_t* elist, int nslots, int64_t N, int64_t K,
           _Float16* hout, float* fout, const float* rw, float* yacc, hipStream_t st);
int gemm_dispatch(const void* w, const void* X, int32_t x_dtype, float* Y, int64_t M, int64_t N, int64_t K,
                  int32_t type, int32_t variant, void* ws, size_t ws_bytes, hipStream_t st);

}  // namespace vb
