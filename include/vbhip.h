/*
 * libvbhip -- gfx950 (MI355X) GGUF quantized matmul: the C ABI.
 *
 * Every function returns an int status (0 = VB_OK, negative = error) unless
 * stated otherwise; vb_last_error() returns the thread-local text of the last
 * failure.  No C++ exception crosses this boundary.  All pointers passed to
 * the op functions are device pointers; `stream` is a hipStream_t (NULL =
 * the default stream).  Launches are asynchronous on `stream`.  Apart from
 * vb_sparse_ffn_noalloc (a static device array, described at its
 * declaration) there is no global scratch state: functions that need
 * temporaries take a caller-owned workspace, so calls on different streams
 * or threads are independent.
 * Every buffer of a call (inputs, outputs, workspace) must be ready in the
 * order of `stream` when the call is enqueued: memory that work on another
 * stream still writes (a block a caching allocator handed out again while a
 * kernel on its old stream is pending, say) needs an event wait or a
 * synchronisation first.  (The MoE expert kernels clamp the routing lists
 * they read from the workspace, so a race there gives wrong values, not
 * accesses outside the buffers.)
 *
 * Weights are GGUF tensors in the on-disk layout: n rows of k elements, each
 * row a sequence of blocks along k (rows = outputs).  Supported ggml types
 * (decode, GEMV, FFN block, sparse FFN with GGUF-layout down): F32 (0),
 * F16 (1), Q4_0 (2), Q4_1 (3), Q5_0 (6), Q5_1 (7), Q8_0 (8), Q2_K (10),
 * Q3_K (11), Q4_K (12), Q5_K (13), Q6_K (14), BF16 (30).  Each op's comment
 * lists the subset it takes where that is narrower (vb_gemm, the fused
 * neuron-major sparse FFN, vb_moe_grouped_ffn, vb_quantize_rows).
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
    VB_TYPE_Q4_0 = 2,
    VB_TYPE_Q4_1 = 3,
    VB_TYPE_Q5_0 = 6,
    VB_TYPE_Q5_1 = 7,
    VB_TYPE_Q8_0 = 8,
    VB_TYPE_Q2_K = 10,
    VB_TYPE_Q3_K = 11,
    VB_TYPE_Q4_K = 12,
    VB_TYPE_Q5_K = 13,
    VB_TYPE_Q6_K = 14,
    VB_TYPE_BF16 = 30,
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
/* Select the device and check that it is a gfx950; also reads the launch
 * tuning overrides (VB_GEMV_RING, VB_GEMV_CFG, VB_GEMV_Q4K_PATH,
 * VB_GEMV_Q6K_PATH, VB_GEMV_Q8_PATH, VB_GEMV_SPLIT, VB_GEMV_MFMA_CFG,
 * VB_GEMM_NF, VB_GEMM_TILE, VB_GEMM_SPLIT_MIN_M, VB_GEMM_XR_KQ,
 * VB_SPARSE_FUSED, VB_SPARSE_NPW) from the environment, once per process, and the device's
 * compute-unit count. */
int vb_init(int device);
/* Re-read the tuning overrides from the environment (for tuning sweeps and
 * tests).  Not synchronised with op calls running on other threads: their
 * launches use either the old or the new settings.  No counterpart in the
 * reference, which has no launch tuning. */
int vb_tuning_reload(void);
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

/* out[t, :] = decoded row tokens[t] of table (n_vocab rows x k, GGUF layout)
 * for t < n_tokens; ids outside [0, n_vocab) give a row of zeros.  The
 * token-embedding lookup of the decode step, dequantize_row of row token_id
 * (cpp/src/fast_model.cpp:1042-1046), on the device for device token ids.
 * Bit-exact as vb_dequant_rows.  out: 16-byte aligned for block types. */
int vb_embed_rows(const void* table, int32_t ggml_type, int64_t n_vocab, int64_t k, const int32_t* tokens,
                  int64_t n_tokens, float* out, void* stream);

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
 * orientation (rows = outputs), as real .gguf tensors are stored.
 * Kernels: Q4_K, Q6_K and Q8_0 rows of whole 16-byte slots with k <= 4096
 * run the short-row kernel (one 64-element unit per lane, whole rows per
 * wave), 4096 < k <= 16384 the split-row kernel (rows in slices over 2-8
 * waves); other shapes and types the general kernel.  Activations are
 * encoded as 15- or 16-bit fixed point per unit or run (rel-L2 near 5e-5
 * against the fp64 product). */
int vb_gemv(const void* w, const float* x, float* y, int64_t n, int64_t k,
            int32_t ggml_type, void* stream);

/* ---- dequant-fused GEMM on MFMA ----------------------------------------
 * Y[m, n] = sum_k X[m, k] * W[n, k]; X row-major (m x k) in fp32
 * (x_dtype = 0) or fp16 (x_dtype = 1), Y fp32 row-major (m x n).  Products
 * run on v_mfma_f32_16x16x32_f16 with W dequantized to fp16 in registers and
 * fp32 accumulation.  variant: 0 = choose, 1 = skinny (m <= 32; m <= 64 with
 * fp16 X), 2 = tiled
 * (every type; Q6_K / Q8_0 need k % 256 == 0), 3 = role-split (fp16 X only),
 * 4 = K-split (every type).  Variant 0 for Q4_K: 1 at m <= 32 (m <= 64 for
 * fp16 X and n >= 8192), 2 above, with
 * 4 at 17 <= m <= 32 for fp32 X and n < 12288, and at n < 8192 for
 * 33 <= m <= 64 and (k >= 8192) 2 <= m <= 16; 3 at 257 <= m <= 768 for fp16
 * X and n >= 8192.  Q6_K / Q8_0: 4 up to m = 64 (at n < 8192: Q6_K up to
 * m = 256 with fp16 X, both up to 128 with fp32 X), 2 above.  Q5_K: 4 up to
 * m = 32 (64 at n < 8192), 2 above.  Variants 1 and 3 are Q4_K-only.  With variant 0 and
 * m == 1 the GEMV runs instead: vb_gemv's kernels for fp32 X (bit-identical
 * to vb_gemv), and for fp16 X the short-row kernels reading the halves
 * directly (Q4_K k <= 4096; Q6_K k = 2048 / 4096; Q8_0 k % 256 == 0 up to
 * 4096), and the split-row kernels for 4096 < k <= 16384 (the shapes vb_gemv
 * takes there); other fp16 cases stay on MFMA.
 * Replaces the reference's batched path, a per-token loop of gemv_dequant
 * (cpp/src/fast_model.cpp:644-669, :905-960) over rows decoded by
 * dequantize_row (cpp/src/dequant.cpp:407-425), and cuda::gemm_f32
 * (cpp/include/cuda_kernels.h, cpp/src/cuda_kernels.cu:184-212).
 * Weight types: Q4_K (variants 0-5), Q6_K and Q8_0 (variants 0, 2, 4, 5; Q8_0
 * needs k % 128 == 0 at every m, m == 1 included, although vb_gemv itself
 * takes Q8_0 rows of any whole number of blocks); Q5_K (variants 0, 2, 4, 5)
 * with its own decoder in each kernel; Q4_0, Q4_1, Q5_0, Q5_1 (variants 0,
 * 2, 4, 5) with their decoder in the K-split kernel (variant 4, k % 128 ==
 * 0; variant 0 up to m = 256 at n < 8192, 128 above), the tiled kernel
 * (variant 2; variant 0 between those ranges for Q4_0 / Q4_1) and the
 * packed-X kernel (variant 5; variant 0 above m = 256 where Q4_K takes it);
 * Q5_0 / Q5_1 between the ranges with variant 0, and Q2_K, Q3_K, BF16 and
 * F32 at every m (k % 256 == 0 except on the GEMV): decoded once to fp16
 * (each value rounded once) into n x k x 2 bytes of workspace and
 * multiplied on the tiled kernel; F16 on the tiled kernel in place.  vb_gemm allocates that
 * workspace on the stream for the call (stream-ordered), vb_gemm_ws takes
 * it from the caller.  W and x 16-byte aligned. */
int vb_gemm(const void* w, const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n,
            int64_t k, int32_t ggml_type, int32_t variant, void* stream);
/* vb_gemm with a caller-owned workspace, which lets variant 0 (and variant 5)
 * use the GEMM that needs one: 5 = X in registers (Q4_K, Q5_K, Q6_K, Q8_0,
 * Q4_0, Q4_1, Q5_0, Q5_1; fp16 X,
 * m >= 256, k % 256 == 0): a pack pass writes X into the workspace in MFMA
 * fragment order, then the MFMA waves load their A fragments from it
 * directly and only the dequantized weight tile goes through LDS.  Variant
 * 0 takes it for m > 256 where n >= 8192 or the output tiles are fewer than
 * the CUs (then K is split between workgroups; VB_GEMM_XR_KQ=0 keeps Q6_K /
 * Q8_0 on the tiled kernel, with its own K splits).  vb_gemm_workspace returns the
 * bytes variant `variant` needs for the shape (0: none, then vb_gemm_ws is
 * vb_gemm; the fp16 decode of the types without a fused decoder, n x k x 2,
 * at any x_dtype); the workspace must be 16-byte aligned.  Same reference path as
 * vb_gemm (cpp/src/fast_model.cpp:644-669, :905-960); the reference's
 * batched loop has no workspace (its scratch row is decoded per token). */
int64_t vb_gemm_workspace(int64_t m, int64_t n, int64_t k, int32_t ggml_type, int32_t x_dtype, int32_t variant);
int vb_gemm_ws(const void* w, const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n, int64_t k,
               int32_t ggml_type, int32_t variant, void* workspace, size_t workspace_bytes, void* stream);

/* ---- measurement utility ----------------------------------------------
 * Reads n rows of row_bytes (a multiple of 16, at most 4096) with the launch
 * shape and load pattern of the short-row Q4_K GEMV (one 8-wave workgroup
 * per CU slot, n / (CUs x 8) rows per wave, contiguous 16-byte
 * non-temporal pieces per row; `ring` rows loaded ahead of the row being
 * consumed into registers, as the register-ring GEMV's ring of 3; 0 = all
 * of a wave's rows at once; -1..-3 = 1..3 rows ahead landing in LDS by DMA,
 * as the default GEMV's DMA ring of 2) and computes nothing from them: the
 * time one launch
 * needs to read what the GEMV reads.  sink: 4 bytes of device memory the
 * kernel may write (it keeps the loads in the program).  No counterpart in
 * the reference: it exists for the bench's floor table. */
int vb_stream_read(const void* w, int64_t n, int64_t row_bytes, int32_t ring, uint32_t* sink, void* stream);

/* ---- TurboSparse activation-sparse FFN, one token ------------------------
 * y[h] = sum_{r < n_active} act(g_r, u_r) * Wd[:, active[r]] with
 * g_r = Wg[active[r], :] . x, u_r = Wu[active[r], :] . x; only the rows of
 * the active set are read from Wg / Wu.  active: sorted ascending, unique,
 * within [0, i) (indices outside are clamped, never dereferenced).
 * act_kind: 0 = silu(g) * u (vibeblade/sparse.py:269-272),
 *           1 = relu(g) * relu(u) (ReLU after both projections),
 *           2 = gelu_tanh(g) * u (GeGLU, cpp/src/fast_model.cpp:943-948).
 * down_layout: 0 = GGUF down, Wd is h rows x i (all of Wd is read);
 *              1 = neuron-major down, Wd holds W_down^T as i rows x h and
 *                  only the active rows are read (Q4_K only).
 * Wg / Wu: i rows x h.  Replaces sparse_ffn_silu's up / down steps
 * (vibeblade/sparse.py:261-276) and ffn_silu(sparse_mask=)
 * (vibeblade/transformer.py:177-208).  workspace: at least
 * vb_sparse_ffn_workspace(h, i, n_active, down_layout) bytes. */
int64_t vb_sparse_ffn_workspace(int64_t h, int64_t i, int32_t n_active, int32_t down_layout);
int vb_sparse_ffn(const void* wg, const void* wu, const void* wd, int32_t down_layout,
                  const float* x, const int32_t* active, int32_t n_active, int32_t act_kind,
                  float* y, int64_t h, int64_t i, int32_t ggml_type, void* workspace,
                  size_t workspace_bytes, void* stream);
/* vb_sparse_ffn without a workspace argument and without any allocation:
 * the workspace is a static 8 MiB device array per GPU (held until the
 * process ends), enough for config-4 shapes (h = 4096, i = 14336) up to
 * about 4096 active neurons on the fused path; shapes that need more
 * (vb_sparse_ffn_workspace above 8 MiB) return VB_E_INVAL with a message.
 * All calls on one GPU share the array: calls that overlap on one GPU (other
 * streams or threads) race.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). */
int vb_sparse_ffn_noalloc(const void* wg, const void* wu, const void* wd, int32_t down_layout,
                          const float* x, const int32_t* active, int32_t n_active, int32_t act_kind,
                          float* y, int64_t h, int64_t i, int32_t ggml_type, void* stream);
/* The TurboSparse FFN block: vb_sparse_ffn over n = x / sqrt(mean(x^2) +
 * eps) * norm_w (n = x when norm_w is NULL), plus x when add_residual != 0;
 * y may be x.  The sparse branch of the decoder layer with its pre-FFN
 * RMSNorm and residual (vibeblade/transformer.py:789-815 with
 * _sparse_ffn_layer :211-229; cpp/src/fast_model.cpp:837-840, :915-940,
 * :966-975).  The norm runs inside the gate/up encode and the residual in
 * the launch that writes y (neuron-major Q4_K, h <= 4096: 2 launches).
 * n_active_dev (optional): the active-set size as the device wrote it (an
 * on-device prediction, vb_ema_predict); n_active is then the host's bound
 * (launch sizes, workspace) and the kernels stop at the device count, so no
 * host round trip is needed.  Same workspace as vb_sparse_ffn for n_active;
 * x and norm_w 16-byte aligned. */
int vb_sparse_ffn_block(const void* wg, const void* wu, const void* wd, int32_t down_layout,
                        const float* x, const float* norm_w, float eps, const int32_t* active,
                        int32_t n_active, const int32_t* n_active_dev, int32_t act_kind, int32_t add_residual,
                        float* y, int64_t h, int64_t i, int32_t ggml_type, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ---- EMA neuron predictor on the device ------------------------------------
 * EMANeuronPredictor (vibeblade/sparse.py:431-650) with its per-layer state,
 * a probs vector of n fp32 per layer, in device memory.
 * vb_ema_update: probs = alpha * mask + (1 - alpha) * probs (update,
 * sparse.py:494-515); mask: n bytes, 0 or 1.  Rounded as the reference's
 * float32 numpy expression: bit-identical. */
int vb_ema_update(float* probs, int64_t n, const uint8_t* mask, double alpha, void* stream);
/* vb_ema_predict (predict, sparse.py:517-569; predict_combined :571-598):
 *   warm != 0 (the layer has more than 5 updates):
 *       {probs >= threshold}, topped up to k with the most probable neurons
 *       (= top-k(probs) | {probs >= threshold});
 *   warm == 0: top-k(gate_values) when given, else neurons 0 .. k-1;
 *   combined != 0: the prediction without gate values | top-k(gate_values).
 * Ties at a top-k threshold go to the lowest indices.  Writes mask_out (n
 * bytes), active_out (the selected indices ascending; room for n) and
 * count_out (1 int32), all on the device: feed active_out / count_out to
 * vb_sparse_ffn_block with n_active = n.  1 <= k <= n. */
int vb_ema_predict(const float* probs, const float* gate_values, int64_t n, int32_t k, float threshold,
                   int32_t warm, int32_t combined, uint8_t* mask_out, int32_t* active_out, int32_t* count_out,
                   void* stream);

/* ---- FFN block, one token ------------------------------------------------
 * y = [x +] Wd act(Wg n, Wu n), n = x / sqrt(mean(x^2) + eps) * norm_w
 * (n = x when norm_w is NULL; the x term when add_residual != 0).
 * act_kind: 0 = silu(g) * u, 1 = relu(g) * relu(u),
 *           2 = gelu_tanh(g) * u (GeGLU, cpp/src/fast_model.cpp:943-948).
 * Wg, Wu: inter rows x hd, one type (gate_up_type); Wd: hd rows x inter
 * (down_type); GGUF layout.  x, norm_w: hd fp32, 16-byte aligned; y: hd fp32,
 * may be x (in-place residual update).  Replaces the dense FFN step of the
 * decoder layer, RMSNorm -> gate/up -> act -> down -> residual
 * (cpp/src/fast_model.cpp:837-975; vibeblade/transformer.py:789-815 with
 * ffn_silu, :177-208).  Two launches when gate/up and down are Q4_K / Q6_K /
 * Q8_0 (norm and activation fused into the gate/up GEMV, residual into the
 * down GEMV); other type mixes run unfused, on the device.  workspace: at
 * least vb_ffn_block_workspace(hd, inter) bytes, 16-byte aligned. */
int64_t vb_ffn_block_workspace(int64_t hd, int64_t inter);
int vb_ffn_block(const float* x, const float* norm_w, float eps, const void* w_gate, const void* w_up,
                 int32_t gate_up_type, const void* w_down, int32_t down_type, int64_t hd, int64_t inter,
                 int32_t act_kind, int32_t add_residual, float* y, void* workspace, size_t workspace_bytes,
                 void* stream);

/* out_idx[0..k) = indices of the k largest v[i], ascending index order (ties
 * at the threshold resolve to the lowest indices).  The top-k neuron
 * prediction of sparse_ffn_silu (vibeblade/sparse.py:250-261) and
 * topk_activation_mask (:142-168), on the device. */
int vb_topk_indices(const float* v, int64_t n, int32_t k, int32_t* out_idx, void* stream);

/* ---- MoE expert-grouped FFN ---------------------------------------------
 * For each of n_tokens tokens: p = softmax(clamp(logits_t, -50, 50)), top-k
 * experts by p, weights renormalised to sum 1 (vibeblade/moe.py:170-206,
 * cpp/src/fast_model.cpp:534-548); y_t = sum_k w_tk *
 * Wd_e (silu(Wg_e x_t) * (Wu_e x_t)) with e = e_tk
 * (vibeblade/moe_executor.py:331-344, vibeblade/moe.py:457-482,
 * cpp/src/fast_model.cpp:552-572).  wg / wu / wd: host arrays of n_exp
 * device pointers; Wg_e, Wu_e: i rows x h, Wd_e: h rows x i (GGUF layout,
 * Q4_K, Q6_K, Q8_0, Q5_K, Q4_0, Q4_1, Q5_0 or Q5_1).  x: n_tokens x h fp32;
 * router_logits: n_tokens x n_exp fp32;
 * y: n_tokens x h fp32; out_idx / out_w (optional, may be NULL):
 * n_tokens x topk routing result.  Experts may also be F32 (same shapes).
 * Replaces HotColdExecutor.dispatch's
 * per-expert loop (vibeblade/moe_executor.py:139-329) and the engine's MoE
 * branch (cpp/src/fast_model.cpp:844-902).  Limits: n_exp <= 64,
 * topk <= 8, n_tokens * topk <= 1024.  workspace: at least
 * vb_moe_workspace(n_tokens, topk, h, i) bytes. */
int64_t vb_moe_workspace(int32_t n_tokens, int32_t topk, int64_t h, int64_t i);
int vb_moe_grouped_ffn(const void* const* wg, const void* const* wu, const void* const* wd,
                       int32_t n_exp, const float* x, int32_t n_tokens, const float* router_logits,
                       int32_t topk, float* y, int32_t* out_idx, float* out_w, int64_t h, int64_t i,
                       int32_t ggml_type, void* workspace, size_t workspace_bytes, void* stream);
/* vb_moe_grouped_ffn with the gate/up type and the down type given apart:
 * each Q4_K, Q6_K, Q8_0, Q5_K, Q4_0, Q4_1, Q5_0 or Q5_1 (or both F32), as a
 * GGUF MoE layer stores
 * ffn_gate_exps / ffn_up_exps and ffn_down_exps with their own types (the
 * engine's expert FFN, cpp/src/fast_model.cpp:552-572, takes each matrix with
 * its own type).  Same layout, limits and workspace as vb_moe_grouped_ffn,
 * which is this call with gate_up_type == down_type == ggml_type. */
int vb_moe_grouped_ffn_types(const void* const* wg, const void* const* wu, const void* const* wd,
                             int32_t n_exp, const float* x, int32_t n_tokens, const float* router_logits,
                             int32_t topk, float* y, int32_t* out_idx, float* out_w, int64_t h, int64_t i,
                             int32_t gate_up_type, int32_t down_type, void* workspace, size_t workspace_bytes,
                             void* stream);

/* Routing only: out_idx / out_w (n_tokens x topk) as vb_moe_grouped_ffn
 * computes them (ExpertRouter.route, vibeblade/moe.py:170-206, with the
 * selected experts ordered by descending weight). */
int vb_moe_route(const float* router_logits, int32_t n_tokens, int32_t n_exp, int32_t topk,
                 int32_t* out_idx, float* out_w, void* stream);

/* ---- elementwise ----------------------------------------------------------
 * y = silu(x) (kind 0) or max(x, 0) (kind 1); GPUBackend.silu / .drelu
 * (vibeblade/gpu.py:100-124). */
int vb_activation(const float* x, float* y, int64_t n, int32_t kind, void* stream);
/* y[r] = x[r] / sqrt(mean(x[r]^2) + eps) * w for rows x dim fp32
 * (GPUBackend.rms_norm, vibeblade/gpu.py:126-146). */
int vb_rms_norm(const float* x, const float* w, float* y, int64_t rows, int64_t dim, float eps,
                void* stream);
/* Row-wise softmax over rows x n fp32 (GPUBackend.softmax,
 * vibeblade/gpu.py:192-198). */
int vb_softmax(const float* x, float* y, int64_t rows, int64_t n, void* stream);

/* ---- GGUF ingestion --------------------------------------------------------
 * A .gguf file mapped read-only and parsed (header, metadata, tensor table).
 * Replaces GGUFFile (cpp/include/gguf.h:29-60, cpp/src/gguf.cpp) and the
 * parsing half of GGUFLoader (vibeblade/loader.py:490-783).  The data
 * section follows general.alignment when the file sets it (32 otherwise);
 * the reference always uses 32.  Host-side calls need no GPU; the handle
 * is read-only after vb_gguf_open and may be shared between threads. */
typedef struct vb_gguf vb_gguf;
/* GGUFFile::GGUFFile (gguf.h:30); errors (bad magic, version > 3, reads past
 * the end, unaligned or out-of-file tensor data, unknown types) return
 * E_INVAL with the reason in vb_last_error. */
int vb_gguf_open(const char* path, vb_gguf** out);
/* GGUFFile::~GGUFFile (gguf.h:31); unmaps the file.  NULL is accepted. */
int vb_gguf_close(vb_gguf* f);
/* version(), file_size() (gguf.h:58-59), plus the data alignment and the
 * absolute offset of the data section. */
int vb_gguf_info(const vb_gguf* f, uint32_t* version, uint64_t* alignment, uint64_t* data_offset,
                 uint64_t* file_size);
/* tensors() (gguf.h:55): count, lookup by name (-1 when absent, as
 * tensor_info returns nullptr, gguf.h:41), and one entry: name (valid until
 * vb_gguf_close), ggml type, dims (GGUF order, dims[0] along the row,
 * unused dims 1), absolute file offset and byte size of the data. */
int64_t vb_gguf_n_tensors(const vb_gguf* f);
int64_t vb_gguf_find_tensor(const vb_gguf* f, const char* name);
int vb_gguf_tensor_info(const vb_gguf* f, int64_t i, const char** name, int32_t* ggml_type, int32_t* n_dims,
                        int64_t* dims, uint64_t* offset, uint64_t* nbytes);
/* tensor_data (gguf.h:38): host pointer into the mapping. */
int vb_gguf_tensor_data(const vb_gguf* f, int64_t i, const void** host_ptr);
/* Copies tensor i's bytes (GGUF block layout, unchanged) to device memory
 * dst (at least nbytes) on `stream` through two pinned staging buffers;
 * returns when the copy has completed.  The buffers (min(8 MiB, largest
 * tensor) each) are made on the first upload and kept until vb_gguf_close;
 * uploads from one handle run one at a time. */
int vb_gguf_upload(const vb_gguf* f, int64_t i, void* dst, void* stream);
/* Metadata (meta_* accessors, gguf.h:44-52): count, lookup by key (-1 when
 * absent), the entry's key, value type (GGUF: 0 u8, 1 i8, 2 u16, 3 i16,
 * 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64),
 * array element type (-1 for scalars) and element count (1 for scalars),
 * then element j as an integer (integer and bool types), a double (f32,
 * f64) or a string (pointer into the mapping, not NUL-terminated, and its
 * length). */
int64_t vb_gguf_n_kv(const vb_gguf* f);
int64_t vb_gguf_find_kv(const vb_gguf* f, const char* key);
int vb_gguf_kv_info(const vb_gguf* f, int64_t i, const char** key, int32_t* value_type, int32_t* elem_type,
                    uint64_t* count);
int vb_gguf_kv_int(const vb_gguf* f, int64_t i, uint64_t j, int64_t* out);
int vb_gguf_kv_float(const vb_gguf* f, int64_t i, uint64_t j, double* out);
int vb_gguf_kv_str(const vb_gguf* f, int64_t i, uint64_t j, const char** s, uint64_t* len);

#ifdef __cplusplus
}
#endif

#endif /* VBHIP_H */
