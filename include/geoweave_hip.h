/*
 * geoweave_hip.h - C ABI of the MI355X (gfx950) sparse global-attention hot path.
 *
 * One shared library, libgeoweave_hip.so, exports these entry points. Every argument is
 * a plain pointer, size or scalar; no framework types cross the boundary.
 *
 * Conventions (all entry points):
 *  - Pointers are device pointers unless stated; outputs and workspaces are allocated by
 *    the caller (the reference allocates them with torch before each launch:
 *    easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:2061-2080,
 *    easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:1288-1297).
 *  - Strides are in elements; the innermost (head-dim) stride must be 1.
 *  - `stream` is a hipStream_t (NULL = default stream). Work is only enqueued on it; no
 *    entry point synchronises the host.
 *  - Return value: GW_OK or an error code; gw_last_error() then gives a message for the
 *    calling thread. The Python binding turns a non-zero code into RuntimeError, as the
 *    reference's TORCH_CHECK does (custom_indexer/csrc/topk_exact.cpp:12-35).
 *  - dtype: the attention entry points take GW_DTYPE_BF16 or GW_DTYPE_FP16 for q/k/v (the
 *    reference's attention accepts only fp16/bf16: sparse_index_flash_attn.py:2036; its
 *    caller casts fp32 to 16 bits first, dsa_attention.py:5296-5300). The indexer top-k,
 *    its backward and its view-bias gradient also take GW_DTYPE_FP32 (the reference's
 *    indexer computes in q.dtype, any float type: sparse_topk_indexer.py:1293, and its
 *    caller may cast to score_dtype float32: indexer.py:321-326).
 */
#ifndef GEOWEAVE_HIP_H
#define GEOWEAVE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GW_OK 0
#define GW_ERR_INVALID 1     /* bad shape, stride, pointer or size */
#define GW_ERR_UNSUPPORTED 2 /* valid request this build does not implement */
#define GW_ERR_HIP 3         /* a HIP runtime call failed */

#define GW_DTYPE_BF16 0
#define GW_DTYPE_FP16 1
#define GW_DTYPE_FP32 2 /* the indexer entry points and gw_indexer_kl_* only */

/* Message for the last failed call on this thread ("" if none). */
const char* gw_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int gw_abi_version(void);

/* ------------------------------------------------------------------------------------
 * Sparse-index attention, forward.
 *
 * Replaces _flash_attn_forward + _fwd_kernel + _attn_sum_kernel
 * (easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:2001-2233, :129-259,
 * :375-458), i.e. the compute behind sparse_index_flash_attn_func (:3286),
 * sparse_index_flash_attn_inference_func (:3138-3163) and their bhtd twins
 * (:3166-3193, :3370).
 *
 * For every (b, t, h): over the K candidates j with 0 <= kv_pos[b,t,j] < S,
 *   p_j = softmax_j(scale * q[b,t,h] . k[b,pos_j,h]),  o[b,t,h] = sum_j p_j v[b,pos_j,h].
 * Candidates outside [0, S) are masked (sparse_index_flash_attn.py:207-218). A row with
 * no valid candidate gets o = 0, lse = -inf.
 *
 * q/o index (b, t, h, d); k/v index (b, s, h, d); *_strides = {stride_b, stride_t|s,
 * stride_h}. Both the bthd and the bhtd layouts are expressed through the strides.
 * kv_pos: int32, element (b,t,j) at b*pos_stride_b + t*pos_stride_t + j.
 * lse (nullable): fp32 [B, T, H] contiguous, natural-log log-sum-exp of the scaled scores.
 * attn_sum (nullable): fp32 [B, T, K] contiguous, attn_sum[b,t,j] = sum_h p_j (the
 *   reference's atomic sum over heads, :375-458; here written once, no atomics).
 * workspace: gw_sparse_attn_fwd_workspace_size(...) bytes (0 when attn_sum is NULL).
 * Supported: D in {64, 128}; any H >= 1; K >= 1; dtype bf16/fp16.
 */
size_t gw_sparse_attn_fwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K,
                                         int want_attn_sum);
int gw_sparse_attn_fwd(int dtype,
                       const void* q, const int64_t* q_strides,
                       const void* k, const int64_t* k_strides,
                       const void* v, const int64_t* v_strides,
                       const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                       void* o, const int64_t* o_strides,
                       float* lse, float* attn_sum,
                       int64_t B, int64_t T, int64_t S, int64_t H, int64_t D, int64_t K,
                       float softmax_scale,
                       void* workspace, size_t workspace_bytes,
                       void* stream);

/* ------------------------------------------------------------------------------------
 * Lightning-indexer score + exact top-k, forward.
 *
 * Replaces SparseTopkIndexerFunc.forward -> _blockwise_topk_scores(_impl)
 * (easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:2047-2088, :1779-1844,
 * :1241-1776) and the opt-in CUDA kernels it can call (custom_indexer/csrc/
 * score_topk_fused_kernel.cu:53-224, topk_exact_kernel.cu:26-149,
 * merge_two_topk_kernel.cu:25-142), i.e. the compute behind sparse_topk_indexer_func
 * (:2188-2253).
 *
 *   score[b,t,s] = sum_h w[b,s,h] * relu(softmax_scale * q[b,t,h,:] . k[b,s,h,:])
 *                  (+ mask[b,t,s] when mask != NULL)
 * out_indices[b,t,:] (int32) = the Kk = min(topk, S) keys with the largest scores, in
 * unspecified order (the reference uses sorted=False); out_scores (same dtype as q) = their
 * scores. Exact: the set equals the fp32 top-k except where scores tie within rounding;
 * ties are broken deterministically. Scores are accumulated in fp32 (bf16/fp16 products
 * are exact in fp32; fp32 inputs use fp32 matrix-core products).
 *
 * q: [B,T,Hi,Di], k: [B,S,Hi,Di], w: [B,S,Hi], mask: [B,T,S], all contiguous, same dtype
 * (bf16, fp16 or fp32). Supported: Di = 64, Hi in {1,2,4,8} ({1,2,4} for fp32),
 * any topk >= 1 (K = min(topk, S); a K whose expected candidates exceed 3/4 of the 8192
 * candidate slots per query scores every row over every key on the matrix cores and selects
 * it exactly, in rounds of up to 2,048 rows per batch element), softmax_scale > 0.
 * workspace: gw_indexer_topk_workspace_size(B, T, S, topk) bytes, 16-byte aligned.
 * flags: 0 normally. Test hooks that force the exact fallback paths:
 *   GW_TOPK_FLAG_TAU_PLUS_INF  - no key passes the candidate filter (every query falls
 *                                back to the brute-force path);
 *   GW_TOPK_FLAG_TAU_MINUS_INF - every key passes (the per-query candidate lists overflow
 *                                once S exceeds their 8192 slots: brute force again);
 *   GW_TOPK_FLAG_FORCE_WIDE    - every query with complete candidates is selected by the
 *                                LDS path meant for rows the register path cannot hold.
 */
#define GW_TOPK_FLAG_TAU_PLUS_INF 1
#define GW_TOPK_FLAG_TAU_MINUS_INF 2
#define GW_TOPK_FLAG_FORCE_WIDE 4

size_t gw_indexer_topk_workspace_size(int64_t B, int64_t T, int64_t S, int64_t topk);
int gw_indexer_topk_fwd(int dtype, const void* q, const void* k, const void* w, const void* mask,
                        int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di, int64_t topk,
                        float softmax_scale, int flags,
                        int32_t* out_indices, void* out_scores,
                        void* workspace, size_t workspace_bytes,
                        void* stream);

/* The same top-k with the soft view bias added to every score (replaces
 * SparseTopkIndexerViewBiasFunc.forward, easyvolcap/utils/custom_indexer/
 * sparse_topk_indexer.py:2108-2157, whose _blockwise_topk_scores adds the term after the
 * mask, :935-951; the bias itself is indexer.py:509-519):
 *   score[b,t,s] = ... (+ mask[b,t,s]) + view_bias[b, q_view_ids[b,t], s_view_ids[b,s]]
 * view_bias: [B, Vq, Vs] contiguous, in q's dtype; q_view_ids [B, T] and s_view_ids [B, S]
 * int32, in [0, Vq) and [0, Vs) (ids outside are clamped into the table). Other arguments
 * and the workspace as gw_indexer_topk_fwd.
 */
int gw_indexer_topk_fwd_view_bias(int dtype, const void* q, const void* k, const void* w, const void* mask,
                                  const void* view_bias, const int32_t* q_view_ids,
                                  const int32_t* s_view_ids, int64_t Vq, int64_t Vs,
                                  int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di, int64_t topk,
                                  float softmax_scale, int flags,
                                  int32_t* out_indices, void* out_scores,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);

/* ------------------------------------------------------------------------------------
 * Key-major (CSR) transpose of a [B, T, K] position table, shared by both backward
 * passes below (the attention's kv_positions and the indexer's topk_indices are the
 * same table in a DSA layer, so one build serves both).
 *
 * Replaces the reference's key grouping of the opt-in grouped backward (device radix
 * sort + run-length encoding + scan, custom_flash_attn/csrc/sparse_bwd_grouped_kernel.cu:
 * 232-269, 432-570), and stands in for the fp32 atomics of the default backward
 * (sparse_index_flash_attn.py:739-740, sparse_topk_indexer.py:1936-1941).
 *
 * pos: int32, element (b,t,j) at b*pos_stride_b + t*pos_stride_t + j. Entries outside
 * [0, S) are skipped. csr: a caller-allocated buffer of gw_kv_csr_size(B,T,S,K) bytes,
 * 16-byte aligned, opaque (per-key offsets and work items, and the (t, j) entries: about
 * 8 bytes per table entry); it stays valid until the buffer is reused. workspace: the
 * build's transient buffer of gw_kv_csr_build_workspace_size(B,T,S,K) bytes (the radix
 * sort's ping-pong buffers, about 16 bytes per table entry), 16-byte aligned; it may be
 * reused once the work queued on `stream` by this call has run. The entries of each key are
 * sorted by (t, j), so results computed from the table are bitwise reproducible. Work runs
 * on `stream`; no host synchronisation.
 */
size_t gw_kv_csr_size(int64_t B, int64_t T, int64_t S, int64_t K);
size_t gw_kv_csr_build_workspace_size(int64_t B, int64_t T, int64_t S, int64_t K);
int gw_kv_csr_build(const int32_t* pos, int64_t pos_stride_b, int64_t pos_stride_t,
                    int64_t B, int64_t T, int64_t S, int64_t K,
                    void* csr, size_t csr_bytes, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ------------------------------------------------------------------------------------
 * Sparse-index attention, backward.
 *
 * Replaces _sparse_index_flash_attn_backward -> _bwd_preprocess_do_o_dot +
 * _bwd_sparse_index_kernel (easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:
 * 2442-2846, :534-576, :579-743) behind SparseIndexFlashAttnFunc.backward (:3240-3283)
 * and its bhtd twin, and the opt-in grouped CUDA backward
 * (custom_flash_attn/csrc/sparse_bwd_grouped_kernel.cu:79-603).
 *
 * Inputs are the forward's: q/k/v/o (strides as in gw_sparse_attn_fwd), kv_pos, lse
 * (fp32 [B,T,H] from gw_sparse_attn_fwd), dout (dO, same dtype, strided like q).
 * dattn_sum (nullable): gradient of attn_sum, [B,T,K] contiguous in the q dtype (the
 * reference casts it to q.dtype, :3244-3245). Outputs dq (strided like q), dk, dv
 * (strided like k, v) in the input dtype, accumulated in fp32 with no atomics; every
 * element of dk/dv is written (keys never selected get 0). csr: built by
 * gw_kv_csr_build from the same kv_pos, B, T, S, K. workspace:
 * gw_sparse_attn_bwd_workspace_size(...) bytes, 16-byte aligned.
 */
size_t gw_sparse_attn_bwd_workspace_size(int64_t B, int64_t T, int64_t S, int64_t H, int64_t D,
                                         int64_t K);
int gw_sparse_attn_bwd(int dtype,
                       const void* q, const int64_t* q_strides,
                       const void* k, const int64_t* k_strides,
                       const void* v, const int64_t* v_strides,
                       const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                       const void* o, const int64_t* o_strides,
                       const void* dout, const int64_t* do_strides,
                       const float* lse, const void* dattn_sum,
                       void* dq, const int64_t* dq_strides,
                       void* dk, const int64_t* dk_strides,
                       void* dv, const int64_t* dv_strides,
                       int64_t B, int64_t T, int64_t S, int64_t H, int64_t D, int64_t K,
                       float softmax_scale,
                       const void* csr, size_t csr_bytes,
                       void* workspace, size_t workspace_bytes,
                       void* stream);

/* ------------------------------------------------------------------------------------
 * Lightning-indexer top-k, backward.
 *
 * Replaces SparseTopkIndexerFunc.backward -> _backward_selected_topk_qkw ->
 * _indexer_topk_bwd_kernel (easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:
 * 2091-2106, :757-895, :1847-1944). For every selected (t, j), s = topk_indices[b,t,j],
 * g = grad_scores[b,t,j], per head h: z = scale * q[t,h].k[s,h];
 * f = g * w[s,h] * [z > 0] * scale; dq[t,h] += f k[s,h]; dk[s,h] += f q[t,h];
 * dw[s,h] += g relu(z). q/k/w/grad contiguous in one dtype (bf16, fp16 or fp32); outputs
 * dq, dk, dw in that dtype, accumulated in fp32 with no atomics; every element is written.
 * csr: built by gw_kv_csr_build from topk_indices (strides K*T, K). Supported: Di = 64,
 * Hi in {1,2,4,8}. workspace: gw_indexer_topk_bwd_workspace_size(...) bytes.
 */
size_t gw_indexer_topk_bwd_workspace_size(int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di,
                                          int64_t K);
int gw_indexer_topk_bwd(int dtype, const void* q, const void* k, const void* w,
                        const int32_t* topk_indices, const void* grad_scores,
                        void* dq, void* dk, void* dw,
                        int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di, int64_t K,
                        float softmax_scale,
                        const void* csr, size_t csr_bytes,
                        void* workspace, size_t workspace_bytes,
                        void* stream);

/* The same backward as masked dense passes on the matrix cores (bf16, Di = 64, Hi in
 * {1,2,4,8}, S <= 65536, K <= 2048; other inputs return GW_ERR_UNSUPPORTED). Every (query,
 * key) pair of a head is computed: z = q.k on the matrix cores, the gradients of the
 * selected pairs enter as a tile gathered from the row's gradients in key order, and
 * dq = scale F (w o k), dk = scale w o (F^T q), dw_s = scale k_s . (F^T q)_s with
 * F = g [z > 0]; fp32 accumulation in a fixed order (no atomics). Replaces the same
 * reference kernel as gw_indexer_topk_bwd (sparse_topk_indexer.py:1847-1944) for layers
 * where a query selects a sizable share of the keys; needs no CSR.
 * route: B device ints, cleared here; route[b] is set when batch element b has a position
 * listed twice in a row (the reference counts it twice) or a non-finite q, k, w or w k (it
 * would reach unselected pairs). Such elements are left untouched: compute them with
 * gw_indexer_topk_bwd. Every element of dq/dk/dw of the other batch elements is written.
 * q/k/w/grad_scores/topk_indices contiguous. workspace:
 * gw_indexer_topk_bwd_dense_workspace_size(...) bytes, 16-byte aligned (selection words and
 * prefixes, 6 * B * round_up(S, 32) / 32 * round_up(T, 32) bytes; gradients in key order,
 * 2 * B * T * K bytes; q^T and (w o k)^T, 2 * B * Hi * 64 * (round_up(T, 32) +
 * round_up(S, 32)) bytes; stream-K partials, 128 KiB per persistent workgroup).
 */
size_t gw_indexer_topk_bwd_dense_workspace_size(int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di,
                                                int64_t K);
int gw_indexer_topk_bwd_dense(int dtype, const void* q, const void* k, const void* w,
                              const int32_t* topk_indices, const void* grad_scores,
                              void* dq, void* dk, void* dw,
                              int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di, int64_t K,
                              float softmax_scale, int* route,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/* Soft view-bias gradient, per query row: the first half of _scatter_view_bias_grad
 * (easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:898-932, called from
 * SparseTopkIndexerViewBiasFunc.backward, :2159-2186). row_grad[b,t,v] (fp32 [B, T, Vs]) =
 * sum of grad_scores[b,t,j] over the j whose key s = topk_indices[b,t,j] has
 * s_view_ids[b,s] == v, summed in a fixed order (no atomics); positions outside [0, S) add
 * nothing. grad_view_bias[b, vq, v] is then the sum of row_grad[b,t,v] over the rows with
 * q_view_ids[b,t] == vq (the host's one-hot product). grad_scores: [B, T, K] in bf16, fp16
 * or fp32; s_view_ids: [B, S] int32.
 */
int gw_indexer_view_bias_bwd_rows(int dtype, const int32_t* topk_indices, const void* grad_scores,
                                  const int32_t* s_view_ids, int64_t B, int64_t T, int64_t S, int64_t K,
                                  int64_t Vs, float* row_grad, void* stream);

/* ------------------------------------------------------------------------------------
 * Indexer KL training loss, forward and backward.
 *
 * Replaces sparse_indexer_kl_loss / _SparseIndexerKLLossFunc
 * (easyvolcap/utils/custom_indexer/indexer_kl_fused.py:164-298: _kl_stats_kernel +
 * _kl_row_loss_kernel forward, _kl_row_bwd_kernel backward), the fused form of the loss
 * the DSA layer computes at easyvolcap/official_vggt/layers/dsa_attention.py:4688-4715.
 * attn_sum and logits: contiguous [rows, K] in one dtype (bf16, fp16 or fp32; the
 * reference casts logits to attn_sum's dtype, indexer_kl_fused.py:171-172); math in fp32.
 * Per row: p = attn / (sum attn + eps), lq = log_softmax(logits),
 * row_loss[r] = sum_j p_j (log(p_j + eps) - lq_j) (fp32). The loss is mean(row_loss).
 * Backward: grad_out is a device fp32 scalar dL/dloss (read on the device: no host
 * synchronisation, where the reference calls .item(), indexer_kl_fused.py:252);
 * d_attn, d_logits: [rows, K] in the input dtype. K <= 4096.
 */
int gw_indexer_kl_fwd(int dtype, const void* attn_sum, const void* logits, int64_t rows, int64_t K,
                      float eps, float* row_loss, void* stream);
int gw_indexer_kl_bwd(int dtype, const void* attn_sum, const void* logits, const float* grad_out,
                      int64_t rows, int64_t K, float eps, void* d_attn, void* d_logits,
                      void* stream);

/* ------------------------------------------------------------------------------------
 * DSA layer glue, forward: per-head LayerNorm + 2D RoPE + 16-bit cast of the attention
 * q/k and the indexer q/k/w, read from one fused projection output.
 *
 * Replaces the torch glue of DSAAttention._project_qkv_and_indexer_fused
 * (easyvolcap/official_vggt/layers/dsa_attention.py:583-625) plus :4928-4948 (q_norm,
 * k_norm, rope, score_dtype cast) and LightningIndexer.project
 * (easyvolcap/official_vggt/layers/indexer.py:302-328), with RotaryPositionEmbedding2D
 * (easyvolcap/official_vggt/layers/rope.py:62-200).
 * y: [rows, ldy] (dtype) = x W^T + b with W = [qkv | indexer q | indexer k | indexer w];
 * the *_off arguments are column offsets (multiples of 8, ldy % 8 == 0); the v block is
 * not touched (read it in place through strides). D = 64. LayerNorm weight/bias pairs are
 * fp32 [64] or both NULL (identity), eps ln_eps. pos: int32 [rows, 2] (y, x) or NULL (no
 * rope); rope_cos/rope_sin: fp32 [rope_len, 16] tables cos/sin(p * base^(-2i/32)), as
 * rope.py:86-117 builds them. Outputs (dtype, contiguous): q_out, k_out [rows, H, 64],
 * idx_q_out, idx_k_out [rows, Hi, 64], idx_w_out [rows, Hi]. Hi = 0 (a dense attention
 * layer's q/k glue, easyvolcap/official_vggt/layers/attention.py:70-85) is allowed; the
 * idx_* outputs may then be NULL.
 */
int gw_dsa_glue_fwd(int dtype, const void* y, int64_t rows, int64_t ldy, int64_t q_off, int64_t k_off,
                    int64_t iq_off, int64_t ik_off, int64_t iw_off, int64_t H, int64_t Hi, int64_t D,
                    const float* q_norm_w, const float* q_norm_b, const float* k_norm_w,
                    const float* k_norm_b, const float* idx_k_norm_w, const float* idx_k_norm_b,
                    float ln_eps, const int32_t* pos, const float* rope_cos, const float* rope_sin,
                    int64_t rope_len, void* q_out, void* k_out, void* idx_q_out, void* idx_k_out,
                    void* idx_w_out, void* stream);

/* ------------------------------------------------------------------------------------
 * DSA layer glue, backward (training through the layer).
 *
 * Gradient of gw_dsa_glue_fwd, i.e. of the reference's q_norm/k_norm + rope + cast glue
 * (dsa_attention.py:4928-4948, indexer.py:302-328; autograd of those torch ops in the
 * reference). Inputs: the forward's arguments (y, layout, LayerNorm parameters, positions,
 * rope tables) and the output gradients dq, dk [rows, H, 64], d_idx_q, d_idx_k
 * [rows, Hi, 64], d_idx_w [rows, Hi] (dtype, contiguous). Writes dy [rows, ldy] (dtype) in
 * the q, k, indexer q/k/w column blocks only (the v block and the padding are not written:
 * the caller zero-fills them or adds the attention's dv there), and d_norm fp32 [3][2][64]
 * = (d weight, d bias) of (q_norm, k_norm, indexer k_norm), summed over all rows and heads
 * in a fixed order (bitwise reproducible). workspace: gw_dsa_glue_bwd_workspace_size bytes.
 */
size_t gw_dsa_glue_bwd_workspace_size(int64_t rows, int64_t H, int64_t Hi);
int gw_dsa_glue_bwd(int dtype, const void* y, int64_t rows, int64_t ldy, int64_t q_off, int64_t k_off,
                    int64_t iq_off, int64_t ik_off, int64_t iw_off, int64_t H, int64_t Hi, int64_t D,
                    const float* q_norm_w, const float* q_norm_b, const float* k_norm_w,
                    const float* k_norm_b, const float* idx_k_norm_w, const float* idx_k_norm_b,
                    float ln_eps, const int32_t* pos, const float* rope_cos, const float* rope_sin,
                    int64_t rope_len, const void* dq, const void* dk, const void* d_idx_q,
                    const void* d_idx_k, const void* d_idx_w, void* dy, float* d_norm,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------
 * Sparse-index attention forward with the indexer KL loss fused into the attn_sum epilogue
 * (training). Same arguments and outputs as gw_sparse_attn_fwd (attn_sum required), plus:
 * logits [B, T, K] of logits_dtype (GW_DTYPE_BF16/FP16/FP32; element (b,t,j) at
 * b*logits_stride_b + t*logits_stride_t + j) - the indexer's top-k scores aligned with
 * kv_pos - and row_loss fp32 [B*T] (contiguous):
 *   row_loss[b*T+t] = sum_j p_j (log(p_j + eps) - log_softmax(z)_j),
 *   p = attn_sum[b,t,:] / (sum_j attn_sum[b,t,j] + eps),  z = logits[b,t,:] in fp32,
 * i.e. gw_indexer_kl_fwd on (attn_sum, logits cast to fp32), the per-row loss of
 * sparse_indexer_kl_loss (easyvolcap/utils/custom_indexer/indexer_kl_fused.py:8-155) with
 * the attention mass as p (easyvolcap/official_vggt/layers/dsa_attention.py:5404-5411),
 * computed while the row is still on chip. Supported: K <= 1024 per head group (a group
 * is 8 heads at D = 64, 4 at D = 128: K <= 2048 at H = 16, D = 64). The backward is
 * gw_indexer_kl_bwd + gw_sparse_attn_bwd.
 */
int gw_sparse_attn_fwd_kl(int dtype,
                          const void* q, const int64_t* q_strides,
                          const void* k, const int64_t* k_strides,
                          const void* v, const int64_t* v_strides,
                          const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                          void* o, const int64_t* o_strides,
                          float* lse, float* attn_sum,
                          int64_t B, int64_t T, int64_t S, int64_t H, int64_t D, int64_t K,
                          float softmax_scale,
                          const void* logits, int logits_dtype, int64_t logits_stride_b,
                          int64_t logits_stride_t, float eps, float* row_loss,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/* ------------------------------------------------------------------------------------
 * Source-downsample coarse selector (inference only, off unless requested): the device
 * steps around an indexer top-k over pooled source rows. Replaces the torch pooling of
 * DSAAttention._prepare_source_downsample_projected, the torch expansion of
 * _expand_source_downsample_chunk and the torch selection of the other strategies
 * (easyvolcap/official_vggt/layers/dsa_attention.py:3386-3542, :4079-4186, :3554-4078;
 * dispatch :4187-4260).
 *
 * source_to_fine: int32 [L, M], the fine tokens (< S) each source row covers, -1 past
 * the row's count (built on the host from the view/grid layout, :3069-3259).
 *
 * gw_source_downsample_pool: source_k [B, L, Hi, Di] and source_w [B, L, Hi] (dtype,
 *   contiguous) = the mean of each row's fine rows of k [B, S, Hi, Di] and w [B, S, Hi]
 *   (contiguous): fp32 sum in listed order / count, rounded once (F.avg_pool2d over a cell,
 *   or the mean of its representative points; special and edge rows are copies). With
 *   round_sum != 0 the sum is rounded to the dtype before the division, as the reference's
 *   query mean does (gathered.sum(dim=2) / denom, :3976-3983). w and source_w may both be
 *   null (queries have no gate). Supported: Hi <= 8, Hi * Di a multiple of 8.
 * gw_source_downsample_expand: out int32 [B, T_out, target] (contiguous) from the chosen
 *   source rows coarse_idx [B, T, Kc] (element (b,t,c) at b*idx_stride_b + t*idx_stride_t
 *   + c) taken in their given order or, when coarse_scores (dtype, same layout) is given,
 *   by score descending and row index ascending on ties (the reference's order is that of
 *   an unsorted torch.topk, i.e. unspecified; Kc <= 4096 then): round_robin != 0 lists the
 *   m-th token of every chosen row for m = 0, 1, ... (full cells), else row by row;
 *   invalid slots are skipped and the list is cut to target; a query with fewer valid
 *   tokens repeats its last min(count, pad_window) tokens cyclically, or gets -1
 *   everywhere if it has none. The table of batch element b starts at source_to_fine +
 *   b * table_stride_b (0: one table; the per-batch tables of subcell_static_pack4,
 *   _expand_source_downsample_chunk_batched :4129-4186). row_map (int32 [T_out], or null
 *   for T_out = T) makes output row t read chosen row row_map[t]: the broadcast of a
 *   coarse query's selection to its fine queries (qk_sym_x2_broadcast, :3999-4017).
 *   Supported: target <= 4096.
 * gw_source_downsample_rerank (exact_rerank, _select_source_downsample_exact_rerank
 *   :3599-3635 with _score_source_downsample_candidates :3554-3597): for every query q
 *   [B, T, Hi, Di] the fine tokens of its chosen rows (row-major over (chosen row, slot))
 *   are scored against k [B, S, Hi, Di] / w [B, S, Hi] with the indexer formula in fp32,
 *   and out int32 [B, T, target] receives the top target of them (ties in candidate order;
 *   tokens > kth first, then those equal to it). A query with fewer valid candidates than
 *   target sets *fail (a device int the caller clears; its out row is then unspecified):
 *   the reference then retries the chunk with a larger coarse budget. Supported: Hi <= 8,
 *   Di a multiple of 8, Hi * Di <= 1024, Kc * M <= 8192.
 * gw_source_downsample_subcell_top1 (_select_source_downsample_subcell_top1 :3629-3812):
 *   chosen rows (coarse_idx + coarse_scores, expanded by score descending) that are
 *   special/edge rows (< first_cell_row) give their token; the rest of the target,
 *   ceil((target - singles) / W) sub-cells at most (and at most those of the chosen
 *   cells), goes to the best-scoring sub-cells of the chosen cells, scored against the
 *   pooled sub-cell keys sub_k [B, C * G, Hi, Di] / sub_w [B, C * G, Hi] (cell c = row
 *   first_cell_row + c; subcell_to_fine int32 [C * G, W] their tokens). out [B, T,
 *   target]: the singles in order, then the kept sub-cells' tokens in (cell order,
 *   sub-cell) order, cut to target; *fail as above. Supported: Kc <= 2048, Kc * G <= 8192.
 * gw_source_downsample_static_pack4 (subcell_static_pack4 table, :3521-3542): table int32
 *   [B, L, W]: rows below first_cell_row keep their token (source_to_fine[r, 0]); cell c
 *   lists the tokens of its sub-cell with the largest head-mean of sub_w [B, C * G, Hi]
 *   (fp32 sum times 1 / Hi, rounded to the dtype; the first on ties).
 */
int gw_source_downsample_pool(int dtype, const void* k, const void* w, int64_t B, int64_t S, int64_t Hi,
                              int64_t Di, const int32_t* source_to_fine, int64_t L, int64_t M, int round_sum,
                              void* source_k, void* source_w, void* stream);
int gw_source_downsample_expand(int dtype, const int32_t* coarse_idx, const void* coarse_scores,
                                int64_t idx_stride_b, int64_t idx_stride_t,
                                int64_t B, int64_t T, int64_t Kc, const int32_t* source_to_fine,
                                int64_t table_stride_b, int64_t L, int64_t M, int round_robin, int64_t target,
                                int64_t pad_window, const int32_t* row_map, int64_t T_out, int32_t* out,
                                void* stream);
int gw_source_downsample_rerank(int dtype, const void* q, const void* k, const void* w, int64_t B, int64_t T,
                                int64_t S, int64_t Hi, int64_t Di, const int32_t* coarse_idx, int64_t idx_stride_b,
                                int64_t idx_stride_t, int64_t Kc, const int32_t* source_to_fine, int64_t L,
                                int64_t M, int64_t target, float scale, int32_t* out, int* fail, void* stream);
int gw_source_downsample_subcell_top1(int dtype, const void* q, const void* sub_k, const void* sub_w, int64_t B,
                                      int64_t T, int64_t C, int64_t G, int64_t Hi, int64_t Di,
                                      const int32_t* coarse_idx, const void* coarse_scores, int64_t idx_stride_b,
                                      int64_t idx_stride_t, int64_t Kc, const int32_t* source_to_fine, int64_t L,
                                      int64_t M, int64_t first_cell_row, const int32_t* subcell_to_fine, int64_t W,
                                      int64_t target, float scale, int32_t* out, int* fail, void* stream);
int gw_source_downsample_static_pack4(int dtype, const void* sub_w, int64_t B, int64_t C, int64_t G, int64_t Hi,
                                      const int32_t* source_to_fine, int64_t L, int64_t M, int64_t first_cell_row,
                                      const int32_t* subcell_to_fine, int64_t W, int32_t* table, void* stream);

/* ------------------------------------------------------------------------------------
 * Sparse-index attention forward as a masked dense pass: the same results as
 * gw_sparse_attn_fwd / gw_sparse_attn_fwd_kl (o, lse, attn_sum and the KL row losses, up to
 * fp32 summation order), computed by matrix-core products over every (query, key) pair with
 * the selection as a mask. Replaces the same reference compute (_flash_attn_forward +
 * _fwd_kernel + _attn_sum_kernel, easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:
 * 2001-2233, :129-259, :375-458, as reached from sparse_index_flash_attn_func :3286 and
 * sparse_index_flash_attn_inference_func :3138-3163; the fused KL as in gw_sparse_attn_fwd_kl);
 * it pays off when a query selects more than roughly 1 % of the keys.
 * Needs D = 64 and a positive softmax_scale, and K <= 1024 and H <= 64 when attn_sum is
 * asked for; the kernels' 32-bit load offsets also need a K token stride below 2^23 elements
 * and S <= 2^25 - 128, and its grid T <= 65528 * 32. Otherwise GW_ERR_UNSUPPORTED (use gw_sparse_attn_fwd /
 * gw_sparse_attn_fwd_kl).
 * The P·V product takes P in fp16 (the fp32 weights rounded to nearest, 11 significant bits)
 * against V in fp16 scaled per (head, d) column by an exact power of two; row sums and lse
 * come from the fp32 weights. A batch element whose K or V holds an inf or nan anywhere is
 * computed by the gather kernel inside this call (the dense products would carry the value
 * from rows a query did not select; the reference reads only the selected rows).
 * attn_sum (nullable) and lse: as for gw_sparse_attn_fwd (lse is required with attn_sum).
 * logits (nullable; needs attn_sum) ... row_loss: the fused KL loss, as for
 * gw_sparse_attn_fwd_kl.
 * Queries that list a position twice are computed by the gather kernel inside this call
 * (the reference counts a repeated position twice).
 * Workspace: gw_sparse_attn_fwd_dense_workspace_size(B, T, S, H, D, K, want_attn_sum) bytes,
 * 16-byte aligned: the selection words (B * round_up(S, 128) / 32 * round_up(T, 256) * 4
 * bytes), per-block and per-batch-element flags, the |V| column maxima (B * H * 64 * 4 bytes), the scaled fp16
 * V^T (B * H * 64 * round_up(S, 128) * 2 bytes) and, with attn_sum, the selected scores
 * (B * T * (round_up(K, 8) + 8) * H * 4 bytes).
 * ------------------------------------------------------------------------------------ */
size_t gw_sparse_attn_fwd_dense_workspace_size(int64_t B, int64_t T, int64_t S, int64_t H, int64_t D,
                                               int64_t K, int want_attn_sum);
int gw_sparse_attn_fwd_dense(int dtype,
                             const void* q, const int64_t* q_strides,
                             const void* k, const int64_t* k_strides,
                             const void* v, const int64_t* v_strides,
                             const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                             void* o, const int64_t* o_strides, float* lse, float* attn_sum,
                             int64_t B, int64_t T, int64_t S, int64_t H, int64_t D, int64_t K,
                             float softmax_scale,
                             const void* logits, int logits_dtype, int64_t logits_stride_b,
                             int64_t logits_stride_t, float eps, float* row_loss,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

/* ------------------------------------------------------------------------------------
 * Allocation-free variant of gw_sparse_attn_fwd_dense. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments and results as
 * gw_sparse_attn_fwd_dense without the workspace: the workspace is a file-scope device
 * array of gw_sparse_attn_fwd_dense_noalloc_capacity() bytes (64 MiB) that a GPU holds
 * from this entry point's first call on it until the process ends (processes that never
 * call it hold none). A call whose
 * gw_sparse_attn_fwd_dense_workspace_size(...) exceeds it returns GW_ERR_UNSUPPORTED (for
 * example the inference forward, no attn_sum, of 16 heads fits up to about 10 views of 1,374
 * tokens). Works on the current device; the first call on a device looks up the array's
 * address there. Calls that overlap on one GPU (other streams, other host threads) race on
 * the array: serialise them. Calls no hipMalloc/hipFree or allocating library routine.
 * ------------------------------------------------------------------------------------ */
size_t gw_sparse_attn_fwd_dense_noalloc_capacity(void);
int gw_sparse_attn_fwd_dense_noalloc(int dtype,
                                     const void* q, const int64_t* q_strides,
                                     const void* k, const int64_t* k_strides,
                                     const void* v, const int64_t* v_strides,
                                     const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                                     void* o, const int64_t* o_strides, float* lse, float* attn_sum,
                                     int64_t B, int64_t T, int64_t S, int64_t H, int64_t D, int64_t K,
                                     float softmax_scale,
                                     const void* logits, int logits_dtype, int64_t logits_stride_b,
                                     int64_t logits_stride_t, float eps, float* row_loss,
                                     void* stream);

/* ------------------------------------------------------------------------------------
 * Sparse-index attention backward as masked dense passes: the same gradients as
 * gw_sparse_attn_bwd without an attn_sum gradient (dq, dk, dv up to fp32 summation order and
 * the rounding of P and dS to the input type for their matrix products), computed on the
 * matrix cores over every (query, key) pair with the selection as a mask. Replaces the same
 * reference compute as gw_sparse_attn_bwd (_sparse_index_flash_attn_backward ->
 * _bwd_preprocess_do_o_dot + _bwd_sparse_index_kernel,
 * easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:2442-2846, :534-576,
 * :579-743, behind SparseIndexFlashAttnFunc.backward :3240-3283) for the case the reference
 * presets train with: the attention mass is detached before the indexer loss (detach_input,
 * easyvolcap/official_vggt/layers/dsa_attention.py:4694-4695), so dattn_sum is absent or zero.
 * It pays off when a query selects more than roughly 1 % of the keys.
 * Needs D = 64, a positive softmax_scale, token strides of q, k, v and dO below 2^23
 * elements and T, S <= 2^25 - 256 (the kernels' 32-bit load offsets; T is padded to a multiple
 * of 256, S to one of 128) and T <= 65528 * 32 (the grid); otherwise
 * GW_ERR_UNSUPPORTED.
 * Arguments as for gw_sparse_attn_bwd (no dattn_sum, no CSR). route: device int array of B
 * entries, written by this call: route[b] = 1 for a batch element it left untouched
 * (dq/dk/dv of that element not written) because a row lists a position twice (the reference
 * counts it twice) or q, k, v, dO, o or lse hold a non-finite value (the dense products would
 * carry it from rows a query did not select); compute such elements with gw_sparse_attn_bwd.
 * Every element of dq/dk/dv of the other batch elements is written.
 * Workspace: gw_sparse_attn_bwd_dense_workspace_size(B, T, S, H, D, K) bytes, 16-byte aligned
 * (selection words query- and key-major, 2 * B * round_up(S, 128) / 32 * round_up(T, 256) * 4
 * bytes; q^T, dO^T and k^T copies, B * H * 64 * (2 round_up(T, 256) + round_up(S, 128)) * 2
 * bytes; per-row lse and delta, B * H * round_up(T, 256) * 8 bytes).
 * ------------------------------------------------------------------------------------ */
size_t gw_sparse_attn_bwd_dense_workspace_size(int64_t B, int64_t T, int64_t S, int64_t H, int64_t D,
                                               int64_t K);
int gw_sparse_attn_bwd_dense(int dtype,
                             const void* q, const int64_t* q_strides,
                             const void* k, const int64_t* k_strides,
                             const void* v, const int64_t* v_strides,
                             const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                             const void* o, const int64_t* o_strides,
                             const void* dout, const int64_t* do_strides,
                             const float* lse,
                             void* dq, const int64_t* dq_strides,
                             void* dk, const int64_t* dk_strides,
                             void* dv, const int64_t* dv_strides,
                             int64_t B, int64_t T, int64_t S, int64_t H, int64_t D, int64_t K,
                             float softmax_scale, int* route,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GEOWEAVE_HIP_H */
