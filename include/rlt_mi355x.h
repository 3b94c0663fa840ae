/*
 * rlt_mi355x -- C ABI of the MI355X (gfx950) speculative-verification hot path.
 *
 * Plain pointers, sizes and strides only.  Every entry point:
 *   - enqueues its kernels on `stream` and never synchronizes the host;
 *   - allocates nothing: callers pass a device workspace of at least the size the
 *     matching *_workspace_size() query returns;
 *   - never writes its inputs;
 *   - returns 0 (RLT_OK) or an rlt_status error code; numerical failure of the
 *     sampler is reported through its `error` / `valid` outputs, not the status.
 *
 * Element types: RLT_F32 = 0, RLT_F16 = 1, RLT_BF16 = 2, RLT_FP8_E4M3 = 3 (OCP e4m3fn).
 * Status codes:  0 ok, 1 bad argument, 2 unsupported, 3 workspace, 4 launch failure.
 * Strides are in elements of the tensor they describe.
 */
#ifndef RLT_MI355X_H
#define RLT_MI355X_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Version of this interface.  It changes whenever an entry point's arguments change
 * (e.g. the (workspace, workspace_bytes) pair of rlt_batched_probabilities and
 * rlt_verify_distributions, added before their `stream` argument in version 2), so a
 * caller built against another header can refuse the library instead of passing its
 * arguments in the wrong slots.  No counterpart in the reference (its kernels are
 * Python / Triton); for callers binding this library directly.
 */
#define RLT_MI355X_ABI_VERSION 4
int rlt_abi_version(void);

/*
 * `flags` bits of the attention entry points that take them:
 *   RLT_ATTN_COMPENSATE: the 16-bit P operand of O = P V is followed by a second MFMA
 *   with what its cast dropped (P - float(bf16(P))), as the reference's compensated
 *   packed kernel does (vllm_rlt/kernels/triton_attention.py:368-371, selected by
 *   vllm_rlt/attention/backend.py:150-161).  MFMA calls only, blocks holding whole
 *   16-position tiles (else RLT_ERR_UNSUPPORTED); packed calls then stay on the verify
 *   kernels at every q_len, so packed rows still equal per-row rows bit for bit.
 */
#define RLT_ATTN_COMPENSATE 1

/* ---------------------------------------------------------------- attention */

/*
 * Paged GQA attention over one layer's KV pool view [block, token, kv_head, dim]
 * (the strided `key_cache[:, layer]` view of the reference pool
 * [num_blocks, layers, block_size, kv_heads, head_dim]).
 *
 * Replaces, behind the same tensors and semantics:
 *   - per-row form (cu_seqlens_q == NULL, one sequence per q row):
 *       vllm_rlt/kernels/paged_attention.py:13-47   torch_paged_attention
 *       vllm_rlt/kernels/triton_attention.py:176-246 paged_attention (split-KV decode)
 *       vllm_rlt/attention/backend.py:54-55          AttentionBackend.__call__
 *   - sliding window (window > 0):
 *       vllm_rlt/kernels/paged_attention.py:50-90   torch_paged_attention_windowed
 *   - packed verify window (cu_seqlens_q != NULL, int32 [num_seqs + 1]):
 *       vllm_rlt/kernels/triton_attention.py:386-404 paged_prefill_attention
 *       vllm_rlt/attention/backend.py:68-69          AttentionBackend.prefill
 *     query i of sequence s sees keys < context_lengths[s] - q_len(s) + i + 1.
 *
 * q / out: [num_q_rows, num_q_heads, head_dim] (dim stride 1).
 * block_tables: int32 [num_seqs, >= table_width] with row stride table_stride.
 * context_lengths: int32 [num_seqs].  Entries outside [0, num_blocks) read block 0.
 * Scales (FP8 pools): scale_mode 0 none, 1 per-tensor (key_scale / value_scale
 * point at one float), 2 per-vector pools [block, token, kv_head] with the given
 * strides (vllm_rlt/core/kv_cache_manager.py:267-271, :936-942).
 * The grid is static (independent of lengths): safe under HIP graph capture.
 */
size_t rlt_paged_attention_workspace_size(int32_t num_q_rows, int32_t num_q_heads, int32_t head_dim,
                                          int32_t table_width, int32_t block_size);

int rlt_paged_attention(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                        const void* key_cache, const void* value_cache, int64_t k_block_stride,
                        int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                        int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
                        const int32_t* block_tables, int64_t table_stride, int32_t table_width,
                        const int32_t* context_lengths, const int32_t* cu_seqlens_q,
                        int32_t num_seqs, int32_t max_q_len, int32_t num_q_rows,
                        const float* key_scale, const float* value_scale, int32_t scale_mode,
                        int64_t s_block_stride, int64_t s_token_stride, int64_t s_head_stride,
                        int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t block_size, int32_t q_dtype, int32_t kv_dtype, int32_t window,
                        void* out, int64_t out_row_stride, int64_t out_head_stride,
                        void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * rlt_paged_attention with explicit per-row key counts for the packed form:
 * query i of sequence s sees keys < row_lengths[cu_seqlens_q[s] + i] (int32
 * [num_q_rows]; with window > 0, the last `window` of them) instead of the causal
 * window's context_lengths[s] - q_len(s) + i + 1.  The rows of a sequence may come
 * in any order (each unit takes the bounds over all of its rows).  It lets rows that read one block table share each
 * KV byte although their positions are not consecutive: the pipelined verify of
 * vllm_rlt/worker/async_speculative.py:449-470, where window row j reads loop-depth
 * plane (d0 + j) mod planes and rows d0 and d0 + planes fall on the same plane.  The
 * reference runs such rows through the per-row call (kernels/paged_attention.py:13-47,
 * one gathered table per row); every row here equals that per-row result bit for bit.
 * Never takes the long-prompt prefill tiling.  row_lengths == NULL with flags == 0 is
 * rlt_paged_attention; row_lengths without cu_seqlens_q is RLT_ERR_ARGUMENT.  flags:
 * RLT_ATTN_COMPENSATE or 0.
 */
int rlt_paged_attention_rows(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                             const void* key_cache, const void* value_cache, int64_t k_block_stride,
                             int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                             int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
                             const int32_t* block_tables, int64_t table_stride, int32_t table_width,
                             const int32_t* context_lengths, const int32_t* row_lengths,
                             const int32_t* cu_seqlens_q, int32_t num_seqs, int32_t max_q_len,
                             int32_t num_q_rows, const float* key_scale, const float* value_scale,
                             int32_t scale_mode, int64_t s_block_stride, int64_t s_token_stride,
                             int64_t s_head_stride, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t block_size, int32_t q_dtype, int32_t kv_dtype,
                             int32_t window, int32_t flags, void* out, int64_t out_row_stride,
                             int64_t out_head_stride, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/*
 * The packed verify window with its own keys and values stored first: row r of
 * new_k / new_v ([num_q_rows, kv_heads, head_dim], strides in elements, 16-byte
 * aligned rows) is written into the pool at the position of packed q row r
 * (context_lengths[s] - q_len_s + i for window row i of sequence s) through the block
 * table, then attention runs as rlt_paged_attention (no scales, no sliding window).
 * Replaces the writer that precedes attention in every layer
 * (vllm_rlt/kernels/graph_kv.py:52-67, the KV scatter of the window rows) followed by
 * the packed attention call (vllm_rlt/kernels/triton_attention.py:386-404), in one
 * launch pair: the attention waves that read a window position store it before
 * reading.  Windows that take the prefill tiling (rlt_paged_attention_uses_prefill)
 * run a window-store kernel, then the tiling, on the stream.  bf16 / fp16 q and pool
 * of one dtype with a head_dim the MFMA kernels serve; other shapes return
 * RLT_ERR_UNSUPPORTED (the caller then stores and attends separately).  Table entries
 * outside [0, num_blocks) are not written.  Workspace: rlt_paged_attention_workspace_size.
 */
int rlt_paged_attention_store(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                              void* key_cache, void* value_cache, int64_t k_block_stride,
                              int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                              int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
                              const int32_t* block_tables, int64_t table_stride,
                              int32_t table_width, const int32_t* context_lengths,
                              const int32_t* cu_seqlens_q, int32_t num_seqs, int32_t max_q_len,
                              int32_t num_q_rows, int32_t num_q_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t block_size, int32_t dtype,
                              const void* new_k, const void* new_v, int64_t new_row_stride,
                              int64_t new_head_stride, void* out, int64_t out_row_stride,
                              int64_t out_head_stride, void* workspace, size_t workspace_bytes,
                              hipStream_t stream);

/*
 * rlt_paged_attention_store with scales, explicit row lengths and either pool type:
 *   - 16-bit pools as rlt_paged_attention_store (scale_mode 0);
 *   - fp8-e4m3 pools (kv_dtype 3; q and the rows bf16 / fp16): the rows are quantized
 *     as they are stored -- codes and scales bitwise rlt_kv_store_fp8's, i.e. the
 *     reference's quantize_fp8 (vllm_rlt/core/kv_cache_manager.py:50-61) -- with the
 *     per-tensor scales (scale_mode 1: key_scale / value_scale point at one float
 *     each, read only) or with per-vector scales computed from each (row, kv head)
 *     vector and written into the [block, token, kv_head] scale pools (scale_mode 2),
 *     then read back by the attention with the same scales.  Replaces the fused
 *     quantize-store vllm_rlt/kernels/triton_attention.py:506-623 (store_fp8)
 *     followed by the packed attention call (:386-404), in one launch pair.
 *   - row_lengths (int32 [num_q_rows], optional): packed row r sits at position
 *     row_lengths[r] - 1 of its sequence (and sees that many keys, as in
 *     rlt_paged_attention_rows) instead of context_lengths[s] - q_len_s + i.
 * Pool strides must be multiples of 16 bytes (16-bit pools) or 8 bytes (fp8).
 * Positions whose block index lies beyond the table, or whose table entry lies
 * outside the pool, are not written.  Windows that take the prefill tiling store first,
 * then attend (two launches); float32 q returns RLT_ERR_UNSUPPORTED.  flags:
 * RLT_ATTN_COMPENSATE or 0.
 * Workspace: rlt_paged_attention_workspace_size.
 */
int rlt_paged_attention_store_scaled(
    const void* q, int64_t q_row_stride, int64_t q_head_stride, void* key_cache,
    void* value_cache, int64_t k_block_stride, int64_t k_token_stride, int64_t k_head_stride,
    int64_t v_block_stride, int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
    const int32_t* block_tables, int64_t table_stride, int32_t table_width,
    const int32_t* context_lengths, const int32_t* row_lengths, const int32_t* cu_seqlens_q,
    int32_t num_seqs, int32_t max_q_len, int32_t num_q_rows, float* key_scale, float* value_scale,
    int32_t scale_mode, int64_t s_block_stride, int64_t s_token_stride, int64_t s_head_stride,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int32_t q_dtype, int32_t kv_dtype, int32_t flags, const void* new_k, const void* new_v,
    int64_t new_row_stride, int64_t new_head_stride, void* out, int64_t out_row_stride,
    int64_t out_head_stride, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* 1 when (q dtype, kv dtype, head_dim) runs on the MFMA kernel, else 0 (vector kernel). */
int rlt_paged_attention_uses_mfma(int32_t q_dtype, int32_t kv_dtype, int32_t head_dim);

/* 1 when a packed call with this longest q window takes the long-prompt prefill
 * tiling (bf16 / fp16 q with KV of the same type or fp8-e4m3, head_dim 64, 96 or 128,
 * max_q_len >= 64; calls with row_lengths or RLT_ATTN_COMPENSATE never take it):
 * 128-row groups, K / V tiles shared through LDS, normalized in one launch.  Rows of
 * such a call match the per-row form within floating-point tolerance; every other
 * call (all verify windows) equals the per-row form bit for bit.  The reference's
 * prefill kernel is a separate tiling too: vllm_rlt/kernels/triton_attention.py:250-383. */
int rlt_paged_attention_uses_prefill(int32_t q_dtype, int32_t kv_dtype, int32_t head_dim,
                                     int32_t max_q_len);

/* ---------------------------------------------------------------- sampler */

/*
 * Batched speculative rejection sampling, bit-exact with the reference's torch-CPU
 * arithmetic given identical fp32 p, q and uniforms.
 * Replaces vllm_rlt/worker/speculative_sampling.py:104-181 speculative_accept
 * (AcceptResult :88-101).
 *   draft_tokens int64 [n, w1], drafts int64 [n], q fp32 [n, w1, V],
 *   p fp32 [n, w1 + 1, V], u_accept fp32 [n, w1], u_final fp32 [n]  (contiguous)
 *   -> tokens int64 [n, w1 + 1], accepted int64 [n], final_token int64 [n],
 *      error uint8 (bool) [n].
 * 0 <= w1 <= 32, 1 <= V < 2^25.
 */
size_t rlt_speculative_accept_workspace_size(int64_t n, int32_t w1, int64_t vocab);

int rlt_speculative_accept(const int64_t* draft_tokens, const int64_t* drafts, const float* q,
                           const float* p, const float* u_accept, const float* u_final, int64_t n,
                           int32_t w1, int64_t vocab, int64_t* tokens, int64_t* accepted,
                           int64_t* final_token, uint8_t* error, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

/*
 * rlt_speculative_accept without a workspace argument and without any allocation:
 * the workspace is a file-scope device array of
 * rlt_speculative_accept_noalloc_max_bytes() bytes (8 MiB) per GPU, held until the
 * process ends.  No counterpart in the reference: this is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, outputs and results as
 * rlt_speculative_accept.  Returns RLT_ERR_WORKSPACE when the call needs more than
 * that maximum (rlt_speculative_accept_workspace_size(n, w1, V) bytes; e.g. n = 256,
 * w1 = 4, V = 65536 needs about 2.5 MiB).  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (on different streams, or from different
 * threads) race and must be serialized by the caller.
 */
size_t rlt_speculative_accept_noalloc_max_bytes(void);

int rlt_speculative_accept_noalloc(const int64_t* draft_tokens, const int64_t* drafts,
                                   const float* q, const float* p, const float* u_accept,
                                   const float* u_final, int64_t n, int32_t w1, int64_t vocab,
                                   int64_t* tokens, int64_t* accepted, int64_t* final_token,
                                   uint8_t* error, hipStream_t stream);

/*
 * Inverse-CDF draw from nonnegative, possibly unnormalized fp32 weights [m, V]
 * (contiguous) with uniforms u [m]: float64 cumulative sum, threshold
 * min(u * mass, nextafter(mass, 0)), right-bisect; invalid rows (mass not finite
 * and positive) give index 0 and valid = 0.
 * Replaces vllm_rlt/worker/speculative_sampling.py:59-85 categorical.
 */
size_t rlt_categorical_workspace_size(int64_t m, int64_t vocab);

int rlt_categorical(const float* weights, const float* u, int64_t m, int64_t vocab,
                    int64_t* index, uint8_t* valid, void* workspace, size_t workspace_bytes,
                    hipStream_t stream);

/*
 * Row sums x.sum(-1, dtype=float32) of a contiguous fp32 [rows, V] matrix in the
 * exact summation order of torch's CPU kernel (the masses computed at
 * vllm_rlt/worker/speculative_sampling.py:138,146).
 */
size_t rlt_row_mass_workspace_size(int64_t rows, int64_t vocab);

int rlt_row_mass_f32(const float* x, int64_t rows, int64_t vocab, float* out, void* workspace,
                     size_t workspace_bytes, hipStream_t stream);

/*
 * Temperature / strict top-k / strict top-p distributions of logits rows.
 * Replaces vllm_rlt/worker/speculative_sampling.py:8-56 batched_probabilities
 * (row form vllm_rlt/worker/sampler.py:28-55 Sampler.probabilities).
 *   logits [n, V] (RLT_F32 / RLT_BF16 / RLT_F16, row stride in elements),
 *   temperature fp32 [n] (> 0), top_k int64 [n], top_p fp32 [n]
 *   -> out fp32 [n, V] (row stride out_stride).
 * Row i: x = logits / T; if max_top_k > 0 and 0 < top_k[i] < V, only the
 * min(top_k[i], max_top_k) largest x survive (ties at the cut: lowest columns);
 * if apply_top_p and top_p[i] < 1, survivors are kept in descending order while
 * the softmax mass before them is <= top_p[i] (the token crossing the threshold is
 * kept); then softmax over the kept set.  max_top_k and apply_top_p are the host
 * plan's values, as in the reference.  Rows holding NaN (or with a non-finite
 * max) are written as NaN.  V <= 262144.
 * Workspace (optional): with rlt_probabilities_workspace_size(n, 0, vocab) bytes, a
 * call that filters no row (max_top_k == 0, apply_top_p == 0) runs the row-split
 * form: each row spread over several workgroups (slice max and mass, then the
 * normalized slices; two launches).  Otherwise (filtering calls, workspace == NULL)
 * one workgroup per row in one launch.  Both forms give the same values up to the
 * order of the float64 total's summation.
 */
size_t rlt_probabilities_workspace_size(int64_t rows, int64_t argmax_rows, int64_t vocab);

int rlt_batched_probabilities(const void* logits, int32_t logits_dtype, int64_t row_stride,
                              int64_t n, int64_t vocab, const float* temperature,
                              const int64_t* top_k, const float* top_p, int64_t max_top_k,
                              int32_t apply_top_p, float* out, int64_t out_stride,
                              void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Draft proposals of one draft offset: proposed[i] = argmax of logits row i
 * (i < m; first maximal column, NaN the maximum); then for the random rows
 * random_rows[j] (j < r), q_out row j = batched_probabilities of that logits row
 * with temperature[j] / top_k[j] / top_p[j], and proposed[random_rows[j]] =
 * categorical(q_out row j, u[j]) (0 for an invalid row).  Replaces the draft step
 * of vllm_rlt/worker/async_speculative.py:645-663 (argmax, _probabilities on
 * logits[random_rows], categorical, proposed[random_rows] = sampled) in three
 * launches without host synchronization.  q_out rows are q_stride floats apart (pass
 * the q[:, offset] view).  Workspace: rlt_propose_drafts_workspace_size(m, r, vocab)
 * (row-split distributions when no row is filtered), or at least
 * rlt_categorical_workspace_size(r, vocab) (one workgroup per row).
 * A random row index outside [0, m) gives an all-NaN q_out row and proposes nothing.
 */
size_t rlt_propose_drafts_workspace_size(int64_t m, int64_t r, int64_t vocab);

int rlt_propose_drafts(const void* logits, int32_t logits_dtype, int64_t row_stride, int64_t m,
                       int64_t vocab, const int64_t* random_rows, int64_t r,
                       const float* temperature, const int64_t* top_k, const float* top_p,
                       int64_t max_top_k, int32_t apply_top_p, const float* u, float* q_out,
                       int64_t q_stride, int64_t* proposed, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/*
 * The verify side of a round: targets[i] = argmax of logits row i (i < m; first
 * maximal column, NaN the maximum) and, for the random rows random_rows[j] (j < r),
 * p_out row j = batched_probabilities of that logits row with temperature[j] /
 * top_k[j] / top_p[j] (rows p_stride floats apart, e.g. a p[ranks, offsets] view when
 * rows line up).  One launch: the argmax rows are extra workgroups of the
 * distribution launch.  Replaces vllm_rlt/worker/async_speculative.py:678-692
 * (target = logits.argmax(-1); p[v_ranks, v_offsets] = _probabilities(logits[v_rows],
 * ...)).  A random row index outside [0, m) gives an all-NaN p row.  Workspace:
 * rlt_probabilities_workspace_size(r, m, vocab) bytes (row-split form for calls
 * that filter no row, the argmax rows as extra slices), or NULL (one workgroup per
 * row).
 */
int rlt_verify_distributions(const void* logits, int32_t logits_dtype, int64_t row_stride,
                             int64_t m, int64_t vocab, const int64_t* random_rows, int64_t r,
                             const float* temperature, const int64_t* top_k, const float* top_p,
                             int64_t max_top_k, int32_t apply_top_p, float* p_out,
                             int64_t p_stride, int64_t* targets, void* workspace,
                             size_t workspace_bytes, hipStream_t stream);

/*
 * The stochastic verify round in one call: targets = argmax of each of the
 * n * (w1 + 1) target-logit rows, p_out [n, w1 + 1, V] = their batched_probabilities
 * (temperature / top_k / top_p per row), then speculative_accept with p_out.  Bitwise
 * the results of rlt_verify_distributions (all rows random) followed by
 * rlt_speculative_accept; the draft rows' float32 row-sum partials are computed by
 * otherwise idle workgroups of the distribution launch, so the acceptance then sums
 * only p.  Replaces vllm_rlt/worker/async_speculative.py:678-692 (_verify) followed by
 * :727-734 (speculative_accept).  Workspace: rlt_verify_accept_workspace_size
 * (row-split distributions when no row is filtered, the draft rows' partials as
 * extra workgroups of its first launch), or at least
 * rlt_speculative_accept_workspace_size (one workgroup per row).
 */
size_t rlt_verify_accept_workspace_size(int64_t n, int32_t w1, int64_t vocab);

int rlt_verify_accept(const void* target_logits, int32_t logits_dtype, int64_t row_stride,
                      const float* temperature, const int64_t* top_k, const float* top_p,
                      int64_t max_top_k, int32_t apply_top_p, const int64_t* draft_tokens,
                      const int64_t* drafts, const float* q, const float* u_accept,
                      const float* u_final, int64_t n, int32_t w1, int64_t vocab,
                      int64_t* targets, float* p_out, int64_t* tokens, int64_t* accepted,
                      int64_t* final_token, uint8_t* error, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

/*
 * Greedy verify round: targets = argmax of every verify row (first maximal column,
 * NaN counts as the maximum), accepted = number of leading drafts j < drafts[r]
 * with draft_tokens[r, j] == targets[r, j], next_token = targets[r, accepted].
 * Replaces the device greedy round of vllm_rlt/worker/async_speculative.py:706-720
 * (host rule vllm_rlt/worker/speculative.py:41-53 greedy_accept).
 *   draft_tokens int64 [n, w1], drafts int64 [n],
 *   target_logits [n, w1 + 1, V] (RLT_F32 / RLT_BF16 / RLT_F16; row stride in
 *   elements between consecutive verify rows) -> targets int64 [n, w1 + 1],
 *   accepted int64 [n], next_token int64 [n].  No workspace.
 */
int rlt_greedy_accept(const int64_t* draft_tokens, const int64_t* drafts, const void* target_logits,
                      int32_t logits_dtype, int64_t row_stride, int64_t n, int32_t w1,
                      int64_t vocab, int64_t* targets, int64_t* accepted, int64_t* next_token,
                      hipStream_t stream);

/* ---------------------------------------------------------------- KV write side */

/*
 * Scatter of K and V rows [rows, kv_heads, head_dim] (dim stride 1; row / head
 * strides in elements) into one layer's pool view [block, token, kv_head, dim]
 * (`key_cache[:, layer]`, strides in elements) at (blocks[r], offsets[r]).
 * Rows with mask[r] == 0 (mask optional, uint8 [rows]) or r >= *active (active
 * optional, int32 scalar on the device) are skipped, as are rows whose block or
 * offset lies outside [0, num_blocks) x [0, block_size).  dtype: the pool's and the
 * rows' element type (RLT_F32 / RLT_F16 / RLT_BF16 / RLT_FP8_E4M3 codes copied).
 * Replaces vllm_rlt/kernels/routing.py:183-223 masked_kv_store,
 * vllm_rlt/kernels/graph_kv.py:7-67 write_graph_kv and the index_put of
 * vllm_rlt/core/kv_cache_manager.py:893-895.
 */
int rlt_kv_store(const void* k, const void* v, int64_t k_row_stride, int64_t k_head_stride,
                 int64_t v_row_stride, int64_t v_head_stride, void* key_cache, void* value_cache,
                 int64_t c_block_stride, int64_t c_token_stride, int64_t c_head_stride,
                 int64_t num_blocks, int32_t block_size, const int64_t* blocks,
                 const int64_t* offsets, const uint8_t* mask, const int32_t* active, int64_t rows,
                 int32_t kv_heads, int32_t head_dim, int32_t dtype, hipStream_t stream);

/*
 * Quantizing scatter into an FP8 e4m3 pool with per-vector fp32 scales
 * [block, token, kv_head]: per (row, head) scale = max(amax * (1/448), FLT_MIN), or
 * fixed_scale when has_fixed_scale; codes = clamp(x / scale, -448, 448) (IEEE
 * division) rounded to e4m3fn.  Bitwise equal to
 * vllm_rlt/core/kv_cache_manager.py:50-61 quantize_fp8.  Rows src_dtype
 * (RLT_F32 / RLT_F16 / RLT_BF16), head_dim <= 256; mask / active / range skipping as
 * rlt_kv_store.  Replaces vllm_rlt/kernels/triton_attention.py:505-623 store_fp8.
 */
int rlt_kv_store_fp8(const void* k, const void* v, int32_t src_dtype, int64_t k_row_stride,
                     int64_t k_head_stride, int64_t v_row_stride, int64_t v_head_stride,
                     void* key_codes, void* value_codes, int64_t c_block_stride,
                     int64_t c_token_stride, int64_t c_head_stride, float* key_scale,
                     float* value_scale, int64_t s_block_stride, int64_t s_token_stride,
                     int64_t s_head_stride, int64_t num_blocks, int32_t block_size,
                     const int64_t* blocks, const int64_t* offsets, const uint8_t* mask,
                     const int32_t* active, int64_t rows, int32_t kv_heads, int32_t head_dim,
                     int32_t has_fixed_scale, float fixed_scale, hipStream_t stream);

/*
 * LAST_EXITED finalize copy.  descriptors int64 [count, 3] = (slot, exit depth,
 * position); tables int32 [slots, planes, width] (block of each page of each plane).
 * For every plane p > exit depth, the `layers` x bytes_per_token bytes of the
 * position's page offset are copied from the exit plane's block to plane p's block,
 * in both pools [block, layer, token, ...] (strides in elements of elt_bytes; use the
 * same call on the fp32 scale pools of an FP8 cache).  Descriptors or table entries
 * outside the tables / pool copy nothing.  Replaces
 * vllm_rlt/kernels/routing.py:147-180 finalize_kernel (host form
 * vllm_rlt/core/kv_cache_manager.py:1053-1076 finalize_token).
 */
int rlt_kv_finalize(const int64_t* descriptors, int64_t count, const int32_t* tables,
                    int64_t slots, int32_t width, int32_t planes, int32_t block_size,
                    int32_t layers, int64_t num_blocks, void* key_pool, void* value_pool,
                    int64_t block_stride, int64_t layer_stride, int64_t token_stride,
                    int64_t bytes_per_token, int32_t elt_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- routing / metadata */

/*
 * Device routing of the asynchronous verify step.  Descriptors are int64
 * [count, 3] = (request slot, depth, position) and may live in mapped pinned host
 * memory.  Grids depend only on the capacities passed (`size`, `max_rows`, ...), so
 * captured HIP graphs replay with new descriptor contents.  Indices read from
 * memory are bounds-checked: gathers from outside a pool read zeros, scatters
 * outside a pool are skipped, a write block that cannot be formed is -1.
 */

/* slots[row] = descriptor[row].slot for row < count, 0 for count <= row < size.
 * Replaces vllm_rlt/kernels/routing.py:7-11 slots_kernel. */
int rlt_route_slots(const int64_t* descriptor, int64_t* slots, int64_t count, int64_t size,
                    hipStream_t stream);

/* Per-row attention metadata from the descriptor and the slot-major plane tables
 * int32 [table_rows = slots * planes, width]: plane = depth (planes > 1) or 0;
 * slots / positions int64 [size], lengths int32 [size] = pos + 1 (0 past count),
 * blocks / offsets int64 [count] = the position's write address, out_tables int32
 * [size, out_stride] = the plane's first out_width table entries (0 past count).
 * Replaces vllm_rlt/kernels/routing.py:14-49 metadata_kernel (caller
 * vllm_rlt/worker/async_state.py:65-97). */
int rlt_route_metadata(const int64_t* descriptor, const int32_t* tables, int64_t table_rows,
                       int32_t width, int32_t page, int32_t planes, int64_t* slots,
                       int64_t* positions, int32_t* lengths, int64_t* blocks, int64_t* offsets,
                       int32_t* out_tables, int64_t out_stride, int32_t out_width, int64_t count,
                       int64_t size, hipStream_t stream);

/* out[row] = pool[slots[row]] (row_elems elements of elt_bytes) for row < count,
 * zeros for count <= row < size.  Replaces vllm_rlt/kernels/routing.py:52-64
 * gather_kernel (callers vllm_rlt/worker/async_state.py:104-113,
 * vllm_rlt/worker/async_speculative.py:605-615). */
int rlt_route_gather(const void* pool, int64_t pool_rows, int64_t pool_stride,
                     const int64_t* slots, void* out, int64_t out_stride, int64_t count,
                     int64_t size, int64_t row_elems, int32_t elt_bytes, hipStream_t stream);

/* pool[slots[row]] = values[row] for row < count.  Replaces
 * vllm_rlt/kernels/routing.py:67-82 scatter_kernel (callers
 * vllm_rlt/worker/async_state.py:115-123, vllm_rlt/worker/async_speculative.py:754-760). */
int rlt_route_scatter(const void* values, int64_t values_stride, const int64_t* slots, void* pool,
                      int64_t pool_rows, int64_t pool_stride, int64_t count, int64_t row_elems,
                      int32_t elt_bytes, hipStream_t stream);

/* Segments int64 [num_segments, 5] = (slot, row offset, row count, batch row start,
 * keep).  Gather: out[start + r] = pool[slot * rows_per_slot + offset + r] for
 * r < min(count, max_rows).  Replaces vllm_rlt/kernels/routing.py:85-112
 * gather_segments_kernel (caller vllm_rlt/worker/model_runner.py:519-543). */
int rlt_route_gather_segments(const void* pool, int64_t pool_slots, int64_t rows_per_slot,
                              int64_t pool_stride, const int64_t* segments, int64_t num_segments,
                              int64_t max_rows, void* out, int64_t out_rows, int64_t out_stride,
                              int64_t row_elems, int32_t elt_bytes, hipStream_t stream);

/* Scatter of the kept segments: pool[slot * rows_per_slot + offset + r] =
 * values[start + r].  Replaces vllm_rlt/kernels/routing.py:115-144
 * scatter_segments_kernel (caller vllm_rlt/worker/model_runner.py:559-584). */
int rlt_route_scatter_segments(const void* values, int64_t values_rows, int64_t values_stride,
                               const int64_t* segments, int64_t num_segments, int64_t max_rows,
                               void* pool, int64_t pool_slots, int64_t rows_per_slot,
                               int64_t pool_stride, int64_t row_elems, int32_t elt_bytes,
                               hipStream_t stream);

/* KV write addresses of packed query rows: blocks[i] = tables[sequences[i],
 * positions[i] / page], offsets[i] = positions[i] % page.  Replaces
 * vllm_rlt/kernels/metadata.py:7-24 expand_kv_addresses (caller
 * vllm_rlt/worker/buffers.py:289-335). */
int rlt_expand_kv_addresses(const int64_t* positions, const int32_t* sequences,
                            const int32_t* tables, int64_t num_sequences, int32_t width,
                            int32_t page, int64_t* blocks, int64_t* offsets, int64_t n,
                            hipStream_t stream);

/* Per-row depth-table gather of the recurrent step: out_table[row] =
 * tables[row, depth[row]] (tables int32 [n, planes, width] with the given strides),
 * blocks / offsets = the write address of positions[row] in it (floor division),
 * lengths = positions + 1, or 0 where active (bool, may be NULL) is false.  Replaces
 * the tensor formulas of vllm_rlt/worker/async_speculative.py:449-466. */
int rlt_depth_tables(const int32_t* tables, int64_t row_stride, int64_t plane_stride,
                     int32_t planes, int32_t width, const int64_t* depth,
                     const int64_t* positions, const uint8_t* active, int32_t block_size,
                     int32_t* out_table, int64_t out_stride, int64_t* blocks, int64_t* offsets,
                     int32_t* lengths, int64_t n, hipStream_t stream);

/*
 * Sync-mode rejection sampling of a batch of requests: the device part of
 * vllm_rlt/worker/speculative.py:56-72 rejection_sample as its caller _collect_round
 * (:574-625) runs it, draft after draft.  For request i with counts[i] = d <= k drafts
 * candidates[i, :d] (int64 [n, k]), target p fp32 [n, k + 1, V] (row j verifies draft
 * j), proposal q fp32 [n, k, V] and uniforms u fp32 [n, k] (the generator's draws, in
 * order), draft j is taken in order until the first event:
 *   candidate outside [-V, V)  -> status 4 (the reference raises IndexError),
 *   q[j, x] not > 0            -> status 2 (ValueError; u[j] is not consumed),
 *   u[j] * q[j, x] < p[j, x]   -> accepted, next draft,
 *   otherwise                  -> rejected: residual[i] = clamp_min(p[j] - q[j], 0)
 *                                 divided by its float32 total, summed in torch's order
 *                                 for a whole 1-D tensor on `sum_threads` CPU threads;
 *                                 status 1, or 3 if that total is not finite and > 0
 *                                 (RuntimeError).
 * All d accepted -> status 0 (the bonus draw comes from p[d]).  accepted[i] = drafts
 * accepted before the event.  status int32 [n], accepted int64 [n], residual fp32
 * [n, V] (rows of requests whose status is not 1 are unspecified).  The residual draw
 * itself (torch.multinomial on the request's generator) stays with the caller.
 * 1 <= sum_threads <= 256, V < 2^31.
 */
size_t rlt_rejection_sample_workspace_size(int64_t n, int64_t vocab, int32_t sum_threads);

int rlt_rejection_sample(const int64_t* candidates, const int64_t* counts, const float* target,
                         const float* proposal, const float* uniforms, int64_t n, int32_t k,
                         int64_t vocab, int32_t sum_threads, int32_t* status, int64_t* accepted,
                         float* residual, void* workspace, size_t workspace_bytes,
                         hipStream_t stream);

/* Random-round merge: overlay the random requests' speculative_accept outcome on
 * the greedy round, in one launch with no host reads.  Replaces
 * vllm_rlt/worker/async_speculative.py:162-198 merge_random_round (RandomRoundMerge
 * :152-159).  target int64 [num_rows] (argmax per request-major verify row),
 * accepted / next_tokens / starts / input_tokens int64 [n]; the outcome of the r random
 * requests: tokens int64 [r, width], r_accepted / r_final int64 [r], r_error bool [r];
 * random_requests int64 [r]; verify_rows / verify_ranks / verify_offsets int64
 * [num_verify].  Outputs: rows_out [num_rows], accepted_out / next_tokens_out /
 * next_positions_out / error_out [n] (error as 0 / 1), next_values_out [n, 2]
 * (token, position): a failed request keeps (input_token, start).  Index tensors must
 * not repeat an index (the reference's scatters leave the winner unspecified then);
 * an index outside its range (the reference raises) is skipped and fails the whole
 * round: error_out is 1 for every request, whose slot values stay (input_token, start). */
int rlt_merge_random_round(const int64_t* target, int64_t num_rows, const int64_t* accepted,
                           const int64_t* next_tokens, const int64_t* starts,
                           const int64_t* input_tokens, int64_t n, const int64_t* tokens,
                           int32_t width, const int64_t* r_accepted, const int64_t* r_final,
                           const uint8_t* r_error, const int64_t* random_requests, int64_t r,
                           const int64_t* verify_rows, const int64_t* verify_ranks,
                           const int64_t* verify_offsets, int64_t num_verify, int64_t* rows_out,
                           int64_t* accepted_out, int64_t* next_tokens_out,
                           int64_t* next_positions_out, int64_t* next_values_out,
                           int64_t* error_out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RLT_MI355X_H */
