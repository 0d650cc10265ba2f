/*
 * hla_s6.h -- C ABI of the MI355X (gfx950) S6 latent decode-attention library (libhla_s6.so).
 *
 * Every entry point takes plain device pointers, element strides (in elements of the pointed-to
 * type), sizes and a hipStream_t passed as `void *` (NULL = the null stream). The library never
 * allocates or frees device memory, never synchronizes with the host, keeps no per-call global state
 * and only enqueues kernels on the given stream, so every call is safe under HIP graph capture.
 * Floating-point tensors are bf16 (raw 16-bit patterns, `void *`) unless declared `float *`;
 * `lse` outputs are contiguous fp32 [H, T] natural-log log-sum-exps of the already-scaled scores.
 *
 * Conventions shared by every attention entry point (hla/vllm_latent/s6_ops.py:1-10):
 * an empty row gives o = 0 and lse = -inf; +inf lse counts as empty in merges; padding
 * (invalid) rows are zeroed; no NaN leaves a merge.
 *
 * Return value: HLA_S6_OK or one of the error codes below; hla_s6_last_error() returns the
 * message of the calling thread's last failure. No exception crosses the ABI.
 */
#ifndef HLA_S6_H
#define HLA_S6_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HLA_S6_ABI_VERSION 11

#define HLA_S6_OK 0
#define HLA_S6_EINVAL 1       /* bad shape, stride or argument            (Python: ValueError)   */
#define HLA_S6_EUNSUPPORTED 2 /* shape outside the compiled kernels       (Python: ValueError)   */
#define HLA_S6_EWORKSPACE 3   /* caller workspace too small               (Python: RuntimeError) */
#define HLA_S6_ELAUNCH 4      /* HIP launch / runtime error               (Python: RuntimeError) */
#define HLA_S6_EDEVICE 5      /* no usable gfx950 device                  (Python: RuntimeError) */

int hla_s6_abi_version(void);
const char *hla_s6_last_error(void);

/* Number of compute units of `device` (the `sm_count` argument of num_kv_splits,
 * hla/vllm_latent/ouro_latent.py:204). */
int hla_s6_device_cus(int device, int *cus);

/* ---- a1: step metadata ------------------------------------------------------------------------
 * Replaces s6_ops.token_requests (hla/vllm_latent/s6_ops.py:61-68), s6_ops.history_lengths
 * (hla/vllm_latent/s6_ops.py:71-73) and the ctx / ctx_latent math of StepContext.__init__
 * (hla/vllm_latent/s6_layer.py:64-70).
 *   query_start_loc [num_reqs + 1] int32, seq_lens [num_reqs] int32.
 *   seq_lens may be NULL when ctx, ctx_latent and history are NULL.
 *   Outputs (each nullable): token_requests [num_tokens] int64 (clamped to num_reqs - 1),
 *   valid [num_tokens] uint8 (t < query_start_loc[num_reqs]), invalid [num_tokens] uint8 (1 - valid, the
 *   StepContext.invalid mask), ctx [num_tokens] int32
 *   (history length of the token's request, 0 on padding), ctx_latent [num_tokens] int32
 *   (max(ctx - window, 0), ctx when window == 0), history [num_reqs] int32. */
int hla_s6_step_metadata(const int32_t *query_start_loc, int32_t num_reqs, const int32_t *seq_lens,
                         int32_t num_tokens, int32_t window, int64_t *token_requests, uint8_t *valid,
                         uint8_t *invalid, int32_t *ctx, int32_t *ctx_latent, int32_t *history, void *stream);

/* Replaces StepContext.block_table (hla/vllm_latent/s6_layer.py:75-80):
 * out[t, c] = table[token_requests[t], c] for c < cols. */
int hla_s6_gather_block_table(const int32_t *table, int64_t table_stride, int32_t num_reqs, int32_t cols,
                              const int64_t *token_requests, int32_t num_tokens, int32_t *out,
                              int64_t out_stride, void *stream);

/* ---- a2/a3: latent RoPE -----------------------------------------------------------------------
 * Replaces s6_ops.latent_rope with the in-place kernel semantics (hla/vllm_latent/s6_ops.py:23-41):
 * x[t, h, :width] <- x*cos + rotate_half(x)*sin with table[positions[t]] = [cos | sin] halves
 * (width/2 each, row stride table_stride), bf16 rounding after each of the three products/sums as
 * the torch formula does. x is [num_tokens, num_heads, width] with strides (stride_t, stride_h, 1).
 * Positions are clamped into [0, table_rows). */
int hla_s6_latent_rope(void *x, int32_t num_tokens, int32_t num_heads, int32_t width, int64_t stride_t,
                       int64_t stride_h, const int64_t *positions, const void *table, int32_t table_rows,
                       int64_t table_stride, void *stream);

/* ---- a3/a5: absorbed projections ----------------------------------------------------------------
 * out[t, h, :n_dim] = x[t, h, :k_dim] @ w[h, :k_dim, :n_dim] (bf16 operands, fp32 accumulation, bf16
 * result), i.e. torch.einsum('thd,hdr->thr') of the A_t absorption (hla/vllm_latent/s6_layer.py:37)
 * and of the B_t projection (hla/vllm_latent/s6_layer.py:114). When rope_table != NULL the latent
 * RoPE of hla_s6_latent_rope is applied to the rounded product before it is stored, which fuses
 * s6_layer.latent_query (hla/vllm_latent/s6_layer.py:32-40). x, w and out need a unit last stride;
 * w is [H, k_dim, n_dim] with strides (w_sh, w_sk, 1). k_dim in {128, 256, 512, 1024}, n_dim % 64 == 0. */
int hla_s6_absorb(const void *x, int32_t num_tokens, int32_t num_heads, int32_t k_dim, int64_t x_st,
                  int64_t x_sh, const void *w, int64_t w_sh, int64_t w_sk, int32_t n_dim, void *out,
                  int64_t o_st, int64_t o_sh, const int64_t *positions, const void *rope_table,
                  int32_t table_rows, int64_t table_stride, void *stream);

/* ---- a4: paged latent-history attention --------------------------------------------------------
 * Replaces s6_ops.history_attention / history_attention_kv for the MQA S6 cache
 * (hla/vllm_latent/s6_ops.py:117-161; semantics of _history_reference, 204-222): fully visible
 * softmax of q[t] (num_heads == 16 query heads, width in {128, 256, 512, 1024}) over the first
 * ctx[t] rows of the paged latent cache. Row j of token t is at
 *   k_cache + block_table[row(t)*bt_stride + j / block_size] * page_stride + (j % block_size) * row_stride
 * (and likewise for v_cache), row(t) = bt_rows ? bt_rows[t] : t; only table columns
 * < ceil(ctx[t] / block_size) are read. Metadata outside the buffers never faults: a row reads at most
 * bt_cols * block_size keys and page ids are clamped into [0, num_blocks). block_size % 16 == 0; q, K and V rows need a unit last
 * stride and 16-byte alignment. num_splits in [1, 1024] partitions each row's keys (split-KV): every row
 * is cut in chunks sized from the longest row of the call, partials go to `workspace` (fp32, caller-owned,
 * >= num_tokens * num_splits * 16 * (width + 1) floats; unused when num_splits == 1) and a second launch
 * reduces them by LSE. Calls that share a workspace must not overlap in time.
 * Outputs o [T, 16, width] bf16 (strides o_st, o_sh, 1) and lse [16, T] fp32. */
int hla_s6_history_attention(const void *q, int32_t num_tokens, int32_t num_heads, int32_t width,
                             int64_t q_st, int64_t q_sh, const void *k_cache, const void *v_cache,
                             int64_t page_stride, int64_t row_stride, int32_t block_size, int64_t num_blocks,
                             const int32_t *block_table, int64_t bt_stride, int32_t bt_cols, const int64_t *bt_rows,
                             const int32_t *ctx, float scale, int32_t num_splits, float *workspace,
                             int64_t workspace_floats, void *out, int64_t o_st, int64_t o_sh, float *lse,
                             void *stream);

/* hla_s6_history_attention for multi-query steps (chunked prefill, s6_layer.attend with max_query_len > 1,
 * hla/vllm_latent/s6_layer.py:97-115): one workgroup serves `group` (1, 2 or 4) consecutive tokens, and the
 * tokens of a group that share a block-table row (bt_rows[t] equal: one request) read each K/V tile once for all
 * of them; a group spanning two rows takes one pass per row. Each token still sees its own ctx[t] rows. Same
 * arguments, outputs and checks as hla_s6_history_attention. shared_rows != 0 declares that several tokens read the
 * same rows (any multi-query step, also with group == 1): K/V loads are then cached for the re-reads instead of
 * non-temporal. */
int hla_s6_history_attention_grouped(const void *q, int32_t num_tokens, int32_t num_heads, int32_t width,
                                     int64_t q_st, int64_t q_sh, const void *k_cache, const void *v_cache,
                                     int64_t page_stride, int64_t row_stride, int32_t block_size, int64_t num_blocks,
                                     const int32_t *block_table, int64_t bt_stride, int32_t bt_cols,
                                     const int64_t *bt_rows, const int32_t *ctx, float scale, int32_t num_splits,
                                     float *workspace, int64_t workspace_floats, void *out, int64_t o_st,
                                     int64_t o_sh, float *lse, int32_t group, int32_t shared_rows, void *stream);

/* The two launches of hla_s6_history_attention as separate calls, as the reference launches the
 * stage-1 split kernel and the stage-2 LSE reduction separately (hla/vllm_latent/s6_ops.py:186-202,
 * _fwd_grouped_kernel_stage1 then _decode_softmax_reducev_fwd). hla_s6_history_partials writes the
 * per-split normalized partials and their lse to `workspace` for every num_splits >= 1 (same
 * arguments and checks as hla_s6_history_attention); hla_s6_history_reduce reads them back and writes
 * o and lse exactly as hla_s6_history_attention does (bitwise: the same kernels). The workspace layout
 * is private to the library: o partials [T][S][16][width] then lse [T][S][16], fp32. `plan` (nullable) is the
 * step's hla_s6_split_plan for (ctx, bt_cols * block_size, num_splits), as for hla_s6_attend_decode. */
int hla_s6_history_partials(const void *q, int32_t num_tokens, int32_t num_heads, int32_t width,
                            int64_t q_st, int64_t q_sh, const void *k_cache, const void *v_cache,
                            int64_t page_stride, int64_t row_stride, int32_t block_size, int64_t num_blocks,
                            const int32_t *block_table, int64_t bt_stride, int32_t bt_cols, const int64_t *bt_rows,
                            const int32_t *ctx, float scale, int32_t num_splits, float *workspace,
                            int64_t workspace_floats, const int32_t *plan, int64_t plan_len, void *stream);
int hla_s6_history_reduce(const float *workspace, int64_t workspace_floats, int32_t num_tokens, int32_t num_heads,
                          int32_t width, int32_t num_splits, void *out, int64_t o_st, int64_t o_sh, float *lse,
                          void *stream);

/* hla_s6_history_partials_grouped and hla_s6_split_epilogue: no counterpart in the reference. Together with
 * hla_s6_chunk_window_attention they replace the op sequence of s6_layer.attend for multi-token steps with split
 * history (hla/vllm_latent/s6_layer.py:101-115: history_attention, the B_t einsum, merge_states) by three launches:
 * hla_s6_history_partials_grouped runs the kernels of hla_s6_history_attention_grouped (group 2 or 4 tokens per
 * workgroup, same arguments and checks) but only writes the split partials to `workspace` (layout as for
 * hla_s6_history_partials; every slot is written, slots without keys with lse = -inf), and hla_s6_split_epilogue
 * (num_splits >= 2) reduces them by LSE, rounds o_hist to bf16 as the history op returns it, and writes
 * out = merge(bf16(o_hist @ B[h]), o_win) with the merge_states conventions (invalid rows zeroed; o_win
 * [T, 16, 128] bf16 and lse_win [16, T] contiguous, e.g. the chunk + window partial of
 * hla_s6_chunk_window_attention): the epilogue of hla_s6_attend_decode. */
int hla_s6_history_partials_grouped(const void *q, int32_t num_tokens, int32_t num_heads, int32_t width,
                                    int64_t q_st, int64_t q_sh, const void *k_cache, const void *v_cache,
                                    int64_t page_stride, int64_t row_stride, int32_t block_size, int64_t num_blocks,
                                    const int32_t *block_table, int64_t bt_stride, int32_t bt_cols,
                                    const int64_t *bt_rows, const int32_t *ctx, float scale, int32_t num_splits,
                                    float *workspace, int64_t workspace_floats, int32_t group, void *stream);
int hla_s6_split_epilogue(const float *workspace, int64_t workspace_floats, int32_t num_tokens, int32_t num_heads,
                          int32_t width, int32_t num_splits, const void *B, int64_t b_sh, int64_t b_sr,
                          const void *o_win, const float *lse_win, const uint8_t *invalid, void *out, int64_t o_st,
                          int64_t o_sh, void *stream);

/* ---- a6/a7: exact-window attention over the per-loop exact paged cache --------------------------
 * The exact cache is the TRITON_ATTN layout [num_blocks, block, H, 2d] (K then V per head); key row j of
 * head h is at k_cache + block_table[row*bt_stride + j / block_size] * page_stride
 * + (j % block_size) * row_stride + h * head_stride (likewise v_cache).
 * mode 0 replaces s6_ops.window_attention_fa (hla/vllm_latent/s6_ops.py:317-331): per-request tables
 *   (row = request of the token); query i of a request with Lq queries sits at p = seq_len - Lq + i and
 *   reads keys [max(0, p - window), p] (causal, window_size = (window, 0)); tokens >= query_start_loc[num_reqs]
 *   get o = 0, lse = -inf.
 * mode 1 replaces s6_ops.window_history_fa / s6_ops.window_attention (hla/vllm_latent/s6_ops.py:290-314,
 *   334-350): token t reads history rows [max(0, ctx[t] - window), ctx[t]) with row = bt_rows ? bt_rows[t] : t.
 * Keys at table columns >= bt_cols are not read and page ids are clamped into [0, num_blocks).
 * head_dim == 128. Outputs o [T, H, 128] bf16 and lse [H, T] fp32. */
int hla_s6_window_attention(const void *q, int32_t num_tokens, int32_t num_heads, int32_t head_dim, int64_t q_st,
                            int64_t q_sh, const void *k_cache, const void *v_cache, int64_t page_stride,
                            int64_t row_stride, int64_t head_stride, int32_t block_size, int64_t num_blocks,
                            const int32_t *block_table, int64_t bt_stride, int32_t bt_cols, const int64_t *bt_rows,
                            int32_t mode,
                            const int32_t *query_start_loc, const int32_t *seq_lens, int32_t num_reqs,
                            const int32_t *ctx, int32_t window, float scale, void *out, int64_t o_st,
                            int64_t o_sh, float *lse, void *stream);

/* ---- a7: causal current-chunk attention ---------------------------------------------------------
 * Replaces s6_ops.chunk_attention (hla/vllm_latent/s6_ops.py:234-259): token i of request r attends
 * causally to the tokens [query_start_loc[r], i] of its own chunk; tokens >= query_start_loc[num_reqs] get
 * o = 0, lse = -inf. q, k, v are [T, H, 128] bf16 with unit last stride. */
int hla_s6_chunk_attention(const void *q, const void *k, const void *v, int32_t num_tokens, int32_t num_heads,
                           int32_t head_dim, int64_t q_st, int64_t q_sh, int64_t k_st, int64_t k_sh,
                           int64_t v_st, int64_t v_sh, const int32_t *query_start_loc, int32_t num_reqs,
                           float scale, void *out, int64_t o_st, int64_t o_sh, float *lse, void *stream);

/* ---- a7+a6: causal current chunk and its exact window history in one softmax ----------------------
 * Replaces the prefill / mixed-step sequence of hla/vllm_latent/s6_layer.py:101-110: chunk_attention
 * (s6_ops.py:234-259), window_history_fa (s6_ops.py:334-350) and merge_lse (s6_ops.py:353-361). Every token of
 * request r attends to the exact-cache rows [ctx_r - window, ctx_r), ctx_r = seq_lens[r] - (query_start_loc[r+1] -
 * query_start_loc[r]), read through the per-request block_table (rows >= bt_cols * block_size are not read), and
 * causally to its own chunk tokens. Cache geometry as hla_s6_window_attention (K at k_cache, V at v_cache, same
 * strides). Tokens >= query_start_loc[num_reqs] get o = 0, lse = -inf. */
int hla_s6_chunk_window_attention(const void *q, const void *k, const void *v, int32_t num_tokens,
                                  int32_t num_heads, int32_t head_dim, int64_t q_st, int64_t q_sh, int64_t k_st,
                                  int64_t k_sh, int64_t v_st, int64_t v_sh, const int32_t *query_start_loc,
                                  const int32_t *seq_lens, int32_t num_reqs, const void *k_cache, const void *v_cache,
                                  int64_t page_stride, int64_t row_stride, int64_t head_stride, int32_t block_size,
                                  int64_t num_blocks, const int32_t *block_table, int64_t bt_stride, int32_t bt_cols,
                                  int32_t window, float scale, void *out, int64_t o_st, int64_t o_sh, float *lse,
                                  void *stream);

/* ---- a8: LSE merge of two partial attentions -----------------------------------------------------
 * mode 0 replaces s6_ops.merge_states (hla/vllm_latent/s6_ops.py:262-284): +inf lse counts as empty,
 *   both empty -> 0, rows with invalid[t] != 0 -> 0 (invalid nullable); lse_out must be NULL.
 * mode 1 replaces s6_ops.merge_lse (hla/vllm_latent/s6_ops.py:353-361): NaN inputs become 0, the merged
 *   lse = peak + log(w_a + w_b) is written to lse_out ([H, T] fp32, nullable).
 * head_dim % 8 == 0; o tensors need a unit last stride. */
int hla_s6_merge_states(const void *o_a, int64_t a_st, int64_t a_sh, const float *lse_a, const void *o_b,
                        int64_t b_st, int64_t b_sh, const float *lse_b, const uint8_t *invalid,
                        int32_t num_tokens, int32_t num_heads, int32_t head_dim, int32_t mode, void *out,
                        int64_t o_st, int64_t o_sh, float *lse_out, void *stream);

/* ---- split plan of a step (no reference counterpart: scheduling metadata of the split-KV kernels) -------
 * The history kernels cut every row of a step in chunks of `chunk` 16-row tiles, one chunk per slot (num_splits
 * slots per row), chunk = max(ceil(max_tiles / S), ceil(2 * total_tiles / (T * S)), min(max_tiles, floor)) with
 * tiles = ceil(min(ctx[t], cap) / 16) and floor = 4 when total_tiles < 768, else 8, grown one tile at a time until
 * the step has at most T * S / 2 chunks with work (or chunk = max_tiles),
 * and give the chunks to workgroups as one balanced list. hla_s6_split_plan computes that list once
 * per step (one small launch) into `plan` (int32, hla_s6_split_plan_ints(T, S) entries; caller-owned) so that every
 * fused decode call of the step reads it instead of deriving it per workgroup. It depends only on ctx, cap, S and
 * query_start_loc. cap = the latent table's columns * block_size. With query_start_loc (nullable; num_reqs + 1
 * entries), the tokens of a request of 2..16 tokens that all use the same number of slots (a short prefill chunk:
 * they read the same latent rows) have their chunks listed chunk-major, so one XCD reads each chunk for all of them
 * at about the same time. */
int64_t hla_s6_split_plan_ints(int32_t num_tokens, int32_t num_splits);
int hla_s6_split_plan(const int32_t *ctx, int32_t num_tokens, int64_t cap, int32_t num_splits,
                      const int32_t *query_start_loc, int32_t num_reqs, int32_t *plan, int64_t plan_len,
                      void *stream);
/* The plans of `count` (1..4) slot counts over the same ctx, cap and query_start_loc in one launch (one workgroup
 * per plan): a step's latent widths run different slot counts over the same rows. `num_splits`, `plans` (device
 * pointers) and `plan_lens` are host arrays of `count` entries; plan i equals hla_s6_split_plan's for
 * num_splits[i]. No reference counterpart. */
int hla_s6_split_plans(const int32_t *ctx, int32_t num_tokens, int64_t cap, int32_t count,
                       const int32_t *num_splits, const int32_t *query_start_loc, int32_t num_reqs,
                       int32_t *const *plans, const int64_t *plan_lens, void *stream);

/* ---- a9: fused decode attention of one layer x loop --------------------------------------------------
 * Replaces the decode branch of s6_layer.attend (hla/vllm_latent/s6_layer.py:97-100,110-115):
 * window_attention_fa + history_attention + the B_t einsum + merge_states, in two launches:
 *   1. the split kernel of hla_s6_history_partials over q_lat and the latent cache (per-request table
 *      `lat_table`, row of token t = token_requests[t], ctx_latent[t] rows); workgroups appended after the history
 *      ones compute the exact windows of the step over q_rope and the loop's exact cache: query i of a request with
 *      Lq queries (p = seq_len - Lq + i) reads the exact keys [max(0, seq_len - Lq - window), p] (for Lq = 1 the
 *      window_attention_fa keys [p - window, p] of mode 0 of hla_s6_window_attention; for a short prefill chunk the
 *      window history and the chunk's causal keys, which the caller has written to the exact cache);
 *   2. an epilogue that reduces the split partials by LSE (o_hist rounded to bf16 as the history op returns
 *      it), then writes out = merge(bf16(o_hist @ B[h]), o_win) with the merge_states conventions (invalid
 *      rows zeroed).
 * The intermediates o_hist [T, 16, width] bf16, lse_hist [16, T], o_win [T, 16, 128] bf16 and lse_win [16, T]
 * are caller-owned contiguous buffers: o_win / lse_win hold the exact-window partial on return, o_hist / lse_hist
 * the history partial when num_splits == 1 (with more slots it lives in the workspace). B is [16, width, 128]
 * with strides (b_sh, b_sr, 1). max_query_len > 1 (tokens of a request read the same latent rows) loads the rows
 * through the caches instead of streaming them. Workspace as for hla_s6_history_attention. `plan` (nullable,
 * plan_len ints) is the step's hla_s6_split_plan for (ctx_latent, lat_bt_cols * block_size, num_splits); without it
 * each workgroup derives its share itself. */
int hla_s6_attend_decode(const void *q_lat, int64_t ql_st, int64_t ql_sh, int32_t width, const void *lat_k,
                         const void *lat_v, int64_t lat_page_stride, int64_t lat_row_stride, int32_t block_size,
                         int64_t lat_num_blocks, const int32_t *lat_table, int64_t lat_bt_stride, int32_t lat_bt_cols,
                         const int64_t *token_requests, const int32_t *ctx_latent, const void *q_rope, int64_t qr_st,
                         int64_t qr_sh, const void *ex_k, const void *ex_v, int64_t ex_page_stride,
                         int64_t ex_row_stride, int64_t ex_head_stride, int32_t ex_block_size, int64_t ex_num_blocks,
                         const int32_t *ex_table, int64_t ex_bt_stride, int32_t ex_bt_cols,
                         const int32_t *query_start_loc, const int32_t *seq_lens, int32_t num_reqs, int32_t window,
                         const void *B, int64_t b_sh, int64_t b_sr, const uint8_t *invalid, int32_t num_tokens,
                         int32_t num_heads, float scale, int32_t num_splits, int32_t max_query_len,
                         float *workspace, int64_t workspace_floats, const int32_t *plan, int64_t plan_len,
                         void *o_hist, float *lse_hist, void *o_win, float *lse_win, void *out, int64_t o_st,
                         int64_t o_sh, void *stream);

/* hla_s6_attend_decode_static: no counterpart in the reference. hla_s6_attend_decode for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid allocation): the
 * same arguments without workspace, plan, o_hist, lse_hist, o_win and lse_win, which live in a static device array
 * of the library instead (48 MiB on every GPU the library runs on, held until the process ends). The caller passes
 * the inputs and `out`; the call computes the step's split plan itself (one extra small launch), then runs the
 * kernels of hla_s6_attend_decode, so `out` equals what hla_s6_attend_decode writes for the same inputs. It calls no
 * allocator. Sizes whose buffers exceed the array (T * S * 16 * (width + 1) floats of split partials plus the plan
 * and the window outputs, each rounded up to 256 bytes) return HLA_S6_EWORKSPACE before any launch. Calls on one
 * GPU share the array: calls that overlap in time on one GPU (other streams, other threads) race. */
int hla_s6_attend_decode_static(const void *q_lat, int64_t ql_st, int64_t ql_sh, int32_t width, const void *lat_k,
                                const void *lat_v, int64_t lat_page_stride, int64_t lat_row_stride,
                                int32_t block_size, int64_t lat_num_blocks, const int32_t *lat_table,
                                int64_t lat_bt_stride, int32_t lat_bt_cols, const int64_t *token_requests,
                                const int32_t *ctx_latent, const void *q_rope, int64_t qr_st, int64_t qr_sh,
                                const void *ex_k, const void *ex_v, int64_t ex_page_stride, int64_t ex_row_stride,
                                int64_t ex_head_stride, int32_t ex_block_size, int64_t ex_num_blocks,
                                const int32_t *ex_table, int64_t ex_bt_stride, int32_t ex_bt_cols,
                                const int32_t *query_start_loc, const int32_t *seq_lens, int32_t num_reqs,
                                int32_t window, const void *B, int64_t b_sh, int64_t b_sr, const uint8_t *invalid,
                                int32_t num_tokens, int32_t num_heads, float scale, int32_t num_splits,
                                int32_t max_query_len, void *out, int64_t o_st, int64_t o_sh, void *stream);

/* ---- a10 (slot-mapped row commit) -----------------------------------------------------------------
 * Slot of each token: block_table[token_requests[t], positions[t] / block_size] * block_size
 * + positions[t] % block_size, -1 for padding (valid[t] == 0). Closed form of
 * hla/tests/test_s6_serving.py:54 and the padding convention of hla/vllm_latent/ouro_latent.py:8-9.
 * A position beyond the table (column >= bt_cols) also maps to -1. */
int hla_s6_slot_mapping(const int32_t *block_table, int64_t bt_stride, int32_t bt_cols,
                        const int64_t *token_requests, const uint8_t *valid, const int64_t *positions,
                        int32_t num_tokens, int32_t block_size, int64_t *slots, void *stream);

/* Replaces unified_kv_cache_update of a committed latent row (hla/vllm_latent/ouro_latent.py:127-129):
 * the row [key[t, :width] | value[t, :width]] is stored at page slots[t] / block_size, row
 * slots[t] % block_size of `cache` (negative slots and slots past num_blocks * block_size skipped).
 * key/value need a unit last stride; rows move in 16-byte pieces when width % 8 == 0 and the rows are
 * 16-byte aligned, element by element otherwise. */
int hla_s6_store_rows(const void *key, int64_t k_st, const void *value, int64_t v_st, int32_t num_tokens,
                      int32_t width, const int64_t *slots, void *cache, int64_t page_stride, int64_t row_stride,
                      int32_t block_size, int64_t num_blocks, void *stream);

/* ---- writer (candidate projection, register accumulation, fused row commit) --------------------------
 * Replaces LatentLayer.write_step / write1 (hla/latent/register.py:45-61) as called by write_rows
 * (hla/vllm_latent/s6_layer.py:124-132), and, when `cache` is given, also committed_row
 * (hla/vllm_latent/s6_layer.py:135-147) plus its store (hla/vllm_latent/ouro_latent.py:127-129):
 *   u = bf16(h[t, :hidden] @ weight[n, :hidden]^T) for n < 2 * width   (nn.Linear, fp32 accumulation)
 *   r = prev ? bf16(prev[t, n] + u) : u;  reg[t, n] = r  (when reg != NULL; all num_tokens rows)
 *   cache row at slots[t] <- [RoPE_lat(r[:width]) by rope_table[positions[t]] | r[width:]]  (when cache != NULL;
 *   negative slots and slots past num_blocks * block_size skipped; rotation per element as latent_rope).
 * weight is the [2 * width, hidden] nn.Linear weight (w_st elements between rows); hidden must be a multiple
 * of 512 and width of 16; h and weight rows 16-byte aligned with a unit last stride. One launch. */
int hla_s6_write_rows(const void *h, int32_t num_tokens, int32_t hidden, int64_t h_st, const void *weight,
                      int32_t width, int64_t w_st, const void *prev, int64_t prev_st, void *reg, int64_t reg_st,
                      const int64_t *slots, const int64_t *positions, const void *rope_table, int32_t table_rows,
                      int64_t table_stride, void *cache, int64_t page_stride, int64_t row_stride,
                      int32_t block_size, int64_t num_blocks, void *stream);

/* ---- rollout cache (s6-rollout-cache-v1 export) ------------------------------------------------------
 * Replaces the per-layer gather of RolloutCacheExporter.export (hla/vllm_latent/cache_export.py:159-188):
 * out[l, pos, :] = [main_l[block_main[pos / bs_main], 0, pos % bs_main, :2r] |
 *                   l1_l[block_l1[pos / bs_l1], 0, pos % bs_l1, :2r1]]  for pos < length, every layer l,
 * i.e. the packed row layout of hla/latent/register.py:73-79. cache_addrs is a DEVICE array of 2 * num_layers
 * cache base addresses (main of layer l at 2l, loop-1 at 2l + 1); main_blocks / l1_blocks are the request's
 * device block lists, at least ceil(length / block_size) long; a block id outside [0, num_blocks) yields a zero
 * row. vector_ok != 0 promises 16-byte aligned cache bases (16-byte moves are then used when every row width and
 * stride allows them). One launch. */
int hla_s6_gather_packed_rows(const int64_t *cache_addrs, int32_t num_layers, int64_t main_page_stride,
                              int64_t main_row_stride, int32_t main_width, int64_t main_num_blocks,
                              const int32_t *main_blocks, int32_t main_block_size, int64_t l1_page_stride,
                              int64_t l1_row_stride, int32_t l1_width, int64_t l1_num_blocks,
                              const int32_t *l1_blocks, int32_t l1_block_size, int32_t length, void *out,
                              int64_t out_layer_stride, int64_t out_row_stride, int32_t vector_ok, void *stream);

/* ---- multi-query causal history attention with backward (K-hop replay / training) ---------------------------
 * Replaces causal_history_gemm (hla/latent/history_gemm.py:159-220,270-294) for bf16 GEMM operands with fp32
 * accumulation: q [B, Lq, 16, width] (strides q_sb, q_si, q_sh), k / v [B, N, width] (strides *_sb, *_sn), mask
 * [B, Lq, N] bytes (nonzero = visible; strides m_sb, m_si, unit last stride, m_si 0 for one row shown to every
 * query of a batch row; NULL = all keys below the bound),
 * width in {128, 256, 512}, bf16 rows 16-byte aligned with unit last stride.
 * hla_s6_khop_bounds: bound[b * Lq + i] = 1 + the last key mask row (b, i) shows (0 if none; N without a mask).
 * hla_s6_khop_forward: z [B, Lq, 16, width] bf16 and lse [B, 16, Lq] fp32 (natural log; -inf and z = 0 for a row
 *   without visible keys); one launch.
 * hla_s6_khop_backward: from dz [B, Lq, 16, width] bf16 and dlse [B, 16, Lq] (NULL = 0): delta = dz.z into
 *   `delta` [B, 16, Lq], then dq [B, Lq, 16, width] (NULL: skipped) and dk / dv [B, N, width] fp32 (both NULL:
 *   skipped). key_splits > 1 splits each key tile's query rows over that many workgroups, with fp32 partials in
 *   `workspace` (at least 2 * key_splits * B * N * width floats; dk / dv then contiguous) summed in a fixed order,
 *   so results are deterministic for a given key_splits. With grads_bf16 != 0, dq / dk / dv are bf16 arrays (the
 *   float pointers are reinterpreted, strides in bf16 elements), each value the fp32 result rounded to nearest
 *   even. Up to 5 launches. */
int hla_s6_khop_bounds(const uint8_t *mask, int64_t m_sb, int64_t m_si, int32_t B, int32_t Lq, int32_t N,
                       int32_t *bound, void *stream);
int hla_s6_khop_forward(const void *q, int64_t q_sb, int64_t q_si, int64_t q_sh, const void *k, int64_t k_sb,
                        int64_t k_sn, const void *v, int64_t v_sb, int64_t v_sn, const uint8_t *mask, int64_t m_sb,
                        int64_t m_si, const int32_t *bound, int32_t B, int32_t Lq, int32_t N, int32_t heads,
                        int32_t width, float scale, void *z, int64_t z_sb, int64_t z_si, int64_t z_sh, float *lse,
                        void *stream);
/* hla_s6_khop_backward_workspace: the workspace floats hla_s6_khop_backward uses for these sizes and key_splits:
 *   the dk / dv partials (2 * key_splits * B * N * width with key_splits > 1) or, when few token groups leave the
 *   GPU idle (B * ceil(Lq / 4) < 128, widths 512 / 256, N a multiple of 16), dq partials over key ranges (then dq
 *   must be contiguous), whichever is larger; with less workspace dq runs without key ranges. */
int64_t hla_s6_khop_backward_workspace(int32_t B, int32_t Lq, int32_t N, int32_t width, int32_t key_splits);
int hla_s6_khop_backward(const void *q, int64_t q_sb, int64_t q_si, int64_t q_sh, const void *k, int64_t k_sb,
                         int64_t k_sn, const void *v, int64_t v_sb, int64_t v_sn, const uint8_t *mask, int64_t m_sb,
                         int64_t m_si, const int32_t *bound, int32_t B, int32_t Lq, int32_t N, int32_t heads,
                         int32_t width, float scale, const void *z, int64_t z_sb, int64_t z_si, int64_t z_sh,
                         const float *lse, const void *dz, int64_t dz_sb, int64_t dz_si, int64_t dz_sh,
                         const float *dlse, float *delta, float *dq, int64_t dq_sb, int64_t dq_si, int64_t dq_sh,
                         float *dk, int64_t dk_sb, int64_t dk_sn, float *dv, int64_t dv_sb, int64_t dv_sn,
                         int32_t key_splits, float *workspace, int64_t workspace_floats, int32_t grads_bf16,
                         void *stream);

/* ---- the same in fp32 arithmetic (the reference's default precision) ------------------------------------------
 * Replace causal_history_gemm with precision 'fp32' / 'tf32' (hla/latent/history_gemm.py:19-24,37,46-66,270-294)
 * and causal_history_attention's fp32 'triton' / 'reference' backends (hla/latent/fused_history.py:62-153):
 * every GEMM on fp32 MFMA (fp32 operands, fp32 accumulation), softmax in fp32. Arguments as hla_s6_khop_forward /
 * hla_s6_khop_backward with fp32 q / k / v / z / dz (rows 16-byte aligned, unit last stride), width in {128, 256,
 * 512, 1024}, no grads_bf16 (dq / dk / dv are fp32). z is the fp32 forward output (delta = dz.z uses it).
 * key_splits > 1 splits each key block's query tokens into that many ranges, with fp32 partials in `workspace` (at
 * least hla_s6_khop_backward_f32_workspace floats; dk / dv then contiguous) summed in a fixed order: deterministic
 * for a given key_splits. The forward is one launch, the backward up to 5. */
int hla_s6_khop_forward_f32(const float *q, int64_t q_sb, int64_t q_si, int64_t q_sh, const float *k, int64_t k_sb,
                            int64_t k_sn, const float *v, int64_t v_sb, int64_t v_sn, const uint8_t *mask,
                            int64_t m_sb, int64_t m_si, const int32_t *bound, int32_t B, int32_t Lq, int32_t N,
                            int32_t heads, int32_t width, float scale, float *z, int64_t z_sb, int64_t z_si,
                            int64_t z_sh, float *lse, void *stream);
/* hla_s6_khop_backward_f32_workspace: 2 * key_splits * B * N * width floats with key_splits > 1, else 0. */
int64_t hla_s6_khop_backward_f32_workspace(int32_t B, int32_t Lq, int32_t N, int32_t width, int32_t key_splits);
int hla_s6_khop_backward_f32(const float *q, int64_t q_sb, int64_t q_si, int64_t q_sh, const float *k, int64_t k_sb,
                             int64_t k_sn, const float *v, int64_t v_sb, int64_t v_sn, const uint8_t *mask,
                             int64_t m_sb, int64_t m_si, const int32_t *bound, int32_t B, int32_t Lq, int32_t N,
                             int32_t heads, int32_t width, float scale, const float *z, int64_t z_sb, int64_t z_si,
                             int64_t z_sh, const float *lse, const float *dz, int64_t dz_sb, int64_t dz_si,
                             int64_t dz_sh, const float *dlse, float *delta, float *dq, int64_t dq_sb, int64_t dq_si,
                             int64_t dq_sh, float *dk, int64_t dk_sb, int64_t dk_sn, float *dv, int64_t dv_sb,
                             int64_t dv_sn, int32_t key_splits, float *workspace, int64_t workspace_floats,
                             void *stream);

/* ---- single-query history attention over contiguous rows with a key mask (HF rolling engine) ---------------
 * Replaces the forward of fused_history.history_attention (hla/latent/fused_history.py:23-35,49-54; Triton
 * _forward, hla/latent/history_kernels.py:11-33): q [B, 16, width] (strides q_sb, q_sh), k / v [B, N, width] with
 * the same strides (kv_sb, kv_sn), mask [B, N] bytes (nonzero = visible; row stride m_sb, unit last stride; NULL =
 * every key below the bound), bound [B] = 1 + the last visible key (hla_s6_khop_bounds with Lq = 1). Writes z
 * [B, 16, width] bf16 (strides z_sb, z_sh) and lse [B, 16] fp32 (natural log; z = 0 and lse = -inf for a row with no
 * visible key). width in {128, 256, 512, 1024}; num_splits > 1 splits each row's keys over that many workgroups
 * (workspace of at least B * num_splits * 16 * (width + 1) floats) and adds the reduction launch. The backward is
 * hla_s6_khop_backward with Lq = 1. */
int hla_s6_masked_history(const void *q, int64_t q_sb, int64_t q_sh, const void *k, const void *v, int64_t kv_sb,
                          int64_t kv_sn, const uint8_t *mask, int64_t m_sb, const int32_t *bound, int32_t B,
                          int32_t N, int32_t num_heads, int32_t width, float scale, int32_t num_splits,
                          float *workspace, int64_t workspace_floats, void *z, int64_t z_sb, int64_t z_sh,
                          float *lse, void *stream);

/* ---- a11: the HF rolling engine's current-chunk attention with backward ----------------------------------
 * Replaces the exact part of batched_engine.mixed_attention (hla/latent/batched_engine.py:156-162): per batch row
 * and head, one softmax of the chunk's queries over its keys, q / k / v [B, 16, n, 128] bf16 (strides (sb, sh, si),
 * unit last) already RoPE'd, scores scaled by `scale`; valid [B, n] bytes (row stride valid_sb): a valid query i
 * sees the valid keys j <= i, an invalid query every key of the chunk (batched_engine.py:157-160). Forward: o
 * [B, 16, n, 128] fp32, lse [B, 16, n] fp32 (natural log, strides (l_sb, l_sh, 1)); one launch. Backward: from dout
 * (fp32, o's layout) and dlse (nullable, lse's layout): delta = dout . o into `delta` (lse's layout), then dq, dk,
 * dv fp32 [B, 16, n, 128] (strides (g_sb, g_sh, g_si)); two launches. */
int hla_s6_hf_chunk_forward(const void *q, int64_t q_sb, int64_t q_sh, int64_t q_si, const void *k, int64_t k_sb,
                            int64_t k_sh, int64_t k_si, const void *v, int64_t v_sb, int64_t v_sh, int64_t v_si,
                            const uint8_t *valid, int64_t valid_sb, int32_t B, int32_t heads, int32_t n,
                            int32_t head_dim, float scale, float *o, int64_t o_sb, int64_t o_sh, int64_t o_si,
                            float *lse, int64_t l_sb, int64_t l_sh, void *stream);
int hla_s6_hf_chunk_backward(const void *q, int64_t q_sb, int64_t q_sh, int64_t q_si, const void *k, int64_t k_sb,
                             int64_t k_sh, int64_t k_si, const void *v, int64_t v_sb, int64_t v_sh, int64_t v_si,
                             const uint8_t *valid, int64_t valid_sb, int32_t B, int32_t heads, int32_t n,
                             int32_t head_dim, float scale, const float *o, int64_t o_sb, int64_t o_sh, int64_t o_si,
                             const float *lse, int64_t l_sb, int64_t l_sh, const float *dout, int64_t d_sb,
                             int64_t d_sh, int64_t d_si, const float *dlse, float *delta, float *dq, float *dk,
                             float *dv, int64_t g_sb, int64_t g_sh, int64_t g_si, void *stream);

/* ---- a11: the joint softmax's merge and B_t projection with backward ------------------------------------------
 * Replaces the LSE merge and the B_t product of batched_engine.mixed_attention (hla/latent/batched_engine.py:
 * 171-181): with the chunk part (o_c [B, H, n, 128] fp32, strides (oc_sb, oc_sh, oc_si), unit last; lse_c [B, H, n]
 * fp32 contiguous) and `parts` (1 to 8) history blocks (z[p] [B, H, n, width] bf16, strides z_strides[3p ..
 * 3p+2] = (sb, sh, si), unit last; lse_z[p] [B, H, n] fp32 contiguous; -inf where the query sees no row of the
 * block), w_j = exp(lse_j - logsumexp(lse_c, lse_z[0], ..)) and
 *   out = bf16(w_c o_c + bf16(sum_p w_p z[p]) @ Bt[h])      (Bt [H, width, 128] bf16, strides (b_sh, b_sr, 1))
 * into out [B, H, n, 128] bf16 (strides (o_sb, o_sh, o_si)); a query with no key anywhere gets 0. width in
 * {256, 512}, head_dim 128. `z`, `z_strides`, `lse_z` (and `dz`, `dz_strides`, `d_lse_z`) are host arrays of
 * `parts` entries holding device pointers. One launch each.
 * Backward, from dout [B, H, n, 128] bf16 (strides (do_sb, do_sh, do_si)): d_oc = w_c dout (fp32, o_c's layout
 * with its own strides), dz[p] = bf16(w_p dout @ Bt[h]^T) (z's layout with its own strides), d_lse_c and
 * d_lse_z[p] = w_j (a_j - <dout, out>) with a_c = <dout, o_c>, a_p = <dout @ Bt[h]^T, z[p]> (fp32, lse layout).
 * The gradient of Bt is not computed here. */
int hla_s6_mixed_merge_forward(int32_t batch, int32_t num_heads, int32_t chunk, int32_t width, int32_t head_dim,
                               const float *o_c, int64_t oc_sb, int64_t oc_sh, int64_t oc_si, const float *lse_c,
                               int32_t parts, const void *const *z, const int64_t *z_strides,
                               const float *const *lse_z, const void *Bt, int64_t b_sh, int64_t b_sr, void *out,
                               int64_t o_sb, int64_t o_sh, int64_t o_si, void *stream);
int hla_s6_mixed_merge_backward(int32_t batch, int32_t num_heads, int32_t chunk, int32_t width, int32_t head_dim,
                                const float *o_c, int64_t oc_sb, int64_t oc_sh, int64_t oc_si, const float *lse_c,
                                int32_t parts, const void *const *z, const int64_t *z_strides,
                                const float *const *lse_z, const void *Bt, int64_t b_sh, int64_t b_sr,
                                const void *dout, int64_t do_sb, int64_t do_sh, int64_t do_si, float *d_oc,
                                int64_t doc_sb, int64_t doc_sh, int64_t doc_si, float *d_lse_c, void *const *dz,
                                const int64_t *dz_strides, float *const *d_lse_z, void *stream);

/* a11: RoPE of the chunk's queries and keys (batched_engine.py:156 with register.apply_rope, register.py:14-20):
 * y = bf16(x cos + rotate_half(x) sin) for `count` (1 or 2) tensors x[t] [B, H, n, d] bf16 (strides x_strides[3t ..
 * 3t+2] = (sb, sh, si), unit last) into y[t] (bf16, its own strides), cos / sin [B, n, d] broadcast over the heads
 * (strides (c_sb, c_si, 1), both tables alike, 16-byte aligned rows; fp32, or bf16 with trig_bf16 != 0), evaluated as torch does: each
 * product and the sum rounded to the tables' precision, then once to bf16. Backward: dx[t] = bf16(bf16(dy cos) +
 * rotate_half^T(bf16(dy sin))) from dy[t] fp32 (its own strides), the roundings of autograd for a bf16 x. `x`, `y`,
 * `dy`, `dx` and their strides are host arrays of `count` entries. d a multiple of 16, rows 16-byte aligned
 * (strides multiples of 8 elements); one launch each. */
int hla_s6_rope_rows_forward(int32_t count, const void *const *x, const int64_t *x_strides, void *const *y,
                             const int64_t *y_strides, int32_t batch, int32_t num_heads, int32_t chunk,
                             int32_t head_dim, const void *cos, const void *sin, int64_t c_sb, int64_t c_si,
                             int32_t trig_bf16, void *stream);
int hla_s6_rope_rows_backward(int32_t count, const float *const *dy, const int64_t *dy_strides, void *const *dx,
                              const int64_t *dx_strides, int32_t batch, int32_t num_heads, int32_t chunk,
                              int32_t head_dim, const void *cos, const void *sin, int64_t c_sb, int64_t c_si,
                              int32_t trig_bf16, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HLA_S6_H */
