/*
 * delta_hip.h -- C ABI of the MI355X (gfx950) selective-KV decode hot path.
 *
 * The library (delta_amd/_delta_hip.so) replaces the device work behind the
 * reference's torch.library ops and planner helpers (hoenza/DELTA):
 *
 *   FlashInfer BatchPrefillWithPagedKVCacheWrapper.run  (backend.py:461-512)
 *   FlashInfer JIT BatchDumpAttentionWeights + run      (backend.py:175-222, 518-585)
 *   _compute_page_scores_from_attention_buffer_legacy_softmax (backend.py:887-904)
 *   PageSelectorV2.select / _prepare_scores             (page_selector_v2.py:113-212)
 *   Triton _pack_page_indices_kernel                    (page_metadata.py:6-70)
 *   _collect_decode_page_info_fast (device half)        (backend.py:2040-2172)
 *   FlashInfer append_paged_kv_cache (mylib::update_kv) (utils.py:31-79)
 *   FlashInfer apply_rope / apply_llama31_rope          (model.py:152-175)
 *
 * Conventions shared by every entry point:
 *   - all pointers are device pointers unless stated; sizes and strides are in
 *     ELEMENTS of the pointed-to type;
 *   - the paged KV cache is [num_pages, 2, page_size=16, num_kv_heads, head_dim=128]
 *     (model.py:102), K at [:,0], V at [:,1]; dtype bf16 (DELTA_BF16) or fp16
 *     (DELTA_FP16);
 *   - page tables are CSR: kv_indptr [batch+1], kv_indices [kv_indices_len],
 *     kv_last_page_len [batch] in [0,16]; row b holds
 *     (pages_b - 1) * 16 + last_page_len_b tokens;
 *   - kernels never allocate, never synchronise and never read host memory, so
 *     every call can be recorded in a hipGraph; caller-provided workspaces are
 *     sized by the *_workspace_bytes queries and 256-byte aligned;
 *   - out-of-range page ids / indptr entries are masked (the kernel never
 *     faults on a bad table, it drops the offending pages);
 *   - return 0 on success; otherwise a non-zero code and delta_last_error()
 *     (thread local) describes the failure.
 */
#ifndef DELTA_HIP_H_
#define DELTA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *delta_stream_t; /* a hipStream_t (0 = the null stream) */

enum {
  DELTA_BF16 = 0,
  DELTA_FP16 = 1,
};

enum {
  DELTA_OK = 0,
  DELTA_ERR_INVALID = 1,   /* bad argument (shape, dtype, null pointer, size) */
  DELTA_ERR_WORKSPACE = 2, /* workspace too small */
  DELTA_ERR_HIP = 3,       /* a HIP runtime call failed */
};

/* Last error message of the calling thread ("" when none). */
const char *delta_last_error(void);

/* ABI version (major * 100 + minor). */
int delta_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Paged decode attention (one query token per row)                          */
/* ------------------------------------------------------------------------ */

/* Most split-K work units a row is cut into for this shape (1 = unsplit).  A
 * split launch cuts each row into clamp(ceil(pages_b / chunk), 1, splits)
 * units of at most 128 pages and packs them row by row, so ragged rows cost in
 * proportion to their pages.  Depends only on its arguments, so a value
 * computed at graph capture stays valid for every replay.  max_pages_per_row
 * is the planned maximum of pages_b (a longer row is still covered whole: its
 * last unit takes the remainder). */
int delta_decode_num_splits(int batch, int num_kv_heads, int max_pages_per_row);

/* Bytes of workspace delta_paged_decode needs: 0 when the shape runs unsplit,
 * else the split partials, one slot per (row, split) (no initial contents
 * needed; calls that share a workspace must not overlap). */
size_t delta_paged_decode_workspace_bytes(int batch, int num_qo_heads, int num_kv_heads,
                                          int max_pages_per_row);

/* o[b,h,:] = softmax(q[b,h,:] . K_b[:, h/G, :] * sm_scale) @ V_b[:, h/G, :].
 *
 * Replaces BatchPrefillWithPagedKVCacheWrapper.run with causal=True and
 * qo_len=1 per row (backend.py:461-484 target_decode over the full CSR,
 * backend.py:486-512 target_subset_decode over the subset CSR; plan at
 * backend.py:1091-1105).
 *
 *   q   [batch, num_qo_heads, 128] with row stride q_stride_b, head stride q_stride_h
 *   o   [batch, num_qo_heads, 128] with strides o_stride_b / o_stride_h (same dtype)
 *   lse [batch, num_qo_heads] fp32 natural-log log-sum-exp of the scaled logits
 *       (-inf for an empty row), or NULL
 *   logits_dump (planner layer, or NULL): fp32, receives
 *       dump[b*dump_stride_b + h*dump_stride_h + t] = (q.k_t) * sm_scale for t < kv_len_b,
 *       exactly the BatchDumpAttentionWeights side write (backend.py:207-219).
 *       Whole pages are written: t in [kv_len_b, pages_b * 16) receives -inf
 *       (the value the reference's -inf-filled buffer holds there,
 *       backend.py:384-389); nothing at or past pages_b * 16, nor past
 *       max_pages_per_row * 16, is touched.  Strides non-negative, 4-byte
 *       aligned, (G - 1) * dump_stride_h <= 2^28.
 *   num_qo_heads % num_kv_heads == 0 and num_qo_heads / num_kv_heads <= 8.
 */
int delta_paged_decode(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                       const void *kv_cache, int64_t num_pages,
                       const int32_t *kv_indptr, const int32_t *kv_indices,
                       int64_t kv_indices_len, const int32_t *kv_last_page_len,
                       void *o, int64_t o_stride_b, int64_t o_stride_h, float *lse,
                       float *logits_dump, int64_t dump_stride_b, int64_t dump_stride_h,
                       int batch, int num_qo_heads, int num_kv_heads, int head_dim,
                       int dtype, float sm_scale, int max_pages_per_row,
                       void *workspace, size_t workspace_bytes, delta_stream_t stream);

/* delta_paged_decode without a workspace argument: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under hipGraph capture, serving loops or
 * harnesses that forbid hipMalloc): the split-K partials live in a static 64 MiB device array
 * of the library (one per GPU, held until the process ends; its address is looked up on the
 * first call on each device), so the call allocates nothing.  A shape whose partials exceed
 * 64 MiB (delta_paged_decode_workspace_bytes) is rejected with DELTA_ERR_INVALID.  The array
 * needs no initial contents, but it is shared by every call on one GPU: calls that overlap on
 * one GPU (concurrent streams, threads) race and must be serialised by the caller.  Results are
 * bit-identical to delta_paged_decode. */
int delta_paged_decode_noalloc(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                               const void *kv_cache, int64_t num_pages,
                               const int32_t *kv_indptr, const int32_t *kv_indices,
                               int64_t kv_indices_len, const int32_t *kv_last_page_len,
                               void *o, int64_t o_stride_b, int64_t o_stride_h, float *lse,
                               float *logits_dump, int64_t dump_stride_b, int64_t dump_stride_h,
                               int batch, int num_qo_heads, int num_kv_heads, int head_dim,
                               int dtype, float sm_scale, int max_pages_per_row,
                               delta_stream_t stream);

/* The same attention over a *selected* page subset (the subset CSR built by
 * delta_select_pages, sharing kv_last_page_len with the full CSR):
 * target_subset_decode (backend.py:486-512).  Separate entry point (and
 * kernel name) so profiles tell the selective layers from the full ones. */
int delta_paged_decode_subset(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                              const void *kv_cache, int64_t num_pages,
                              const int32_t *kv_indptr, const int32_t *kv_indices,
                              int64_t kv_indices_len, const int32_t *kv_last_page_len,
                              void *o, int64_t o_stride_b, int64_t o_stride_h, float *lse,
                              int batch, int num_qo_heads, int num_kv_heads, int head_dim,
                              int dtype, float sm_scale, int max_pages_per_row,
                              void *workspace, size_t workspace_bytes, delta_stream_t stream);

/* The decode step's RoPE and KV append, fused into the attention launch
 * (Attention.forward, model.py:413-418: mylib::rope, then mylib::update_kv, then the
 * attention op -- here one launch).  Decode steps only: one new token per row.
 *   k, v        [batch, num_kv_heads, 128] the new token's k (before RoPE) and v, row
 *               strides k_stride / v_stride (even), 4-byte aligned
 *   offsets     [batch] the new token's position (its rotation angle), as delta_rope
 *   kv_indptr / kv_indices / kv_indices_len   the cache's full CSR: row b's new token
 *               goes to position kv_len_b - 1 of it (kv_len from kv_last_page_len), the
 *               slot delta_append_kv uses; a row without a valid slot appends nothing
 *   rope_scale, rope_theta, llama31, low/high_freq_factor, old_context_len   as delta_rope
 * The attention entry points that take it treat q as the un-rotated query.  Outputs,
 * the cache bytes, lse and the logits dump are bit-identical to delta_rope_append
 * followed by the plain entry point. */
typedef struct delta_decode_append {
  const void *k;
  int64_t k_stride;
  const void *v;
  int64_t v_stride;
  const int32_t *offsets;
  const int32_t *kv_indptr;
  const int32_t *kv_indices;
  int64_t kv_indices_len;
  float rope_scale;
  float rope_theta;
  int llama31;
  float low_freq_factor;
  float high_freq_factor;
  float old_context_len;
} delta_decode_append_t;

/* delta_paged_decode with the new token's RoPE and append fused in (see above).  No
 * counterpart entry point in the reference: it replaces the three calls of one decode
 * layer.  kv_cache is written (the new token's slot). */
int delta_paged_decode_append(const delta_decode_append_t *append, const void *q, int64_t q_stride_b,
                              int64_t q_stride_h, void *kv_cache, int64_t num_pages,
                              const int32_t *kv_indptr, const int32_t *kv_indices,
                              int64_t kv_indices_len, const int32_t *kv_last_page_len,
                              void *o, int64_t o_stride_b, int64_t o_stride_h, float *lse,
                              float *logits_dump, int64_t dump_stride_b, int64_t dump_stride_h,
                              int batch, int num_qo_heads, int num_kv_heads, int head_dim,
                              int dtype, float sm_scale, int max_pages_per_row,
                              void *workspace, size_t workspace_bytes, delta_stream_t stream);

/* delta_paged_decode_subset with the new token's RoPE and append fused in: attention over
 * the subset CSR, the append into the full CSR of `append`. */
int delta_paged_decode_subset_append(const delta_decode_append_t *append, const void *q,
                                     int64_t q_stride_b, int64_t q_stride_h, void *kv_cache,
                                     int64_t num_pages, const int32_t *kv_indptr,
                                     const int32_t *kv_indices, int64_t kv_indices_len,
                                     const int32_t *kv_last_page_len, void *o, int64_t o_stride_b,
                                     int64_t o_stride_h, float *lse, int batch, int num_qo_heads,
                                     int num_kv_heads, int head_dim, int dtype, float sm_scale,
                                     int max_pages_per_row, void *workspace, size_t workspace_bytes,
                                     delta_stream_t stream);

/* Causal attention of several query tokens per row (prompt steps): FlashInfer
 * BatchPrefillWithPagedKVCacheWrapper.run with causal=True (backend.py:1091-1105).
 * q/o are [nnz, num_qo_heads, 128] (token stride, head stride), row b's tokens at
 * qo_indptr[b] .. qo_indptr[b+1]; the cache already holds them (update_kv runs first,
 * model.py:413-418), so token i of row b sits at kv_len_b - qo_len_b + i and attends
 * tokens 0 .. that position.  lse [nnz, num_qo_heads] or NULL.  max_qo_len must be
 * >= every qo_len_b (it sizes the grid).  o 8-byte aligned with strides in multiples of 4.
 * No workspace. */
int delta_paged_prefill(const void *q, int64_t q_stride_t, int64_t q_stride_h,
                        const void *kv_cache, int64_t num_pages, const int32_t *qo_indptr,
                        const int32_t *kv_indptr, const int32_t *kv_indices,
                        int64_t kv_indices_len, const int32_t *kv_last_page_len, void *o,
                        int64_t o_stride_t, int64_t o_stride_h, float *lse, int batch,
                        int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
                        float sm_scale, int max_qo_len, delta_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Page scoring (del3_legacy_softmax)                                         */
/* ------------------------------------------------------------------------ */

/* scores[b, j] = sum_{t in page j} max_h softmax_t(dump[b, h, :max_pages*16])
 * for b < batch, j < max_pages (backend.py:887-904).
 *
 * dump is the planner logits buffer (layout as in delta_paged_decode);
 * positions t >= kv_len_b are treated as -inf (the reference's -inf fill,
 * backend.py:384-389) and never read.  kv_indptr/kv_last_page_len give
 * kv_len_b.  lse (natural log, [batch, num_qo_heads], as written by
 * delta_paged_decode for the same dump) may be NULL, in which case the
 * softmax normaliser is computed from the dump in a first pass (then
 * workspace must hold delta_page_score_workspace_bytes).  scores has row
 * stride score_stride (>= max_pages). */
size_t delta_page_score_workspace_bytes(int batch, int num_qo_heads);
int delta_page_scores_from_logits(const float *logits_dump, int64_t dump_stride_b,
                                  int64_t dump_stride_h, const float *lse,
                                  const int32_t *kv_indptr, const int32_t *kv_last_page_len,
                                  float *scores, int64_t score_stride, int batch,
                                  int num_qo_heads, int max_pages, void *workspace,
                                  size_t workspace_bytes, delta_stream_t stream);

/* Standalone scorer: reads the paged K cache once (no V) and writes the page
 * scores.  Replaces the dump attention kernel + legacy-softmax torch ops for a
 * caller that only needs scores (backend.py:561-577 + 887-904).  With a
 * logits_dump (caller-provided, layout as above, >= max_pages*16 per (b,h)
 * row) the fp32 logits are written there too.  With logits_dump == NULL the
 * scorer keeps each row's logits on chip -- allowed when
 * delta_page_score_needs_dump(...) == 0 (batch * num_kv_heads >= 256 and the
 * row's logits fit in LDS), else an error -- and writes no logits. */
size_t delta_page_score_kv_workspace_bytes(int batch, int num_qo_heads, int num_kv_heads,
                                           int max_pages_per_row);
int delta_page_score_needs_dump(int batch, int num_qo_heads, int num_kv_heads, int max_pages_per_row);
int delta_page_score(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                     const void *kv_cache, int64_t num_pages, const int32_t *kv_indptr,
                     const int32_t *kv_indices, int64_t kv_indices_len,
                     const int32_t *kv_last_page_len, float *logits_dump,
                     int64_t dump_stride_b, int64_t dump_stride_h, float *scores,
                     int64_t score_stride, int batch, int num_qo_heads, int num_kv_heads,
                     int head_dim, int dtype, float sm_scale, int max_pages,
                     void *workspace, size_t workspace_bytes, delta_stream_t stream);

/* The planner layer without a logits dump: full attention (o, lse, as delta_paged_decode)
 * and the del3_legacy_softmax page scores (as delta_page_scores_from_logits over the dump
 * the same launch would write) in one pass over K and V.  Replaces the pair
 * BatchDumpAttentionWeights.run + _compute_page_scores_from_attention_buffer_legacy_softmax
 * (backend.py:561-577 + 887-904) when the caller needs no dump (no debug parity check).
 * Each (row, kv head) keeps its logits on chip, so it applies when
 * delta_paged_decode_scores_supported(...) == 1 (batch * num_kv_heads >= 256 and the row's
 * logits fit in LDS); else it is an error and the caller uses the dump.  o and lse agree with
 * delta_paged_decode to rounding (another summation order); scores are written for pages
 * [0, max_pages) of each row (past the row: 0).  workspace: delta_paged_decode_scores_
 * workspace_bytes, 256-byte aligned.  The _append variant fuses the new token's RoPE and
 * append as delta_paged_decode_append does. */
int delta_paged_decode_scores_supported(int batch, int num_qo_heads, int num_kv_heads,
                                        int max_pages_per_row, int with_append);
size_t delta_paged_decode_scores_workspace_bytes(int batch, int num_kv_heads, int max_pages_per_row);
int delta_paged_decode_scores(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                              const void *kv_cache, int64_t num_pages, const int32_t *kv_indptr,
                              const int32_t *kv_indices, int64_t kv_indices_len,
                              const int32_t *kv_last_page_len, void *o, int64_t o_stride_b,
                              int64_t o_stride_h, float *lse, float *scores, int64_t score_stride,
                              int batch, int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
                              float sm_scale, int max_pages_per_row, void *workspace,
                              size_t workspace_bytes, delta_stream_t stream);
int delta_paged_decode_scores_append(const delta_decode_append_t *append, const void *q,
                                     int64_t q_stride_b, int64_t q_stride_h, void *kv_cache,
                                     int64_t num_pages, const int32_t *kv_indptr,
                                     const int32_t *kv_indices, int64_t kv_indices_len,
                                     const int32_t *kv_last_page_len, void *o, int64_t o_stride_b,
                                     int64_t o_stride_h, float *lse, float *scores,
                                     int64_t score_stride, int batch, int num_qo_heads,
                                     int num_kv_heads, int head_dim, int dtype, float sm_scale,
                                     int max_pages_per_row, void *workspace, size_t workspace_bytes,
                                     delta_stream_t stream);

/* ------------------------------------------------------------------------ */
/* PageSelectorV2 (top-k page selection)                                     */
/* ------------------------------------------------------------------------ */

/* Selects pages per row exactly as PageSelectorV2.select
 * (page_selector_v2.py:113-212) with ties broken by the smaller page index:
 *
 *   key_j = nan_to_num(score_j, nan=-inf, neginf=-inf) + fp32(-j * pos_bias_scale)
 *   key_j = +inf for j in [max(tp-L,0), tp);  pages j >= tp are not candidates
 *   top-k of key (key desc, j asc), emitted in ascending j as
 *   block_table[b * bt_stride + j].
 *
 * tp_b = kv_indptr[b+1] - kv_indptr[b].  k_b = k, or k_per_row[b] when
 * k_per_row != NULL (extension: per-row budgets).
 *   fixed_count = 0 (general path, 136-164): row b emits min(tp_b, k_b) pages
 *                 and out_indptr = cumsum.
 *   fixed_count = 1 (fixed path, 166-188): row b emits k_b pages and
 *                 out_indptr[b] = b * k (requires k_per_row == NULL).
 * use_subset (optional, device int): when non-NULL and *use_subset == 0 the
 * row's full page list block_table[b, :tp_b] is emitted (the engine's
 * "subset == full" step).  out_indices holds out_indices_len entries (sum of
 * the row counts is needed; writes past it are dropped).  max_pages (Nmax)
 * bounds the columns: tp_b is clamped to it (the reference's Nmax is the
 * largest tp_b, so this never binds there). */
int delta_select_pages(const float *scores, int64_t score_stride, const int32_t *kv_indptr,
                       const int32_t *block_table, int64_t bt_stride, int batch,
                       int max_pages, int k, const int32_t *k_per_row, int L,
                       float pos_bias_scale, int fixed_count, const int32_t *use_subset,
                       int32_t *out_indices, int64_t out_indices_len, int32_t *out_indptr,
                       delta_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Page-table metadata                                                        */
/* ------------------------------------------------------------------------ */

/* In-place pack of page lists (page_metadata.py:6-70): row r copies
 * slot_block_table[active_slots[r] * pages_per_slot + start_cols[r] + c] for
 * c < counts[r] to out_indices[indptr[r] + c] and, when write_row_block, to
 * row_block_table[r * pages_per_slot + c].  slot_block_table has num_slots
 * rows; a row whose slot, columns or destination fall outside the tables
 * (num_slots, pages_per_slot, out_indices_len) is skipped. */
int delta_pack_page_indices(const int32_t *slot_block_table, int num_slots,
                            const int32_t *active_slots, const int32_t *start_cols,
                            const int32_t *counts, const int32_t *indptr,
                            int32_t *out_indices, int64_t out_indices_len,
                            int32_t *row_block_table, int n_rows, int pages_per_slot,
                            int max_count, int write_row_block, delta_stream_t stream);

/* Device-side decode page info for rows 0..batch-1 of a slot block table
 * (backend.py:2040-2172 with scheduler.py:60-66), so a decode step needs no
 * host work: for each row, kv_len = cachelens[b] + 1, pages = kv_len/16 + 1,
 * last = kv_len % 16.  Writes kv_indptr (cumsum), kv_indices (packed from
 * slot_block_table), kv_last_page_len, row_block_table [batch, pages_per_slot]
 * (optional), the subset CSR (subset_indices/subset_indptr, optional) and
 * use_subset[0] = (selective && subset_total > 0 &&
 * full_total / subset_total > compression_ratio) (optional), the totals summed
 * over the rows with active[b] != 0 only (backend.py:2047-2067, 2104-2109:
 * the reference counts its active rows; active == NULL counts every row).
 * Idle rows still get their CSR entries.  The subset CSR holds each row's last
 * min(pages, k) pages when the gate is on and the full CSR when it is off (the
 * reference rebinds the subset lists to the full ones, backend.py:2111-2150),
 * so subset_indices needs batch * pages_per_slot entries.  Rows whose page
 * count would exceed pages_per_slot are clamped (callers bound their rows).
 * k_per_row (int32 [batch], optional; an extension, the reference has one
 * global k) gives row b the budget k_per_row[b] in place of k, clamped to
 * [0, pages_per_slot] as delta_select_pages clamps it: the gate's subset total
 * and the default subset CSR then count min(pages, k_per_row[b]) for row b.
 * budget_rule (optional, exclusive with k_per_row; also an extension) derives
 * row b's budget from its length after the decode token, kv_len = cachelens[b]
 * + 1: max(min_tokens, kv_len / divisor) tokens, in whole pages (/ 16),
 * clamped to [1, k]; the budgets are written to budget_rule->out [batch] for
 * delta_select_pages (k_per_row) in the same step. */
typedef struct {
  int min_tokens;  /* budget floor in tokens (config 5: 512) */
  int divisor;     /* the row's share: kv_len / divisor tokens (config 5: 8) */
  int32_t *out;    /* [batch] device array: each row's budget in pages */
} delta_budget_rule_t;

int delta_decode_page_info(const int32_t *cachelens, const int32_t *active,
                           const int32_t *slot_block_table, int batch, int pages_per_slot, int k,
                           const int32_t *k_per_row, const delta_budget_rule_t *budget_rule,
                           double compression_ratio,
                           int selective, int32_t *kv_indptr, int32_t *kv_indices,
                           int32_t *kv_last_page_len, int32_t *row_block_table,
                           int32_t *subset_indices, int32_t *subset_indptr,
                           int32_t *use_subset, delta_stream_t stream);

/* ------------------------------------------------------------------------ */
/* KV append and RoPE                                                         */
/* ------------------------------------------------------------------------ */

/* mylib::update_kv (utils.py:31-79, FlashInfer append_paged_kv_cache):
 * appended token i of row b (rows from kv_append_indptr) is written at
 * position seq_len_b - append_len_b + i, page kv_indices[kv_indptr[b] + pos/16],
 * slot pos % 16, where seq_len_b comes from kv_indptr/kv_last_page_len.
 * k, v: [nnz, num_kv_heads, 128] with token strides k_stride / v_stride. */
int delta_append_kv(const void *k, int64_t k_stride, const void *v, int64_t v_stride,
                    const int32_t *kv_append_indptr, void *kv_cache, int64_t num_pages,
                    const int32_t *kv_indices, int64_t kv_indices_len,
                    const int32_t *kv_indptr, const int32_t *kv_last_page_len, int nnz,
                    int batch, int num_kv_heads, int head_dim, int dtype,
                    delta_stream_t stream);

/* mylib::rope (model.py:152-175; FlashInfer apply_rope / apply_llama31_rope
 * with interleave=True): token i of row b is at offsets[b] + i - indptr[b];
 * pair (2j, 2j+1) rotates by pos * f_j, f_j = theta^(-2j/d) / rope_scale, or
 * the Llama-3.1 blend when llama31 != 0.  q [nnz, Hq, 128] -> q_out,
 * k [nnz, Hkv, 128] -> k_out (out may alias in). */
int delta_rope(const void *q, int64_t q_stride, const void *k, int64_t k_stride,
               void *q_out, int64_t q_out_stride, void *k_out, int64_t k_out_stride,
               const int32_t *indptr, const int32_t *offsets, int nnz, int batch,
               int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
               float rope_scale, float rope_theta, int llama31, float low_freq_factor,
               float high_freq_factor, float old_context_len, delta_stream_t stream);

/* mylib::rope followed by mylib::update_kv for one layer (Attention.forward,
 * model.py:413-418) in one launch: q -> q_out rotated as delta_rope; k rotated and
 * v copied into the paged cache at the slots delta_append_kv would use (token i of
 * row b at offsets[b] + i - kv_append_indptr[b] for the rotation).  Results are
 * bit-identical to the two calls; the rotated k is not returned. */
int delta_rope_append(const void *q, int64_t q_stride, const void *k, int64_t k_stride,
                      const void *v, int64_t v_stride, void *q_out, int64_t q_out_stride,
                      const int32_t *kv_append_indptr, const int32_t *offsets, void *kv_cache,
                      int64_t num_pages, const int32_t *kv_indices, int64_t kv_indices_len,
                      const int32_t *kv_indptr, const int32_t *kv_last_page_len, int nnz, int batch,
                      int num_qo_heads, int num_kv_heads, int head_dim, int dtype, float rope_scale,
                      float rope_theta, int llama31, float low_freq_factor, float high_freq_factor,
                      float old_context_len, delta_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Dense decode-step helpers (the element-wise chains between the GEMMs)      */
/* ------------------------------------------------------------------------ */

/* out[r * out_stride] = first index of the maximum of logits[r, :cols]
 * (bf16/fp16 rows with stride row_stride; NaN ranks highest), as torch.argmax
 * in _finalize_logits (model.py:320-323).  Two passes through a caller
 * workspace of delta_argmax_workspace_bytes(rows); no memset, so it can sit
 * inside a captured decode step. */
size_t delta_argmax_workspace_bytes(int rows);
int delta_argmax_rows(const void *logits, int64_t row_stride, int rows, int cols, int dtype,
                      int64_t *out, int64_t out_stride, void *workspace, size_t workspace_bytes,
                      delta_stream_t stream);

/* Residual add + RMSNorm of rows of length dim (<= 8192, multiple of 8):
 *   h = x + residual (rounded to the dtype; skipped when residual == NULL, h = x),
 *   out = dtype(dtype(h * rsqrt(mean(h^2) + eps)) * weight),
 * i.e. RMSNorm.forward (model.py:527-532) applied to TransformerBlock's residual
 * sum (model.py:338-341).  sum_out (optional) receives h. */
int delta_add_rmsnorm(const void *x, int64_t x_stride, const void *residual, int64_t r_stride,
                      const void *weight, float eps, void *sum_out, int64_t s_stride, void *out,
                      int64_t out_stride, int rows, int dim, int dtype, delta_stream_t stream);

/* delta_add_rmsnorm with the residual given as nsplit fp32 partials [nsplit][rows][dim]
 * (contiguous, a split-K delta_gemm_rows32's output): residual = dtype(sum of the partials in
 * split order), then the same h and out.  nsplit is 2, 4, 8 or 16 (the splits
 * delta_gemm_rows32 makes).  Same limits; partials 16-byte aligned. */
int delta_add_rmsnorm_partials(const void *x, int64_t x_stride, const float *partials, int nsplit,
                               const void *weight, float eps, void *sum_out, int64_t s_stride, void *out,
                               int64_t out_stride, int rows, int dim, int dtype, delta_stream_t stream);

/* out[r, i] = dtype(dtype(silu(g)) * u) with g = gate_up[r, i], u = gate_up[r, inter + i]:
 * FeedForward's silu(w1 x) * w3 x (model.py:509-514) on the merged w1|w3 GEMM output. */
int delta_silu_mul(const void *gate_up, int64_t gu_stride, void *out, int64_t out_stride, int rows,
                   int inter, int dtype, delta_stream_t stream);

/* out[m, n] = sum_k x[m, k] * w[n, k] (+ bias[n]) for decode-sized M: the nn.Linear
 * projections of a decode step (model.py:412 wqkv, 432 wo, 509-514 w1/w3/w2, 328 lm_head),
 * which torch runs through cuBLAS in the reference.  x [M, K] (row stride ldx), w [N, K]
 * (row stride ldw, the nn.Linear weight layout), out [M, N] (row stride ldo), bias [N] or
 * NULL, all of dtype; fp32 accumulation, one rounding.  K % 64 == 0, N % 16 == 0, x and w
 * rows 16-byte aligned.  Built for M <= 32 (larger M works, re-reading w per 32 rows). */
int delta_gemm_skinny(const void *x, int64_t ldx, const void *w, int64_t ldw, const void *bias,
                      void *out, int64_t ldo, int M, int N, int K, int dtype, delta_stream_t stream);

/* K splits delta_gemm_rows32 uses for an [M, K] x [N, K]^T product (depends only on the
 * shape): 1 = it writes the rounded output, S > 1 = it writes fp32 partials [S][M][N];
 * 0 = the shape is not taken (M, K % 64 or N % 64). */
int delta_gemm_rows32_splits(int M, int N, int K);

/* The same decode projections as delta_gemm_skinny for M <= 32 token rows, with x staged in
 * LDS once per block and K split across the grid so that narrow weights still fill the GPU.
 * With delta_gemm_rows32_splits(M, N, K) == 1: out [M, N] (row stride ldo, even, 4-byte
 * aligned rows) = dtype(x w^T + bias).  With S > 1: partials [S][M][N] fp32 (contiguous,
 * 8-byte aligned), sum over S = x w^T + bias (bias in split 0 only), for a consumer that sums
 * them (delta_add_rmsnorm_partials); out is unused.  K % 64 == 0,
 * N % 64 == 0, x and w rows 16-byte aligned. */
int delta_gemm_rows32(const void *x, int64_t ldx, const void *w, int64_t ldw, const void *bias, void *out,
                      int64_t ldo, float *partials, int M, int N, int K, int dtype, delta_stream_t stream);

/* FeedForward's gate/up projections and SiLU-mul (model.py:509-514) in one launch for M <= 32
 * rows: w13 [2 * inter, K] row-major (row stride ldw) holds w1's rows then w3's; out [M, inter]
 * (row stride ldo, even, 4-byte aligned rows) = dtype(dtype(silu(g)) * u) with g = dtype(x w1^T),
 * u = dtype(x w3^T): bit for bit delta_gemm_rows32 (unsplit) followed by delta_silu_mul.
 * inter % 32 == 0, K % 64 == 0, x and w13 rows 16-byte aligned. */
int delta_gemm_rows32_silu(const void *x, int64_t ldx, const void *w13, int64_t ldw, void *out, int64_t ldo,
                           int M, int inter, int K, int dtype, delta_stream_t stream);

/* The same fused gate/up GEMM + SiLU-mul for M <= 8 rows on delta_gemm_skinny's kernel: bit
 * for bit delta_gemm_skinny over w13 followed by delta_silu_mul.  inter % 16 == 0; out rows
 * any alignment (row stride ldo >= inter). */
int delta_gemm_skinny_silu(const void *x, int64_t ldx, const void *w13, int64_t ldw, void *out, int64_t ldo,
                           int M, int inter, int K, int dtype, delta_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DELTA_HIP_H_ */
