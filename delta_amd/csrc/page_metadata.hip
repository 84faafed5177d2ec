// Page-table metadata kernels for gfx950.
//
// delta_pack_page_indices restates the Triton _pack_page_indices_kernel of
// hoenza/DELTA page_metadata.py:6-70 (gather per-slot block-table rows into a
// CSR list and, optionally, a row-major block table).
//
// delta_decode_page_info moves the per-step metadata of
// _collect_decode_page_info_fast (backend.py:2040-2172) onto the device: the
// per-slot Python loop of Request.plan(1, 16) (scheduler.py:60-66), the
// cumsum'd indptr, the packed CSR, the row block table, the default subset
// CSR of the last k pages and the use_subset gate are all derived from
// `cachelens` and a preallocated slot block table, so a whole decode step can
// be replayed from a hipGraph without host work.  One block per row; each
// block recomputes its row offset from the counts of the rows before it.
// Idle slots (active[b] == 0) keep their CSR entries (one scratch page) but are
// left out of the gate's page totals, which the reference sums over its active
// rows only (backend.py:2047-2067, 2104-2109).  With per-row budgets
// (k_per_row, an extension: the reference has one global subset_cache_size),
// row b's subset count is min(pages_b, k_per_row[b]) in the gate's totals and
// in the default subset CSR, as the selector counts it.  A budget rule (max(min_tokens,
// kv_len / divisor) tokens per row, config 5's shape) derives each row's budget from its current
// length on the device and writes it out for the selector of the same step.
#include "delta_common.h"

namespace delta {
namespace {

__global__ void __launch_bounds__(256)
    pack_page_indices_kernel(const int32_t *slot_bt, const int32_t *active_slots, const int32_t *start_cols,
                             const int32_t *counts, const int32_t *indptr, int32_t *out_indices,
                             int64_t out_len, int32_t *row_bt, int num_slots, int pages_per_slot,
                             int write_row_block) {
  const int r = blockIdx.x;
  const int64_t slot = active_slots[r];
  const int64_t start = start_cols[r];
  const int64_t dst = indptr[r];
  int64_t cnt = counts[r];
  // A row that would read outside the slot table or write outside the output is dropped.
  if (slot < 0 || slot >= num_slots || start < 0 || cnt <= 0 || start + cnt > pages_per_slot || dst < 0 ||
      dst + cnt > out_len)
    return;
  const int32_t *src = slot_bt + slot * pages_per_slot + start;
  for (int c = threadIdx.x; c < cnt; c += blockDim.x) {
    const int32_t v = src[c];
    out_indices[dst + c] = v;
    if (write_row_block) row_bt[(int64_t)r * pages_per_slot + c] = v;
  }
}

struct PageInfoArgs {
  const int32_t *cachelens;
  const int32_t *active;  // [batch] or null (every row active)
  const int32_t *slot_bt;
  int batch, pages_per_slot, k;
  const int32_t *k_per_row;  // [batch] or null (every row takes k)
  int rule_min_tokens, rule_divisor;  // budget rule (rule_divisor > 0): see row_budget
  int32_t *rule_out;                  // [batch]: each row's budget under the rule
  double compression_ratio;
  int selective;
  int32_t *kv_indptr, *kv_indices, *last_page_len, *row_bt, *subset_indices, *subset_indptr, *use_subset;
};

__device__ __forceinline__ void row_pages(const PageInfoArgs &a, int b, int *np, int *last) {
  int64_t kv_len = (int64_t)a.cachelens[b] + 1;
  kv_len = kv_len < 1 ? 1 : kv_len;
  int64_t n = kv_len / kPageSize + 1;
  int lp = (int)(kv_len % kPageSize);
  if (n > a.pages_per_slot) {  // row outgrew its allocation: clamp to a full table
    n = a.pages_per_slot;
    lp = kPageSize;
  }
  *np = (int)n;
  *last = lp;
}

// Row b's subset budget in pages.  With the budget rule: max(min_tokens, kv_len / divisor)
// tokens after the decode token, in whole pages, clamped to [1, k]; else k_per_row[b] or k, clamped
// to [0, pages_per_slot] as the selector's row_budget clamps it.
__device__ __forceinline__ int row_budget(const PageInfoArgs &a, int b) {
  if (a.rule_divisor > 0) {
    int64_t kv_len = (int64_t)a.cachelens[b] + 1;
    kv_len = kv_len < 1 ? 1 : kv_len;
    const int64_t share = kv_len / a.rule_divisor;
    const int64_t tokens = share > a.rule_min_tokens ? share : a.rule_min_tokens;
    int64_t kb = tokens / kPageSize;
    kb = kb > a.k ? a.k : kb;
    return kb < 1 ? 1 : (int)kb;
  }
  int kb = a.k_per_row ? a.k_per_row[b] : a.k;
  kb = kb < 0 ? 0 : kb;
  return kb > a.pages_per_slot ? a.pages_per_slot : kb;
}

__global__ void __launch_bounds__(256) decode_page_info_kernel(PageInfoArgs a) {
  __shared__ long long s_red[4][4];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  long long full_before = 0, sub_before = 0, full_tot = 0, sub_tot = 0;
  for (int i = tid; i < a.batch; i += 256) {
    int np, lp;
    row_pages(a, i, &np, &lp);
    const int kb = row_budget(a, i);
    const int sc = np < kb ? np : kb;
    if (a.active == nullptr || a.active[i] != 0) {
      full_tot += np;
      sub_tot += sc;
    }
    if (i < b) {
      full_before += np;
      sub_before += sc;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    full_before += __shfl_xor(full_before, off);
    sub_before += __shfl_xor(sub_before, off);
    full_tot += __shfl_xor(full_tot, off);
    sub_tot += __shfl_xor(sub_tot, off);
  }
  const int wave = tid >> 6;
  if ((tid & 63) == 0) {
    s_red[wave][0] = full_before;
    s_red[wave][1] = sub_before;
    s_red[wave][2] = full_tot;
    s_red[wave][3] = sub_tot;
  }
  __syncthreads();
  full_before = s_red[0][0] + s_red[1][0] + s_red[2][0] + s_red[3][0];
  sub_before = s_red[0][1] + s_red[1][1] + s_red[2][1] + s_red[3][1];
  full_tot = s_red[0][2] + s_red[1][2] + s_red[2][2] + s_red[3][2];
  sub_tot = s_red[0][3] + s_red[1][3] + s_red[2][3] + s_red[3][3];

  int np, lp;
  row_pages(a, b, &np, &lp);
  // use_subset gate (backend.py:2104-2109); when it is off the subset CSR is the full CSR.
  const bool gate = a.selective && sub_tot > 0 && ((double)full_tot / (double)sub_tot) > a.compression_ratio;
  const int kb = row_budget(a, b);
  const int sc = gate ? (np < kb ? np : kb) : np;
  if (a.rule_out && tid == 0) a.rule_out[b] = kb;  // the selector reads this step's budgets
  const long long sb = gate ? sub_before : full_before;
  if (tid == 0) {
    a.kv_indptr[b + 1] = (int32_t)(full_before + np);
    a.last_page_len[b] = lp;
    if (a.subset_indptr) a.subset_indptr[b + 1] = (int32_t)(sb + sc);
    if (b == 0) {
      a.kv_indptr[0] = 0;
      if (a.subset_indptr) a.subset_indptr[0] = 0;
      if (a.use_subset) a.use_subset[0] = gate ? 1 : 0;
    }
  }
  const int32_t *src = a.slot_bt + (int64_t)b * a.pages_per_slot;
  const int sub_start = np - sc;
  // Eight 256-page batches' ids are loaded before any of their stores: the stores may alias the
  // source as far as the compiler knows, so a load-store loop waits one memory round trip per
  // batch (a 4097-page row: 17 round trips, ~9 us).
  constexpr int kCopyUnroll = 8;
  for (int c0 = tid; c0 < a.pages_per_slot; c0 += 256 * kCopyUnroll) {
    int32_t v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int c = c0 + 256 * u;
      v[u] = c < np ? src[c] : 0;
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int c = c0 + 256 * u;
      if (c >= a.pages_per_slot) break;
      if (c < np) {
        a.kv_indices[full_before + c] = v[u];
        if (a.row_bt) a.row_bt[(int64_t)b * a.pages_per_slot + c] = v[u];
        if (a.subset_indices && c >= sub_start) a.subset_indices[sb + c - sub_start] = v[u];
      } else if (a.row_bt) {
        a.row_bt[(int64_t)b * a.pages_per_slot + c] = 0;  // no stale ids past the row (backend.py:2080-2086)
      }
    }
  }
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT int delta_pack_page_indices(const int32_t *slot_block_table, int num_slots,
                                                    const int32_t *active_slots, const int32_t *start_cols,
                                                    const int32_t *counts, const int32_t *indptr,
                                                    int32_t *out_indices, int64_t out_indices_len,
                                                    int32_t *row_block_table, int n_rows, int pages_per_slot,
                                                    int max_count, int write_row_block, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  if (n_rows <= 0 || max_count <= 0) return DELTA_OK;  // page_metadata.py:55-56
  if (!slot_block_table || !active_slots || !start_cols || !counts || !indptr || !out_indices)
    return set_error(DELTA_ERR_INVALID, "delta_pack_page_indices: null pointer");
  if (write_row_block && !row_block_table)
    return set_error(DELTA_ERR_INVALID, "delta_pack_page_indices: null row block table");
  const int threads = max_count >= 256 ? 256 : 64;
  hipLaunchKernelGGL(pack_page_indices_kernel, dim3(n_rows), dim3(threads), 0, (hipStream_t)stream, slot_block_table,
                     active_slots, start_cols, counts, indptr, out_indices, out_indices_len, row_block_table,
                     num_slots, pages_per_slot, write_row_block);
  return check_launch("delta_pack_page_indices");
}

extern "C" DELTA_EXPORT int delta_decode_page_info(const int32_t *cachelens, const int32_t *active,
                                                   const int32_t *slot_block_table, int batch, int pages_per_slot,
                                                   int k, const int32_t *k_per_row,
                                                   const delta_budget_rule_t *budget_rule, double compression_ratio,
                                                   int selective, int32_t *kv_indptr, int32_t *kv_indices,
                                                   int32_t *kv_last_page_len, int32_t *row_block_table,
                                                   int32_t *subset_indices, int32_t *subset_indptr,
                                                   int32_t *use_subset, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  if (batch <= 0) return DELTA_OK;
  if (!cachelens || !slot_block_table || !kv_indptr || !kv_indices || !kv_last_page_len)
    return set_error(DELTA_ERR_INVALID, "delta_decode_page_info: null pointer");
  if (pages_per_slot <= 0) return set_error(DELTA_ERR_INVALID, "delta_decode_page_info: pages_per_slot <= 0");
  if ((subset_indices == nullptr) != (subset_indptr == nullptr))
    return set_error(DELTA_ERR_INVALID, "delta_decode_page_info: subset_indices and subset_indptr go together");
  if (budget_rule && (k_per_row || budget_rule->divisor <= 0 || budget_rule->min_tokens < 0 || !budget_rule->out))
    return set_error(DELTA_ERR_INVALID,
                     "delta_decode_page_info: a budget rule needs divisor > 0, min_tokens >= 0, an output array, "
                     "and no k_per_row");
  PageInfoArgs a;
  a.cachelens = cachelens;
  a.active = active;
  a.slot_bt = slot_block_table;
  a.batch = batch;
  a.pages_per_slot = pages_per_slot;
  a.k = k < 0 ? 0 : k;
  a.k_per_row = k_per_row;
  a.rule_min_tokens = budget_rule ? budget_rule->min_tokens : 0;
  a.rule_divisor = budget_rule ? budget_rule->divisor : 0;
  a.rule_out = budget_rule ? budget_rule->out : nullptr;
  a.compression_ratio = compression_ratio;
  a.selective = selective;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.last_page_len = kv_last_page_len;
  a.row_bt = row_block_table;
  a.subset_indices = subset_indices;
  a.subset_indptr = subset_indptr;
  a.use_subset = use_subset;
  hipLaunchKernelGGL(decode_page_info_kernel, dim3(batch), dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("delta_decode_page_info");
}
