// PageSelectorV2 top-k page selection for gfx950.
//
// Restates hoenza/DELTA page_selector_v2.py:113-212 for one row per block:
//   key_j = nan_to_num(score_j, nan=-inf, neginf=-inf) + fp32(-j * bias)   (113-118)
//   key_j = +inf for j in [max(tp - L, 0), tp)                               (123-126)
//   pages j >= tp are not candidates (their key is -inf, 128-129)
//   top-k of key, ties broken by the smaller page index (torch.topk leaves
//   tie order unspecified; this build fixes it), positions emitted in
//   ascending j (132-134) as physical ids from the row's block table (147-150).
//
// Algorithm per row (one block of 256, 512 or 1024 threads): fp32 keys map to order-preserving uint32
// (+0/-0 folded); an 8-bit radix select (up to 4 passes; it stops once every key of the k-th
// key's bin is taken) finds the k-th largest key T and
// how many keys equal to T are taken (r); one ordered pass then marks
// key > T, or key == T among the first r such pages, and compacts the marked
// pages in ascending j -- the output is sorted by construction, no sort pass.
// Rows of up to 1024 (256 threads), 4096 (512 threads) or 8192 pages (1024 threads) keep their
// keys in registers, each thread a contiguous run of up to 4 or 8 pages loaded at the kernel's
// start, so
// the compaction is one block prefix sum of the threads' counts (two when keys equal to T must
// be ranked).  Longer rows recompute the keys from the fp32 scores in every pass (they stay in
// L2) and compact 1024 pages at a time with ballot prefix sums, so any row length works.  When
// every key equal to T is taken (the usual case), the compaction needs no rank among them.
#include <float.h>

#include "delta_common.h"

namespace delta {
namespace {

// Block sizes by the launch's longest row: 256 threads x 4 keys up to 1024 pages, 512 x 4 up to
// 2048, 512 x 8 up to 4096, 1024 x 8 up to 8192 (a 128 k-token context) and past it (keys
// re-read every pass).  Fewer waves wait at each of a pass's barriers; against 1024-thread
// blocks, 512 x 4 took 64 rows of 1125 pages 9.0 -> 7.0 us and config 5 (2046 pages) 10.0 -> 7.8
// us, 512 x 8 16 rows of 3000 pages 10.4 -> 9.2 us and 4096-page rows the same 10.3 us.
constexpr int kSelThreadsLong = 1024;
constexpr int kSelThreadsMid = 512;
constexpr int kSelThreadsShort = 256;
constexpr int kKeysLong = 8;
constexpr int kKeysShort = 4;
constexpr int kBins = 256;         // radix digit bins, handled by the first 4 waves
constexpr int kHistCopies = 8;     // pass-1 histogram copies
constexpr int kCopyStride = kBins + 1;
constexpr uint32_t kKeyPosInf = 0xFF800000u;  // order_key(+inf)

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Prepared fp32 score exactly as the reference's sequence of fp32 tensor ops.
// The product and the sum are two separately rounded fp32 operations, as the
// reference's `-arange(n) * scale` followed by `scores.add_(bias)`: contraction
// into an FMA would change the keys, so it is switched off here.
__device__ __forceinline__ float prepare(float s, int j, float bias_scale) {
#pragma clang fp contract(off)
  if (s != s) s = -INFINITY;           // nan -> -inf
  else if (s == INFINITY) s = FLT_MAX;  // posinf -> largest finite (nan_to_num default)
  if (bias_scale != 0.f) {
    const float bj = (-(float)j) * bias_scale;
    s = s + bj;
  }
  return s == 0.f ? 0.f : s;  // -0 and +0 compare equal
}

struct SelArgs {
  const float *scores;
  int64_t score_stride;
  const int32_t *kv_indptr;
  const int32_t *block_table;
  int64_t bt_stride;
  int batch, max_pages, k;
  const int32_t *k_per_row;
  int L;
  float bias_scale;
  int fixed_count;
  const int32_t *use_subset;
  int32_t *out_indices;
  int64_t out_len;  // capacity of out_indices
  int32_t *out_indptr;
};

// Pages of row b that can be scored (the reference's Nmax is the largest row,
// so tp <= max_pages there; a larger row is clamped to max_pages columns).
__device__ __forceinline__ int row_pages(const SelArgs &a, int b) {
  const int tp = a.kv_indptr[b + 1] - a.kv_indptr[b];
  return tp < 0 ? 0 : (tp > a.max_pages ? a.max_pages : tp);
}

__device__ __forceinline__ int row_budget(const SelArgs &a, int b) {
  int kb = a.k_per_row ? a.k_per_row[b] : a.k;
  kb = kb < 0 ? 0 : kb;
  return kb > a.max_pages ? a.max_pages : kb;
}

// Number of pages row b emits.
__device__ __forceinline__ int row_count(const SelArgs &a, int b, bool subset) {
  const int tp = row_pages(a, b);
  if (!subset) return tp;
  const int kb = row_budget(a, b);
  if (a.fixed_count) return kb;
  return tp < kb ? tp : kb;
}

// Block-wide sum over NW waves (all threads receive it).
template <int NW>
__device__ int block_sum(int v, int *scratch) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  int s = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) s += scratch[w];
  __syncthreads();
  return s;
}

// Exclusive block prefix of an int in thread order over NW waves; *total gets the block total.
template <int NW>
__device__ int block_prefix_int(int v, int *scratch, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(inc, off);
    if (lane >= off) inc += y;
  }
  if (lane == 63) scratch[wave] = inc;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int x = scratch[w];
    before += w < wave ? x : 0;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return before + inc - v;
}

// Exclusive block prefix of a 0/1 flag in thread order over NW waves; *total gets the block total.
template <int NW>
__device__ int block_prefix(bool flag, int *scratch, int *total) {
  int wtot;
  const int wpre = wave_prefix_exclusive(flag, &wtot);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = wtot;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int x = scratch[w];
    before += w < wave ? x : 0;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return before + wpre;
}

template <int kSelThreads, int kKeys>
__global__ void __launch_bounds__(kSelThreads) select_pages_kernel(SelArgs a) {
  constexpr int kSelWaves = kSelThreads / 64;
  static_assert(kSelThreads >= kBins, "the bins are handled by the first kBins threads");
  __shared__ int s_scratch[kSelWaves];
  __shared__ uint32_t s_hist[2][kBins];                    // passes 2-4 alternate between the two
  __shared__ uint32_t s_hcopy[kHistCopies * kCopyStride];  // pass 1: one histogram per (lane & 7)
  __shared__ int s_digit, s_remaining, s_eq;

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float *srow = a.scores + (int64_t)b * a.score_stride;
  const int32_t *bt = a.block_table + (int64_t)b * a.bt_stride;
  // When max_pages fits kKeys * kSelThreads, every row keeps its keys in registers, thread t
  // holding the contiguous run j0 = t * kpt .. j0 + kpt - 1 with kpt = ceil(max_pages /
  // kSelThreads) <= kKeys (so every wave holds keys).  The scores are loaded first, up to
  // max_pages (inside the scores' row), so the loads overlap the row bookkeeping below.
  const bool cached = a.max_pages <= kKeys * kSelThreads;
  const int kpt = (a.max_pages + kSelThreads - 1) / kSelThreads;
  const int j0 = tid * kpt;
  float sv[kKeys];
  if (cached) {
#pragma unroll
    for (int i = 0; i < kKeys; ++i) sv[i] = i < kpt && j0 + i < a.max_pages ? srow[j0 + i] : 0.f;
  }
  for (int x = tid; x < kHistCopies * kCopyStride; x += kSelThreads) s_hcopy[x] = 0;
  if (tid < kBins) s_hist[1][tid] = 0;  // pass 2's bins; pass 3's are cleared during pass 2

  const bool subset = a.use_subset == nullptr || a.use_subset[0] != 0;
  // Output offset of this row: sum of the counts of the rows before it.
  int before = 0;
  if (subset && a.fixed_count) {
    before = b * row_budget(a, 0);
  } else {
    int part = 0;
    for (int i = tid; i < b; i += kSelThreads) part += row_count(a, i, subset);
    before = block_sum<kSelWaves>(part, s_scratch);
  }
  const int cnt = row_count(a, b, subset);
  if (tid == 0) {
    a.out_indptr[b + 1] = before + cnt;
    if (b == 0) a.out_indptr[0] = 0;
  }

  const int tp = row_pages(a, b);
  const int kb = row_budget(a, b);
  int32_t *out = a.out_indices + before;
  // Never write past the caller's buffer (the indptr above still says what was meant).
  const int64_t room = a.out_len - (int64_t)before;
  const int lim = room <= 0 ? 0 : (room < cnt ? (int)room : cnt);

  // Every page of the row is taken (no subset, or fewer pages than the
  // budget): the ascending top-k is 0..cnt-1 (for the fixed path with
  // tp < k the padding columns tp..k-1 follow, as torch.topk over -inf).
  if (!subset || tp <= kb) {
    for (int j = tid; j < lim; j += kSelThreads) out[j] = bt[j];
    return;
  }

  const int last_start = tp - a.L > 0 ? tp - a.L : 0;
  auto key_of = [&](int j, float s) -> uint32_t {
    if (j >= last_start) return kKeyPosInf;
    return order_key(prepare(s, j, a.bias_scale));
  };
  uint32_t kc[kKeys];
  if (cached) {
#pragma unroll
    for (int i = 0; i < kKeys; ++i) kc[i] = i < kpt && j0 + i < tp ? key_of(j0 + i, sv[i]) : 0u;
  }
  __syncthreads();  // the histograms are clear

  // Radix select of the kb-th largest key, 8 bits a pass from the top.  Pass 1 counts into
  // eight lane-indexed copies (one word apart, so one bin's copies sit in different banks): its
  // digits are the keys' sign and exponent, which few values share, and same-address LDS atomics
  // of one wave serialise.  Later passes count into one histogram and clear the other for the
  // pass after, so a pass needs three barriers.
  uint32_t prefix = 0, pmask = 0;
  int remaining = kb;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    uint32_t *hist = s_hist[pass & 1];
    uint32_t *bins = pass == 0 ? s_hcopy + (tid & (kHistCopies - 1)) * kCopyStride : hist;
    if (cached) {
#pragma unroll
      for (int i = 0; i < kKeys; ++i) {
        const uint32_t key = kc[i];
        if (i < kpt && j0 + i < tp && (key & pmask) == prefix) atomicAdd(&bins[(key >> shift) & 255u], 1u);
      }
    } else {
      for (int j = tid; j < tp; j += kSelThreads) {
        const uint32_t key = key_of(j, srow[j]);
        if ((key & pmask) == prefix) atomicAdd(&bins[(key >> shift) & 255u], 1u);
      }
    }
    if (pass > 0 && tid < kBins) s_hist[(pass + 1) & 1][tid] = 0;  // read last in the previous pass
    __syncthreads();
    // Suffix sums over the 256 bins (thread d < 256 holds bin d): suf[d] = #keys with digit >= d.
    const int lane = tid & 63, wave = tid >> 6;
    int hd = 0;
    if (tid < kBins) {
      if (pass == 0) {
#pragma unroll
        for (int c = 0; c < kHistCopies; ++c) hd += (int)s_hcopy[c * kCopyStride + tid];
      } else {
        hd = (int)hist[tid];
      }
    }
    int suf = hd;
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_down(suf, off);
      if (lane + off < 64) suf += y;
    }
    if (lane == 0 && tid < kBins) s_scratch[wave] = suf;
    __syncthreads();
    for (int w = wave + 1; w < kBins / 64; ++w) suf += s_scratch[w];
    if (tid < kBins && suf >= remaining && suf - hd < remaining) {
      s_digit = tid;
      s_remaining = remaining - (suf - hd);
      s_eq = hd;  // after the last digit: the number of keys equal to T
    }
    __syncthreads();
    // s_digit / s_remaining / s_eq are next written after two barriers of the next pass.
    prefix |= (uint32_t)s_digit << shift;
    pmask |= 0xFFu << shift;
    remaining = s_remaining;
    // Every key of the k-th key's bin is taken: the selection is exactly the keys whose digits so
    // far are >= the prefix, i.e. key >= T with T = prefix (lower bits zero) -- no further pass.
    if (remaining == s_eq) break;
  }
  const uint32_t T = prefix;
  const int take_eq = remaining;  // how many keys == T are selected (smallest j first)
  const bool all_eq = take_eq >= s_eq;  // every key equal to T is taken: no rank among them

  if (cached) {
    // Ordered compaction of the thread's contiguous run: the pages it takes go to its prefix of
    // the block's counts, in ascending j.  Keys equal to T are taken from the smallest j on:
    // the thread takes those of its own that rank below take_eq among the block's.
    int n_gt = 0, n_eq = 0;
#pragma unroll
    for (int i = 0; i < kKeys; ++i) {
      const bool in = i < kpt && j0 + i < tp;
      n_gt += in && kc[i] > T;
      n_eq += in && kc[i] == T;
    }
    int eq_take = n_eq;
    if (!all_eq) {
      int eq_tot;
      const int eq_before = block_prefix_int<kSelWaves>(n_eq, s_scratch, &eq_tot);
      const int left = take_eq - eq_before;
      eq_take = left <= 0 ? 0 : (left < n_eq ? left : n_eq);
    }
    int sel_tot;
    int pos = block_prefix_int<kSelWaves>(n_gt + eq_take, s_scratch, &sel_tot);
#pragma unroll
    for (int i = 0; i < kKeys; ++i) {
      const bool in = i < kpt && j0 + i < tp;
      const bool eq = in && kc[i] == T;
      const bool sel = (in && kc[i] > T) || (eq && eq_take > 0);
      eq_take -= eq ? 1 : 0;
      if (sel) {
        if (pos < lim) out[pos] = bt[j0 + i];
        ++pos;
      }
    }
    return;
  }

  // Ordered compaction of longer rows, 1024 pages at a time (block-uniform trip counts: the
  // prefixes hold barriers).
  int eq_seen = 0, written = 0;
  for (int base = 0; base < tp; base += kSelThreads) {
    const int j = base + tid;
    const uint32_t key = j < tp ? key_of(j, srow[j]) : 0u;
    const bool in = j < tp;
    bool sel;
    if (all_eq) {
      sel = in && key >= T;
    } else {
      const bool eq = in && key == T;
      int eq_tot;
      const int eq_rank = eq_seen + block_prefix<kSelWaves>(eq, s_scratch, &eq_tot);
      sel = in && (key > T || (eq && eq_rank < take_eq));
      eq_seen += eq_tot;
    }
    int sel_tot;
    const int pos = written + block_prefix<kSelWaves>(sel, s_scratch, &sel_tot);
    if (sel && pos < lim) out[pos] = bt[j];
    written += sel_tot;
  }
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT int delta_select_pages(const float *scores, int64_t score_stride, const int32_t *kv_indptr,
                                               const int32_t *block_table, int64_t bt_stride, int batch,
                                               int max_pages, int k, const int32_t *k_per_row, int L,
                                               float pos_bias_scale, int fixed_count, const int32_t *use_subset,
                                               int32_t *out_indices, int64_t out_indices_len, int32_t *out_indptr,
                                               delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_select_pages";
  if (batch <= 0) return DELTA_OK;
  if (!scores || !kv_indptr || !block_table || !out_indices || !out_indptr)
    return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (max_pages <= 0) return set_error(DELTA_ERR_INVALID, "%s: max_pages must be positive", who);
  if (score_stride < max_pages || bt_stride < max_pages)
    return set_error(DELTA_ERR_INVALID, "%s: row strides must be >= max_pages", who);
  if (fixed_count && k_per_row) return set_error(DELTA_ERR_INVALID, "%s: fixed_count needs a global k", who);
  if (!k_per_row && k > max_pages)
    return set_error(DELTA_ERR_INVALID, "%s: selected index k out of range (k=%d > %d pages)", who, k, max_pages);
  if (L < 0) return set_error(DELTA_ERR_INVALID, "%s: L must be >= 0", who);
  SelArgs a;
  a.scores = scores;
  a.score_stride = score_stride;
  a.kv_indptr = kv_indptr;
  a.block_table = block_table;
  a.bt_stride = bt_stride;
  a.batch = batch;
  a.max_pages = max_pages;
  a.k = k;
  a.k_per_row = k_per_row;
  a.L = L;
  a.bias_scale = pos_bias_scale;
  a.fixed_count = fixed_count;
  a.use_subset = use_subset;
  a.out_indices = out_indices;
  a.out_len = out_indices_len;
  a.out_indptr = out_indptr;
  if (max_pages <= kKeysShort * kSelThreadsShort)
    hipLaunchKernelGGL((select_pages_kernel<kSelThreadsShort, kKeysShort>), dim3(batch), dim3(kSelThreadsShort), 0,
                       (hipStream_t)stream, a);
  else if (max_pages <= kKeysShort * kSelThreadsMid)
    hipLaunchKernelGGL((select_pages_kernel<kSelThreadsMid, kKeysShort>), dim3(batch), dim3(kSelThreadsMid), 0,
                       (hipStream_t)stream, a);
  else if (max_pages <= kKeysLong * kSelThreadsMid)
    hipLaunchKernelGGL((select_pages_kernel<kSelThreadsMid, kKeysLong>), dim3(batch), dim3(kSelThreadsMid), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((select_pages_kernel<kSelThreadsLong, kKeysLong>), dim3(batch), dim3(kSelThreadsLong), 0,
                       (hipStream_t)stream, a);
  return check_launch(who);
}
