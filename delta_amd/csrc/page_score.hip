// del3_legacy_softmax page scores for gfx950.
//
// Restates hoenza/DELTA backend.py:887-904:
//   probs  = softmax_t(dump[b, h, :max_pages*16])        (per q head)
//   score  = sum_{t in page j} max_h probs[b, h, t]
// The softmax normaliser of each (row, head) is its log-sum-exp: either the
// lse the decode kernel produced for the same logits, or (lse == NULL) a first
// pass over the dump.  Positions t >= kv_len_b hold -inf in the reference's
// buffer (backend.py:384-389); they contribute exp(-inf) = 0 and are not read.
//
// Score kernel: grid (ceil(max_pages*16 / 256), batch), 256 threads, one
// token per thread; per head a fully coalesced 1 KiB read of the dump, the
// reads of up to 64 heads in flight together; the 16-token page sum is a DPP
// reduction inside each 16-lane row.
//
// HBM bytes per launch (algorithmic): the dump rows up to kv_len (read once),
// lse, page table, scores.
#include "delta_common.h"

namespace delta {

int run_decode(const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *kv_cache,
               int64_t num_pages, const int32_t *kv_indptr, const int32_t *kv_indices,
               int64_t kv_indices_len, const int32_t *kv_last_page_len, void *o,
               int64_t o_stride_b, int64_t o_stride_h, float *lse, float *dump,
               int64_t dump_stride_b, int64_t dump_stride_h, int batch, int hq, int hkv,
               int head_dim, int dtype, float sm_scale, int max_pages, int mode,
               void *workspace, size_t workspace_bytes, hipStream_t stream, const char *who,
               const delta_decode_append_t *ap);
int decode_num_splits(int batch, int hkv, int max_pages);
bool tokmax_fits(int batch, int hkv, int G, int max_pages);
bool plan_tokmax_fits(int batch, int hkv, int G, int max_pages, bool rope);
size_t decode_workspace_bytes(int batch, int hq, int nsplit, bool with_acc);

namespace {

constexpr int kScoreThreads = 256;
constexpr int kMaxWaves = 16;  // kv heads a launch takes (the decode kernel's block limit)
constexpr int kMaxHeads = 256;

__device__ __forceinline__ int row_kv_len(const int32_t *kv_indptr, const int32_t *last, int b) {
  int np = kv_indptr[b + 1] - kv_indptr[b];
  np = np < 0 ? 0 : np;
  int lp = last[b];
  lp = lp < 0 ? 0 : (lp > kPageSize ? kPageSize : lp);
  return np > 0 ? (np - 1) * kPageSize + lp : 0;
}

// lse of one (row, head) dump row over t < kv_len (natural log).
__global__ void __launch_bounds__(256) dump_lse_kernel(const float *dump, int64_t sdb, int64_t sdh,
                                                        const int32_t *kv_indptr, const int32_t *last,
                                                        float *lse, int hq, int cap) {
  __shared__ float red[4];
  const int b = blockIdx.x / hq;
  const int h = blockIdx.x % hq;
  const int n = min(row_kv_len(kv_indptr, last, b), cap);
  const float *row = dump + (int64_t)b * sdb + (int64_t)h * sdh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float mx = -INFINITY;
  for (int t = threadIdx.x; t < n; t += 256) mx = fmaxf(mx, row[t]);
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, shfl_xor(mx, off));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  const float mref = mx == -INFINITY ? 0.f : mx;
  float s = 0.f;
  for (int t = threadIdx.x; t < n; t += 256) s += fast_exp2((row[t] - mref) * kLog2e);
  for (int off = 32; off > 0; off >>= 1) s += shfl_xor(s, off);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float tot = red[0] + red[1] + red[2] + red[3];
    lse[(int64_t)b * hq + h] = tot > 0.f ? mref + logf(tot) : -INFINITY;
  }
}

// One token per thread; the max over q heads of exp2(logit log2e - lse log2e), then the 16-lane
// page sum.  Two loads per lane bring the first NH heads' lse values (lane i: head i) and the
// row bounds (lanes 0-2); then each pass requests the logits of NH heads as independent loads,
// so a block waits two memory round trips for hq <= NH.  NH is hq rounded up to a multiple of 8
// (at most 64, then several passes); heads past hq - 1 repeat head hq - 1, which leaves the max
// unchanged.  Blocks wholly past the row's kv_len load no logits.
template <int NH>
__global__ void __launch_bounds__(kScoreThreads)
    legacy_softmax_score_kernel(const float *dump, int64_t sdb, int64_t sdh, const float *lse,
                                const int32_t *kv_indptr, const int32_t *last, float *scores,
                                int64_t score_stride, int hq, int max_pages) {
  static_assert(NH % 8 == 0 && NH >= 8 && NH <= 64, "lse of head h0 + i sits in lane i");
  const int b = blockIdx.y;
  const int tok = blockIdx.x * kScoreThreads + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const int32_t *bsrc = lane == 0 ? kv_indptr + b : lane == 1 ? kv_indptr + b + 1 : last + b;
  const int bw = *bsrc;
  const float *lse_b = lse + (int64_t)b * hq;
  const int lh = lane < NH ? lane : NH - 1;  // lane i < NH holds head h0 + i's lse
  float lv = lse_b[min(lh, hq - 1)];
  asm volatile("" ::"v"(bw), "v"(lv));  // both loads in flight together
  int np = __builtin_amdgcn_readlane(bw, 1) - __builtin_amdgcn_readlane(bw, 0);
  np = np < 0 ? 0 : np;
  int lp = __builtin_amdgcn_readlane(bw, 2);
  lp = lp < 0 ? 0 : (lp > kPageSize ? kPageSize : lp);
  const int n = min(np > 0 ? (np - 1) * kPageSize + lp : 0, max_pages * kPageSize);
  const float *col = dump + (int64_t)b * sdb + tok;
  float best = 0.f;
  if ((int)blockIdx.x * kScoreThreads < n) {
    for (int h0 = 0; h0 < hq; h0 += NH) {
      if (h0 > 0) lv = lse_b[min(h0 + lh, hq - 1)];
      if (tok < n) {
        float x[NH];
#pragma unroll
        for (int i = 0; i < NH; ++i)
          x[i] = __builtin_nontemporal_load(col + (int64_t)min(h0 + i, hq - 1) * sdh);
#pragma unroll
        for (int i = 0; i < NH; ++i) best = fmaxf(best, fast_exp2(x[i] * kLog2e - readlane(lv, i) * kLog2e));
      }
    }
  }
  const float page_sum = row16_sum(best);
  const int page = tok >> 4;
  if ((threadIdx.x & 15) == 0 && page < max_pages) scores[(int64_t)b * score_stride + page] = page_sum;
}

// Page scores from the LDS scorer's per-(kv head, token) maxima tm [batch][hkv][sh]: one token per
// thread, the max over the hkv values (the max over all q heads of the token's probability),
// then the same 16-lane page sum as legacy_softmax_score_kernel.  One load brings the row bounds
// (lanes 0-2); then KH kv heads' maxima (hkv rounded up to a power of two, at most kMaxWaves)
// are requested together (heads past hkv - 1
// repeat head hkv - 1, which leaves the max unchanged).
template <int KH>
__global__ void __launch_bounds__(kScoreThreads)
    tokmax_score_kernel(const float *tm, int64_t sb, int64_t sh, int hkv, const int32_t *kv_indptr,
                        const int32_t *last, float *scores, int64_t score_stride, int max_pages) {
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int32_t *bsrc = lane == 0 ? kv_indptr + b : lane == 1 ? kv_indptr + b + 1 : last + b;
  const int bw = *bsrc;
  asm volatile("" ::"s"(tm), "s"(sb), "s"(sh), "s"(hkv));  // the arguments arrive while the bounds load
  int np = __builtin_amdgcn_readlane(bw, 1) - __builtin_amdgcn_readlane(bw, 0);
  np = np < 0 ? 0 : np;
  int lp = __builtin_amdgcn_readlane(bw, 2);
  lp = lp < 0 ? 0 : (lp > kPageSize ? kPageSize : lp);
  const int n = min(np > 0 ? (np - 1) * kPageSize + lp : 0, max_pages * kPageSize);
  const int tok = blockIdx.x * kScoreThreads + threadIdx.x;
  const float *col = tm + (int64_t)b * sb + tok;
  float best = 0.f;
  if (tok < n) {
    float v[KH];
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) v[kh] = __builtin_nontemporal_load(col + min(kh, hkv - 1) * sh);
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) best = fmaxf(best, v[kh]);
  }
  const float page_sum = row16_sum(best);
  const int page = tok >> 4;
  if ((threadIdx.x & 15) == 0 && page < max_pages) scores[(int64_t)b * score_stride + page] = page_sum;
}

// The page-sum launch over per-(kv head, token) maxima, KH = hkv rounded up to a power of two.
void launch_tokmax_scores(const float *tm, int64_t sb, int64_t sh, int hkv, const int32_t *kv_indptr,
                          const int32_t *last, float *scores, int64_t score_stride, int batch, int max_pages,
                          hipStream_t stream) {
  dim3 grid((unsigned)ceil_div((int64_t)max_pages * kPageSize, kScoreThreads), batch);
  auto launch = [&](auto k) {
    hipLaunchKernelGGL(k, grid, dim3(kScoreThreads), 0, stream, tm, sb, sh, hkv, kv_indptr, last, scores,
                       score_stride, max_pages);
  };
  if (hkv <= 1) launch(tokmax_score_kernel<1>);
  else if (hkv <= 2) launch(tokmax_score_kernel<2>);
  else if (hkv <= 4) launch(tokmax_score_kernel<4>);
  else if (hkv <= 8) launch(tokmax_score_kernel<8>);
  else launch(tokmax_score_kernel<kMaxWaves>);
}

int launch_scores(const float *dump, int64_t sdb, int64_t sdh, const float *lse,
                  const int32_t *kv_indptr, const int32_t *last, float *scores, int64_t score_stride,
                  int batch, int hq, int max_pages, hipStream_t stream, const char *who) {
  dim3 grid((unsigned)ceil_div((int64_t)max_pages * kPageSize, kScoreThreads), batch);
  // Heads per pass: hq rounded up to a multiple of 8, every head in one pass up to 64 (each
  // repeated head would cost a load and an exponential per token).
  const int nh = hq >= 64 ? 64 : ((hq + 7) / 8) * 8;
  auto launch = [&](auto k) {
    hipLaunchKernelGGL(k, grid, dim3(kScoreThreads), 0, stream, dump, sdb, sdh, lse, kv_indptr, last, scores,
                       score_stride, hq, max_pages);
  };
  switch (nh) {
    case 8: launch(legacy_softmax_score_kernel<8>); break;
    case 16: launch(legacy_softmax_score_kernel<16>); break;
    case 24: launch(legacy_softmax_score_kernel<24>); break;
    case 32: launch(legacy_softmax_score_kernel<32>); break;
    case 40: launch(legacy_softmax_score_kernel<40>); break;
    case 48: launch(legacy_softmax_score_kernel<48>); break;
    case 56: launch(legacy_softmax_score_kernel<56>); break;
    default: launch(legacy_softmax_score_kernel<64>); break;
  }
  return check_launch(who);
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT size_t delta_page_score_workspace_bytes(int batch, int num_qo_heads) {
  return ((size_t)batch * num_qo_heads * sizeof(float) + 255) & ~(size_t)255;
}

extern "C" DELTA_EXPORT int delta_page_scores_from_logits(const float *logits_dump, int64_t dump_stride_b,
                                                          int64_t dump_stride_h, const float *lse,
                                                          const int32_t *kv_indptr,
                                                          const int32_t *kv_last_page_len, float *scores,
                                                          int64_t score_stride, int batch, int num_qo_heads,
                                                          int max_pages, void *workspace, size_t workspace_bytes,
                                                          delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_page_scores_from_logits";
  if (batch <= 0 || max_pages <= 0) return DELTA_OK;
  if (!logits_dump || !kv_indptr || !kv_last_page_len || !scores)
    return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (num_qo_heads <= 0 || num_qo_heads > kMaxHeads)
    return set_error(DELTA_ERR_INVALID, "%s: num_qo_heads must be in [1, %d]", who, kMaxHeads);
  if (score_stride < max_pages) return set_error(DELTA_ERR_INVALID, "%s: score_stride < max_pages", who);
  if (dump_stride_h < (int64_t)max_pages * kPageSize)
    return set_error(DELTA_ERR_INVALID, "%s: dump rows shorter than max_pages*16", who);
  hipStream_t st = (hipStream_t)stream;
  if (!lse) {
    const size_t need = delta_page_score_workspace_bytes(batch, num_qo_heads);
    if (!workspace || workspace_bytes < need)
      return set_error(DELTA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed", who, need);
    float *lse_ws = (float *)workspace;
    hipLaunchKernelGGL(dump_lse_kernel, dim3(batch * num_qo_heads), dim3(256), 0, st, logits_dump, dump_stride_b,
                       dump_stride_h, kv_indptr, kv_last_page_len, lse_ws, num_qo_heads,
                       max_pages * kPageSize);
    int rc = check_launch(who);
    if (rc) return rc;
    lse = lse_ws;
  }
  return launch_scores(logits_dump, dump_stride_b, dump_stride_h, lse, kv_indptr, kv_last_page_len, scores,
                       score_stride, batch, num_qo_heads, max_pages, st, who);
}

extern "C" DELTA_EXPORT size_t delta_page_score_kv_workspace_bytes(int batch, int num_qo_heads, int num_kv_heads,
                                                                   int max_pages_per_row) {
  // [partials of the K-only decode][lse], or, for the LDS scorer, its per-(kv head, token)
  // maxima [batch][hkv][max_pages * 16] (the larger of the two).
  const int ns = delta::decode_num_splits(batch, num_kv_heads, max_pages_per_row);
  const size_t lse_bytes = ((size_t)batch * num_qo_heads * sizeof(float) + 255) & ~(size_t)255;
  const size_t dump_path = delta::decode_workspace_bytes(batch, num_qo_heads, ns, false) + lse_bytes;
  if (num_kv_heads <= 0 || num_qo_heads % num_kv_heads ||
      !delta::tokmax_fits(batch, num_kv_heads, num_qo_heads / num_kv_heads, max_pages_per_row))
    return dump_path;
  const size_t tm = ((size_t)batch * num_kv_heads * max_pages_per_row * delta::kPageSize * sizeof(float) + 255) &
                    ~(size_t)255;
  return tm > dump_path ? tm : dump_path;
}

extern "C" DELTA_EXPORT int delta_page_score_needs_dump(int batch, int num_qo_heads, int num_kv_heads,
                                                        int max_pages_per_row) {
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads) return 1;
  return delta::tokmax_fits(batch, num_kv_heads, num_qo_heads / num_kv_heads, max_pages_per_row) ? 0 : 1;
}

extern "C" DELTA_EXPORT int delta_page_score(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                             const void *kv_cache, int64_t num_pages, const int32_t *kv_indptr,
                                             const int32_t *kv_indices, int64_t kv_indices_len,
                                             const int32_t *kv_last_page_len, float *logits_dump,
                                             int64_t dump_stride_b, int64_t dump_stride_h, float *scores,
                                             int64_t score_stride, int batch, int num_qo_heads, int num_kv_heads,
                                             int head_dim, int dtype, float sm_scale, int max_pages,
                                             void *workspace, size_t workspace_bytes, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_page_score";
  if (batch <= 0 || max_pages <= 0) return DELTA_OK;
  if (!scores) return set_error(DELTA_ERR_INVALID, "%s: null output pointer", who);
  if (num_qo_heads > kMaxHeads) return set_error(DELTA_ERR_INVALID, "%s: too many heads", who);
  if (num_kv_heads <= 0 || num_qo_heads % num_kv_heads)
    return set_error(DELTA_ERR_INVALID, "%s: num_qo_heads must be a multiple of num_kv_heads", who);
  if (score_stride < max_pages) return set_error(DELTA_ERR_INVALID, "%s: score_stride < max_pages", who);
  if (logits_dump && dump_stride_h < (int64_t)max_pages * kPageSize)
    return set_error(DELTA_ERR_INVALID, "%s: dump rows shorter than max_pages*16", who);
  const bool lds_path = !logits_dump && tokmax_fits(batch, num_kv_heads, num_qo_heads / num_kv_heads, max_pages);
  if (!logits_dump && !lds_path)
    return set_error(DELTA_ERR_INVALID, "%s: this shape needs a logits dump buffer", who);
  const size_t need = delta_page_score_kv_workspace_bytes(batch, num_qo_heads, num_kv_heads, max_pages);
  if (!workspace || workspace_bytes < need)
    return set_error(DELTA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who, need, workspace_bytes);
  if ((uintptr_t)workspace & 255u) return set_error(DELTA_ERR_INVALID, "%s: workspace must be 256-byte aligned", who);
  hipStream_t st = (hipStream_t)stream;
  if (lds_path) {
    // One launch streams K once and leaves per-(kv head, token) maxima; a second sums pages.
    float *tm = (float *)workspace;
    const int64_t sh = (int64_t)max_pages * kPageSize, sb = (int64_t)num_kv_heads * sh;
    int rc = run_decode(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices, kv_indices_len,
                        kv_last_page_len, nullptr, 0, 0, nullptr, tm, sb, sh, batch, num_qo_heads, num_kv_heads,
                        head_dim, dtype, sm_scale, max_pages, /*kScoreTokmax*/ 4, nullptr, 0, st, who, nullptr);
    if (rc) return rc;
    launch_tokmax_scores(tm, sb, sh, num_kv_heads, kv_indptr, kv_last_page_len, scores, score_stride, batch,
                         max_pages, st);
    return check_launch(who);
  }
  const int ns = decode_num_splits(batch, num_kv_heads, max_pages);
  const size_t dec = decode_workspace_bytes(batch, num_qo_heads, ns, false);
  float *lse_ws = (float *)((char *)workspace + dec);
  int rc = run_decode(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices, kv_indices_len,
                      kv_last_page_len, nullptr, 0, 0, lse_ws, logits_dump, dump_stride_b, dump_stride_h, batch,
                      num_qo_heads, num_kv_heads, head_dim, dtype, sm_scale, max_pages, /*kScoreOnly*/ 2, workspace,
                      dec, st, who, nullptr);
  if (rc) return rc;
  return launch_scores(logits_dump, dump_stride_b, dump_stride_h, lse_ws, kv_indptr, kv_last_page_len, scores,
                       score_stride, batch, num_qo_heads, max_pages, st, who);
}

// The planner layer in one launch pair: attention (o, lse) with the row's logits kept in LDS,
// written as per-(kv head, token) maxima, then the page sums -- the same scores as a logits
// dump followed by delta_page_scores_from_logits, without the dump's HBM round trip.
namespace delta {
namespace {
int run_decode_scores(const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *kv_cache,
                      int64_t num_pages, const int32_t *kv_indptr, const int32_t *kv_indices,
                      int64_t kv_indices_len, const int32_t *kv_last_page_len, void *o, int64_t o_stride_b,
                      int64_t o_stride_h, float *lse, float *scores, int64_t score_stride, int batch,
                      int num_qo_heads, int num_kv_heads, int head_dim, int dtype, float sm_scale, int max_pages,
                      void *workspace, size_t workspace_bytes, hipStream_t st, const char *who,
                      const delta_decode_append_t *ap) {
  clear_error();
  if (batch <= 0) return DELTA_OK;
  if (max_pages <= 0) return set_error(DELTA_ERR_INVALID, "%s: max_pages_per_row must be positive", who);
  if (!scores || !o) return set_error(DELTA_ERR_INVALID, "%s: null output pointer", who);
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads)
    return set_error(DELTA_ERR_INVALID, "%s: num_qo_heads must be a multiple of num_kv_heads", who);
  if (num_qo_heads > kMaxHeads) return set_error(DELTA_ERR_INVALID, "%s: too many heads", who);
  if (score_stride < max_pages) return set_error(DELTA_ERR_INVALID, "%s: score_stride < max_pages", who);
  if (!plan_tokmax_fits(batch, num_kv_heads, num_qo_heads / num_kv_heads, max_pages, ap != nullptr))
    return set_error(DELTA_ERR_INVALID, "%s: this shape does not fit the on-chip planner "
                     "(delta_paged_decode_scores_supported); use the logits dump", who);
  const size_t need = delta_paged_decode_scores_workspace_bytes(batch, num_kv_heads, max_pages);
  if (!workspace || workspace_bytes < need)
    return set_error(DELTA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who, need, workspace_bytes);
  if ((uintptr_t)workspace & 255u) return set_error(DELTA_ERR_INVALID, "%s: workspace must be 256-byte aligned", who);
  float *tm = (float *)workspace;
  const int64_t sh = (int64_t)max_pages * kPageSize, sb = (int64_t)num_kv_heads * sh;
  int rc = run_decode(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices, kv_indices_len,
                      kv_last_page_len, o, o_stride_b, o_stride_h, lse, tm, sb, sh, batch, num_qo_heads,
                      num_kv_heads, head_dim, dtype, sm_scale, max_pages, /*kAttnTokmax*/ 5, nullptr, 0, st, who,
                      ap);
  if (rc) return rc;
  launch_tokmax_scores(tm, sb, sh, num_kv_heads, kv_indptr, kv_last_page_len, scores, score_stride, batch, max_pages,
                       st);
  return check_launch(who);
}
}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT int delta_paged_decode_scores_supported(int batch, int num_qo_heads, int num_kv_heads,
                                                                int max_pages_per_row, int with_append) {
  if (batch <= 0 || num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads) return 0;
  if (num_qo_heads / num_kv_heads > delta::kMaxGroup || num_kv_heads > delta::kMaxWaves) return 0;
  return delta::plan_tokmax_fits(batch, num_kv_heads, num_qo_heads / num_kv_heads, max_pages_per_row,
                                 with_append != 0) ? 1 : 0;
}

extern "C" DELTA_EXPORT size_t delta_paged_decode_scores_workspace_bytes(int batch, int num_kv_heads,
                                                                         int max_pages_per_row) {
  // The per-(kv head, token) maxima [batch][hkv][max_pages * 16].
  if (batch <= 0 || num_kv_heads <= 0 || max_pages_per_row <= 0) return 0;
  return ((size_t)batch * num_kv_heads * max_pages_per_row * delta::kPageSize * sizeof(float) + 255) & ~(size_t)255;
}

extern "C" DELTA_EXPORT int delta_paged_decode_scores(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                                      const void *kv_cache, int64_t num_pages,
                                                      const int32_t *kv_indptr, const int32_t *kv_indices,
                                                      int64_t kv_indices_len, const int32_t *kv_last_page_len,
                                                      void *o, int64_t o_stride_b, int64_t o_stride_h, float *lse,
                                                      float *scores, int64_t score_stride, int batch,
                                                      int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
                                                      float sm_scale, int max_pages_per_row, void *workspace,
                                                      size_t workspace_bytes, delta_stream_t stream) {
  return delta::run_decode_scores(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices,
                                  kv_indices_len, kv_last_page_len, o, o_stride_b, o_stride_h, lse, scores,
                                  score_stride, batch, num_qo_heads, num_kv_heads, head_dim, dtype, sm_scale,
                                  max_pages_per_row, workspace, workspace_bytes, (hipStream_t)stream,
                                  "delta_paged_decode_scores", nullptr);
}

extern "C" DELTA_EXPORT int delta_paged_decode_scores_append(
    const delta_decode_append_t *append, const void *q, int64_t q_stride_b, int64_t q_stride_h, void *kv_cache,
    int64_t num_pages, const int32_t *kv_indptr, const int32_t *kv_indices, int64_t kv_indices_len,
    const int32_t *kv_last_page_len, void *o, int64_t o_stride_b, int64_t o_stride_h, float *lse, float *scores,
    int64_t score_stride, int batch, int num_qo_heads, int num_kv_heads, int head_dim, int dtype, float sm_scale,
    int max_pages_per_row, void *workspace, size_t workspace_bytes, delta_stream_t stream) {
  if (!append) {
    delta::clear_error();
    return delta::set_error(DELTA_ERR_INVALID, "delta_paged_decode_scores_append: null append");
  }
  return delta::run_decode_scores(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices,
                                  kv_indices_len, kv_last_page_len, o, o_stride_b, o_stride_h, lse, scores,
                                  score_stride, batch, num_qo_heads, num_kv_heads, head_dim, dtype, sm_scale,
                                  max_pages_per_row, workspace, workspace_bytes, (hipStream_t)stream,
                                  "delta_paged_decode_scores_append", append);
}
