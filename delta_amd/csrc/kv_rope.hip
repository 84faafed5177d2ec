// KV-cache append and interleaved RoPE for gfx950.
//
// delta_append_kv replaces mylib::update_kv (hoenza/DELTA utils.py:31-79),
// which chains FlashInfer get_seq_lens -> get_batch_indices_positions ->
// append_paged_kv_cache.  One block per appended token; each thread moves 16
// bytes of K or V into page kv_indices[kv_indptr[b] + pos/16], slot pos % 16.
//
// delta_rope replaces mylib::rope (model.py:152-175: FlashInfer apply_rope /
// apply_llama31_rope with interleave=True).  Published formula: pair
// (2j, 2j+1) of every head rotates by angle pos * f_j with
// f_j = theta^(-2j/d) / rope_scale, or for Llama 3.1 the blend
// (1 - s) f_j/rope_scale + s f_j, s = clamp(f_j * old_ctx / (2 pi (hi - lo)) - 1/(hi/lo - 1), 0, 1).
// fp32 angle and fp32 sin/cos as the reference's kernel; fp32 rotation, one
// rounding to the storage dtype.  A block computes the 64 (cos, sin) pairs of its
// token's position once, in LDS, and every head reads them.
//
// delta_rope_append fuses the two for a decode layer (Attention.forward, model.py:
// 413-418): RoPE of q and k, then the append of the rotated k and of v -- one launch,
// and k never makes a round trip through HBM before it lands in its page.  Same
// arithmetic per element as delta_rope followed by delta_append_kv, so q and the
// cache come out bit-identical.
#include "delta_common.h"

namespace delta {
namespace {

// Row of token i under a CSR indptr (uniform binary search).
__device__ __forceinline__ int find_row(const int32_t *indptr, int batch, int i) {
  int lo = 0, hi = batch;  // indptr[lo] <= i < indptr[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (indptr[mid] <= i)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

struct AppendArgs {
  const uint16_t *k;
  int64_t k_stride;
  const uint16_t *v;
  int64_t v_stride;
  const int32_t *append_indptr;
  uint16_t *cache;
  int64_t num_pages;
  const int32_t *kv_indices;
  int64_t kv_indices_len;
  const int32_t *kv_indptr;
  const int32_t *last_page_len;
  int batch, hkv;
};

__global__ void __launch_bounds__(256) append_kv_kernel(AppendArgs a) {
  const int i = blockIdx.x;
  const int b = find_row(a.append_indptr, a.batch, i);
  const int a0 = a.append_indptr[b];
  const int alen = a.append_indptr[b + 1] - a0;
  if (i < a0 || i - a0 >= alen) return;
  int64_t p0 = a.kv_indptr[b], p1 = a.kv_indptr[b + 1];
  if (p0 < 0 || p1 < p0 || p1 > a.kv_indices_len) return;
  const int np = (int)(p1 - p0);
  int lp = a.last_page_len[b];
  lp = lp < 0 ? 0 : (lp > kPageSize ? kPageSize : lp);
  const int seq = np > 0 ? (np - 1) * kPageSize + lp : lp;
  const int pos = seq - alen + (i - a0);
  if (pos < 0 || pos / kPageSize >= np) return;
  const int pid = a.kv_indices[p0 + pos / kPageSize];
  if (pid < 0 || (int64_t)pid >= a.num_pages) return;
  const int slot = pos % kPageSize;
  const int64_t row_elems = (int64_t)a.hkv * kHeadDim;
  const int chunks = a.hkv * (kHeadDim / 8);  // 16-byte chunks per token row
  for (int ch = threadIdx.x; ch < 2 * chunks; ch += blockDim.x) {
    const int which = ch >= chunks;  // 0 = K, 1 = V
    const int r = which ? ch - chunks : ch;
    const uint16_t *src = which ? a.v + (int64_t)i * a.v_stride : a.k + (int64_t)i * a.k_stride;
    uint16_t *dst = a.cache + (((int64_t)pid * 2 + which) * kPageSize + slot) * row_elems;
    st128(dst + 8 * r, ld128(src + 8 * r));
  }
}

struct RopeArgs {
  const uint16_t *q;
  int64_t q_stride;
  const uint16_t *k;
  int64_t k_stride;
  uint16_t *q_out;
  int64_t q_out_stride;
  uint16_t *k_out;
  int64_t k_out_stride;
  const int32_t *indptr;
  const int32_t *offsets;
  int batch, hq, hkv;
  float rcp_scale, log2_theta, smooth_a, smooth_b;
};

constexpr int kPairs = kHeadDim / 2;

// (cos, sin) of pos * f_j for the 64 pairs j, into tab[2 j], tab[2 j + 1] (threads 0..63).
__device__ __forceinline__ void rope_table(const RopeArgs &a, float pos, float *tab) {
  const int j = threadIdx.x;
  if (j < kPairs) rope_cos_sin(j, pos, a.rcp_scale, a.log2_theta, a.smooth_a, a.smooth_b, tab + 2 * j);
}

template <int DT>
__device__ __forceinline__ uint32_t rope_pair(uint32_t pr, const float *tab, int j) {
  return rope_rotate<DT>(pr, tab + 2 * j);
}

template <int DT>
__global__ void __launch_bounds__(256) rope_kernel(RopeArgs a) {
  __shared__ float tab[2 * kPairs];
  const int i = blockIdx.x;
  const int b = find_row(a.indptr, a.batch, i);
  const float pos = (float)(a.offsets[b] + (i - a.indptr[b]));
  rope_table(a, pos, tab);
  __syncthreads();
  const int total = (a.hq + a.hkv) * kPairs;
  for (int w = threadIdx.x; w < total; w += blockDim.x) {
    const int head = w / kPairs;
    const int j = w % kPairs;
    const bool is_q = head < a.hq;
    const uint16_t *src = is_q ? a.q + (int64_t)i * a.q_stride + (int64_t)head * kHeadDim
                               : a.k + (int64_t)i * a.k_stride + (int64_t)(head - a.hq) * kHeadDim;
    uint16_t *dst = is_q ? a.q_out + (int64_t)i * a.q_out_stride + (int64_t)head * kHeadDim
                         : a.k_out + (int64_t)i * a.k_out_stride + (int64_t)(head - a.hq) * kHeadDim;
    const uint32_t pr = *reinterpret_cast<const uint32_t *>(src + 2 * j);
    *reinterpret_cast<uint32_t *>(dst + 2 * j) = rope_pair<DT>(pr, tab, j);
  }
}

// Fused RoPE + append, one block per token: q heads rotated into q_out, k heads rotated
// straight into the token's page slot, v copied there (the slot as delta_append_kv finds it).
template <int DT>
__global__ void __launch_bounds__(256) rope_append_kernel(RopeArgs r, AppendArgs a) {
  __shared__ float tab[2 * kPairs];
  const int i = blockIdx.x;
  const int b = find_row(a.append_indptr, a.batch, i);
  const int a0 = a.append_indptr[b];
  const float pos = (float)(r.offsets[b] + (i - a0));
  rope_table(r, pos, tab);
  // The cache slot (checks as in append_kv_kernel; an invalid slot drops the K/V write only).
  const int alen = a.append_indptr[b + 1] - a0;
  const int64_t p0 = a.kv_indptr[b], p1 = a.kv_indptr[b + 1];
  int pid = -1, slot = 0;
  if (i >= a0 && i - a0 < alen && p0 >= 0 && p1 >= p0 && p1 <= a.kv_indices_len) {
    const int np = (int)(p1 - p0);
    int lp = a.last_page_len[b];
    lp = lp < 0 ? 0 : (lp > kPageSize ? kPageSize : lp);
    const int seq = np > 0 ? (np - 1) * kPageSize + lp : lp;
    const int apos = seq - alen + (i - a0);
    if (apos >= 0 && apos / kPageSize < np) {
      const int p = a.kv_indices[p0 + apos / kPageSize];
      if (p >= 0 && (int64_t)p < a.num_pages) {
        pid = p;
        slot = apos % kPageSize;
      }
    }
  }
  const int64_t row_elems = (int64_t)a.hkv * kHeadDim;
  uint16_t *kdst = a.cache + (((int64_t)(pid < 0 ? 0 : pid) * 2 + 0) * kPageSize + slot) * row_elems;
  uint16_t *vdst = a.cache + (((int64_t)(pid < 0 ? 0 : pid) * 2 + 1) * kPageSize + slot) * row_elems;
  __syncthreads();
  const int total = (r.hq + r.hkv) * kPairs;
  for (int w = threadIdx.x; w < total; w += blockDim.x) {
    const int head = w / kPairs;
    const int j = w % kPairs;
    if (head < r.hq) {
      const uint32_t pr = *reinterpret_cast<const uint32_t *>(r.q + (int64_t)i * r.q_stride + (int64_t)head * kHeadDim + 2 * j);
      *reinterpret_cast<uint32_t *>(r.q_out + (int64_t)i * r.q_out_stride + (int64_t)head * kHeadDim + 2 * j) =
          rope_pair<DT>(pr, tab, j);
    } else if (pid >= 0) {
      const int hk = head - r.hq;
      const uint32_t pr = *reinterpret_cast<const uint32_t *>(r.k + (int64_t)i * r.k_stride + (int64_t)hk * kHeadDim + 2 * j);
      *reinterpret_cast<uint32_t *>(kdst + (int64_t)hk * kHeadDim + 2 * j) = rope_pair<DT>(pr, tab, j);
    }
  }
  if (pid >= 0) {
    for (int ch = threadIdx.x; ch < a.hkv * (kHeadDim / 8); ch += blockDim.x)
      st128(vdst + 8 * ch, ld128(a.v + (int64_t)i * a.v_stride + 8 * ch));
  }
}


// The same fused RoPE + append for 16-byte aligned q, k, v and q_out (the decode layer's
// case), arranged for latency: the token's q, k and v are loaded first (they are addressed by
// the token index alone), the row is found with one parallel probe of the append indptr
// (thread t tests indptr[t] <= i < indptr[t + 1]) instead of a binary search, so the chain
// of dependent loads is indptr -> (offsets, kv_indptr, last_page_len) -> kv_indices.  The
// arithmetic per element is rope_append_kernel's, so both give identical bits.
constexpr int kRopeThreads = 256;
constexpr int kRopePre = 3;  // 16-byte q/k chunks per thread loaded ahead (40 heads at 256 threads)

template <int DT>
__global__ void __launch_bounds__(kRopeThreads) rope_append_vec_kernel(RopeArgs r, AppendArgs a) {
  __shared__ float tab[2 * kPairs];
  __shared__ int row_s;
  const int i = blockIdx.x;
  const int tid = threadIdx.x;
  const int nqk = (r.hq + r.hkv) * (kHeadDim / 8);
  const int nv = a.hkv * (kHeadDim / 8);
  auto qk_src = [&](int u) {
    const int head = u >> 4, c = u & 15;
    return head < r.hq ? r.q + (int64_t)i * r.q_stride + (int64_t)head * kHeadDim + 8 * c
                       : r.k + (int64_t)i * r.k_stride + (int64_t)(head - r.hq) * kHeadDim + 8 * c;
  };
  u32x4 pre[kRopePre];
#pragma unroll
  for (int c = 0; c < kRopePre; ++c) {
    const int u = tid + kRopeThreads * c;
    if (u < nqk) pre[c] = ld128(qk_src(u));
  }
  const u32x4 v0 = tid < nv ? ld128(a.v + (int64_t)i * a.v_stride + 8 * tid) : u32x4{0u, 0u, 0u, 0u};

  if (tid == 0) row_s = -1;
  __syncthreads();
  for (int t = tid; t < a.batch; t += kRopeThreads)
    if (a.append_indptr[t] <= i && i < a.append_indptr[t + 1]) row_s = t;
  __syncthreads();
  // A token outside every row (malformed indptr) takes the binary search's row, as the
  // unfused kernels do.
  const int b = row_s >= 0 ? row_s : find_row(a.append_indptr, a.batch, i);
  const int a0 = a.append_indptr[b];
  const float pos = (float)(r.offsets[b] + (i - a0));
  const int alen = a.append_indptr[b + 1] - a0;
  const int64_t p0 = a.kv_indptr[b], p1 = a.kv_indptr[b + 1];
  int pid = -1, slot = 0;
  if (i >= a0 && i - a0 < alen && p0 >= 0 && p1 >= p0 && p1 <= a.kv_indices_len) {
    const int np = (int)(p1 - p0);
    int lp = a.last_page_len[b];
    lp = lp < 0 ? 0 : (lp > kPageSize ? kPageSize : lp);
    const int seq = np > 0 ? (np - 1) * kPageSize + lp : lp;
    const int apos = seq - alen + (i - a0);
    if (apos >= 0 && apos / kPageSize < np) {
      const int p = a.kv_indices[p0 + apos / kPageSize];
      if (p >= 0 && (int64_t)p < a.num_pages) {
        pid = p;
        slot = apos % kPageSize;
      }
    }
  }
  rope_table(r, pos, tab);
  const int64_t row_elems = (int64_t)a.hkv * kHeadDim;
  uint16_t *kdst = a.cache + (((int64_t)(pid < 0 ? 0 : pid) * 2 + 0) * kPageSize + slot) * row_elems;
  uint16_t *vdst = a.cache + (((int64_t)(pid < 0 ? 0 : pid) * 2 + 1) * kPageSize + slot) * row_elems;
  __syncthreads();

  auto rotate_store = [&](int u, u32x4 x) {
    const int head = u >> 4, c = u & 15;
    u32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = rope_pair<DT>(x[e], tab, 4 * c + e);
    if (head < r.hq)
      st128(r.q_out + (int64_t)i * r.q_out_stride + (int64_t)head * kHeadDim + 8 * c, y);
    else if (pid >= 0)
      st128(kdst + (int64_t)(head - r.hq) * kHeadDim + 8 * c, y);
  };
#pragma unroll
  for (int c = 0; c < kRopePre; ++c) {
    const int u = tid + kRopeThreads * c;
    if (u < nqk) rotate_store(u, pre[c]);
  }
  for (int u = tid + kRopeThreads * kRopePre; u < nqk; u += kRopeThreads) rotate_store(u, ld128(qk_src(u)));
  if (pid >= 0) {
    if (tid < nv) st128(vdst + 8 * tid, v0);
    for (int u = tid + kRopeThreads; u < nv; u += kRopeThreads)
      st128(vdst + 8 * u, ld128(a.v + (int64_t)i * a.v_stride + 8 * u));
  }
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT int delta_append_kv(const void *k, int64_t k_stride, const void *v, int64_t v_stride,
                                            const int32_t *kv_append_indptr, void *kv_cache, int64_t num_pages,
                                            const int32_t *kv_indices, int64_t kv_indices_len,
                                            const int32_t *kv_indptr, const int32_t *kv_last_page_len, int nnz,
                                            int batch, int num_kv_heads, int head_dim, int dtype,
                                            delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_append_kv";
  if (nnz <= 0 || batch <= 0) return DELTA_OK;
  if (head_dim != kHeadDim) return set_error(DELTA_ERR_INVALID, "%s: head_dim must be 128", who);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: bad dtype", who);
  if (!k || !v || !kv_append_indptr || !kv_cache || !kv_indices || !kv_indptr || !kv_last_page_len)
    return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)kv_cache) & 15u || (k_stride % 8) || (v_stride % 8))
    return set_error(DELTA_ERR_INVALID, "%s: k/v/cache must be 16-byte aligned with strides in multiples of 8", who);
  AppendArgs a;
  a.k = (const uint16_t *)k;
  a.k_stride = k_stride;
  a.v = (const uint16_t *)v;
  a.v_stride = v_stride;
  a.append_indptr = kv_append_indptr;
  a.cache = (uint16_t *)kv_cache;
  a.num_pages = num_pages;
  a.kv_indices = kv_indices;
  a.kv_indices_len = kv_indices_len;
  a.kv_indptr = kv_indptr;
  a.last_page_len = kv_last_page_len;
  a.batch = batch;
  a.hkv = num_kv_heads;
  const int threads = 2 * num_kv_heads * (kHeadDim / 8) >= 256 ? 256 : 128;
  hipLaunchKernelGGL(append_kv_kernel, dim3(nnz), dim3(threads), 0, (hipStream_t)stream, a);
  return check_launch(who);
}

extern "C" DELTA_EXPORT int delta_rope(const void *q, int64_t q_stride, const void *k, int64_t k_stride, void *q_out,
                                       int64_t q_out_stride, void *k_out, int64_t k_out_stride, const int32_t *indptr,
                                       const int32_t *offsets, int nnz, int batch, int num_qo_heads, int num_kv_heads,
                                       int head_dim, int dtype, float rope_scale, float rope_theta, int llama31,
                                       float low_freq_factor, float high_freq_factor, float old_context_len,
                                       delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_rope";
  if (nnz <= 0 || batch <= 0) return DELTA_OK;
  if (head_dim != kHeadDim) return set_error(DELTA_ERR_INVALID, "%s: head_dim must be 128", who);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: bad dtype", who);
  if (!q || !k || !q_out || !k_out || !indptr || !offsets) return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)q_out | (uintptr_t)k_out) & 3u)
    return set_error(DELTA_ERR_INVALID, "%s: tensors must be 4-byte aligned", who);
  if (!(rope_scale > 0.f) || !(rope_theta > 0.f)) return set_error(DELTA_ERR_INVALID, "%s: bad rope params", who);
  RopeArgs a;
  a.q = (const uint16_t *)q;
  a.q_stride = q_stride;
  a.k = (const uint16_t *)k;
  a.k_stride = k_stride;
  a.q_out = (uint16_t *)q_out;
  a.q_out_stride = q_out_stride;
  a.k_out = (uint16_t *)k_out;
  a.k_out_stride = k_out_stride;
  a.indptr = indptr;
  a.offsets = offsets;
  a.batch = batch;
  a.hq = num_qo_heads;
  a.hkv = num_kv_heads;
  a.rcp_scale = 1.0f / rope_scale;
  a.log2_theta = log2f(rope_theta);
  if (llama31) {
    if (!(high_freq_factor > low_freq_factor) || !(low_freq_factor > 0.f))
      return set_error(DELTA_ERR_INVALID, "%s: bad llama3.1 frequency factors", who);
    const float two_pi = 6.283185307179586f;
    a.smooth_a = old_context_len / (two_pi * high_freq_factor - two_pi * low_freq_factor);
    a.smooth_b = -1.0f / (high_freq_factor / low_freq_factor - 1.0f);
  } else {
    a.smooth_a = 0.f;
    a.smooth_b = 0.f;
  }
  if (dtype == DELTA_BF16)
    hipLaunchKernelGGL(rope_kernel<DELTA_BF16>, dim3(nnz), dim3(256), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(rope_kernel<DELTA_FP16>, dim3(nnz), dim3(256), 0, (hipStream_t)stream, a);
  return check_launch(who);
}

extern "C" DELTA_EXPORT int delta_rope_append(const void *q, int64_t q_stride, const void *k, int64_t k_stride,
                                              const void *v, int64_t v_stride, void *q_out, int64_t q_out_stride,
                                              const int32_t *kv_append_indptr, const int32_t *offsets,
                                              void *kv_cache, int64_t num_pages, const int32_t *kv_indices,
                                              int64_t kv_indices_len, const int32_t *kv_indptr,
                                              const int32_t *kv_last_page_len, int nnz, int batch,
                                              int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
                                              float rope_scale, float rope_theta, int llama31, float low_freq_factor,
                                              float high_freq_factor, float old_context_len, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_rope_append";
  if (nnz <= 0 || batch <= 0) return DELTA_OK;
  if (head_dim != kHeadDim) return set_error(DELTA_ERR_INVALID, "%s: head_dim must be 128", who);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: bad dtype", who);
  if (!q || !k || !v || !q_out || !kv_append_indptr || !offsets || !kv_cache || !kv_indices || !kv_indptr ||
      !kv_last_page_len)
    return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)q_out) & 3u || ((uintptr_t)v | (uintptr_t)kv_cache) & 15u ||
      (v_stride % 8))
    return set_error(DELTA_ERR_INVALID, "%s: q/k 4-byte, v/cache 16-byte aligned, v stride a multiple of 8", who);
  if (!(rope_scale > 0.f) || !(rope_theta > 0.f)) return set_error(DELTA_ERR_INVALID, "%s: bad rope params", who);
  RopeArgs r;
  r.q = (const uint16_t *)q;
  r.q_stride = q_stride;
  r.k = (const uint16_t *)k;
  r.k_stride = k_stride;
  r.q_out = (uint16_t *)q_out;
  r.q_out_stride = q_out_stride;
  r.k_out = nullptr;
  r.k_out_stride = 0;
  r.indptr = kv_append_indptr;
  r.offsets = offsets;
  r.batch = batch;
  r.hq = num_qo_heads;
  r.hkv = num_kv_heads;
  r.rcp_scale = 1.0f / rope_scale;
  r.log2_theta = log2f(rope_theta);
  if (llama31) {
    if (!(high_freq_factor > low_freq_factor) || !(low_freq_factor > 0.f))
      return set_error(DELTA_ERR_INVALID, "%s: bad llama3.1 frequency factors", who);
    const float two_pi = 6.283185307179586f;
    r.smooth_a = old_context_len / (two_pi * high_freq_factor - two_pi * low_freq_factor);
    r.smooth_b = -1.0f / (high_freq_factor / low_freq_factor - 1.0f);
  } else {
    r.smooth_a = 0.f;
    r.smooth_b = 0.f;
  }
  AppendArgs a;
  a.k = nullptr;
  a.k_stride = 0;
  a.v = (const uint16_t *)v;
  a.v_stride = v_stride;
  a.append_indptr = kv_append_indptr;
  a.cache = (uint16_t *)kv_cache;
  a.num_pages = num_pages;
  a.kv_indices = kv_indices;
  a.kv_indices_len = kv_indices_len;
  a.kv_indptr = kv_indptr;
  a.last_page_len = kv_last_page_len;
  a.batch = batch;
  a.hkv = num_kv_heads;
  const bool vec = !(((uintptr_t)q | (uintptr_t)k | (uintptr_t)q_out) & 15u) && !(q_stride % 8) &&
                   !(k_stride % 8) && !(q_out_stride % 8);
  if (vec && dtype == DELTA_BF16)
    hipLaunchKernelGGL(rope_append_vec_kernel<DELTA_BF16>, dim3(nnz), dim3(kRopeThreads), 0, (hipStream_t)stream, r, a);
  else if (vec)
    hipLaunchKernelGGL(rope_append_vec_kernel<DELTA_FP16>, dim3(nnz), dim3(kRopeThreads), 0, (hipStream_t)stream, r, a);
  else if (dtype == DELTA_BF16)
    hipLaunchKernelGGL(rope_append_kernel<DELTA_BF16>, dim3(nnz), dim3(256), 0, (hipStream_t)stream, r, a);
  else
    hipLaunchKernelGGL(rope_append_kernel<DELTA_FP16>, dim3(nnz), dim3(256), 0, (hipStream_t)stream, r, a);
  return check_launch(who);
}
