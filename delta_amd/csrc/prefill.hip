// Causal paged prefill attention for gfx950 (several query tokens per row, GQA).
//
// Replaces FlashInfer's BatchPrefillWithPagedKVCacheWrapper.run with causal=True for rows
// with qo_len > 1 (hoenza/DELTA backend.py:1091-1105, the prompt steps of the engine).  The
// cache already holds the row's new tokens (update_kv runs before attention, model.py:413-418),
// so query i of row b sits at position kv_len_b - qo_len_b + i and attends tokens 0..position.
//
// Work decomposition: block = 8 waves of one (row, kv head) and 8 * TW consecutive query
// tokens; each wave owns TW = 16 / G tokens and puts their (token, q head) pairs in the 16
// columns of its MFMA tiles.  The block sweeps the pages up to its last token's position:
// each page's K and V (4 KiB each for one head) are loaded once per block, 16 bytes per thread,
// into double-buffered LDS tiles kGroup pages at a time (the next group in flight in
// registers), and all waves read them from there; a wave whose tokens end earlier skips the
// later pages, and groups below every column's diagonal skip the element masks.  No merge.
//   q.K : S^T = K Q^T with v_mfma_f32_16x16x32 -- A = the page's 16 K rows from LDS
//         (lane%16 = token, lane/16 picks d in [32s + 8c, +8) at step s), B = the wave's query
//         columns; D puts tokens 4c..4c+3 of column j = lane%16 in lane (c, j);
//   softmax: online per column in the log2 domain, causal and kv_len masks per element;
//   P.V : v_mfma_f32_16x16x16 -- A = P (row = column j, k = tokens 4c..), B = V from the
//         padded LDS tile read with ds_read_b64_tr_b16, D = O[column 4c + r][16n + lane%16].
// Page ids are preloaded 64 per register, as in the decode kernel.
#include "delta_common.h"

namespace delta {
namespace {

constexpr int kPrefillWaves = 8;  // waves per block: 8 x 16 (token, head) columns share each K/V page
constexpr int kGroup = 2;         // pages per LDS buffer (and per barrier)
constexpr int kVStrideP = 136;    // padded tile row (elements)

struct PrefillArgs {
  const uint16_t *q;
  int64_t q_stride_t, q_stride_h;
  const uint16_t *kv;
  int64_t num_pages;
  const int32_t *qo_indptr;
  const int32_t *kv_indptr;
  const int32_t *kv_indices;
  int64_t kv_indices_len;
  const int32_t *last_page_len;
  uint16_t *o;
  int64_t o_stride_t, o_stride_h;
  float *lse;
  int batch, hq, hkv;
  float sm_scale;
};

template <int DT>
struct PMfma;
template <>
struct PMfma<DELTA_BF16> {
  typedef short s4 __attribute__((ext_vector_type(4)));
  __device__ __forceinline__ static f32x4 run(s4 a, s4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static short pack(float x) { return __builtin_bit_cast(short, (__bf16)x); }
};
template <>
struct PMfma<DELTA_FP16> {
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  __device__ __forceinline__ static f32x4 run(s4 a, s4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static short pack(float x) { return __builtin_bit_cast(short, (_Float16)x); }
};

typedef short ps4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ps4_t lds_ps4_t;

__device__ __forceinline__ float prows4_max(float v) {
  auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
  auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(y[0]), __uint_as_float(y[1]));
}
__device__ __forceinline__ float prows4_sum(float v) {
  auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(y[0]) + __uint_as_float(y[1]);
}

template <int DT, int G>
__global__ void __launch_bounds__(kPrefillWaves * 64) paged_prefill_kernel(PrefillArgs a) {
#pragma clang fp contract(off)
  using E = Elem<DT>;
  using M16 = PMfma<DT>;
  constexpr int TW = 16 / G;                  // query tokens per wave
  constexpr int BT = kPrefillWaves * TW;      // query tokens per block
  constexpr int kTile = kPageSize * kVStrideP;  // one K or V tile (elements)
  // Two page buffers, each K then V (padded rows), shared by the block's waves.
  __shared__ uint16_t tiles[2][kGroup][2 * kTile];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane >> 4, t = lane & 15;
  const int b = blockIdx.z, h = blockIdx.y;
  const int64_t q0 = a.qo_indptr[b], q1 = a.qo_indptr[b + 1];
  const int qn = q1 > q0 ? (int)(q1 - q0) : 0;
  const int btok0 = blockIdx.x * BT;
  if (btok0 >= qn) return;  // whole block
  const int tok0 = btok0 + wave * TW;

  // Row's pages and length (indptr entries clamped as in the decode kernels).
  const int64_t ilen = a.kv_indices_len;
  int64_t p0 = a.kv_indptr[b], p1 = a.kv_indptr[b + 1];
  p0 = p0 < 0 ? 0 : (p0 > ilen ? ilen : p0);
  p1 = p1 < p0 ? p0 : (p1 > ilen ? ilen : p1);
  const int np = (int)(p1 - p0);
  int lp = a.last_page_len[b];
  lp = lp < 0 ? 0 : (lp > kPageSize ? kPageSize : lp);
  const int kv_len = np > 0 ? (np - 1) * kPageSize + lp : 0;

  // Column t = (token tt, head g) of this wave.
  const int tt = t / G, g = t % G;
  const bool col_ok = t < TW * G && tok0 + tt < qn;
  const int qpos = kv_len - qn + tok0 + tt;  // attends tokens 0..qpos
  u32x4 qf[4];
  if (col_ok) {
    const uint16_t *qp = a.q + (q0 + tok0 + tt) * a.q_stride_t + (int64_t)(h * G + g) * a.q_stride_h + 8 * c;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = ld128(qp + 32 * s);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = u32x4{0u, 0u, 0u, 0u};
  }

  // Pages the block sweeps (up to its last token's position) and the ones this wave needs.
  auto pages_upto = [&](int last_tok) {
    const int pos = kv_len - qn + last_tok;
    const int n = pos >= 0 ? pos / kPageSize + 1 : 0;
    return n > np ? np : n;
  };
  const int count = pages_upto((btok0 + BT < qn ? btok0 + BT : qn) - 1);
  const int wcount = tok0 < qn ? pages_upto((tok0 + TW < qn ? tok0 + TW : qn) - 1) : 0;

  const int64_t row_elems = (int64_t)a.hkv * kHeadDim;
  const int64_t page_elems = 2 * kPageSize * row_elems;
  // Cooperative tile load: thread i < 512 moves 16 bytes -- K (i < 256) or V row (i / 16) % 16,
  // chunk i % 16 of head h.
  const bool loader = threadIdx.x < 2 * kPageSize * (kHeadDim / 8);
  const int ld_which = (threadIdx.x >> 8) & 1, ld_row = (threadIdx.x >> 4) & 15, ld_ch = threadIdx.x & 15;
  const int64_t ld_off = (int64_t)(ld_which * kPageSize + ld_row) * row_elems + (int64_t)h * kHeadDim + 8 * ld_ch;
  const int st_off = ld_which * kTile + ld_row * kVStrideP + 8 * ld_ch;

  // Page ids, 64 per register (lane i: page cbase + i), the next 64 a chunk ahead.
  auto load_ids = [&](int base) -> int {
    const int it = base + lane;
    int pid = -1;
    if (it < count) pid = a.kv_indices[p0 + it];
    return (pid >= 0 && (int64_t)pid < a.num_pages) ? pid : -1;
  };
  int cbase = 0;
  int ids = count > 0 ? load_ids(0) : -1;
  int ids_next = count > 64 ? load_ids(64) : -1;
  auto id_of = [&](int q) -> int {  // q in [cbase, cbase + 128)
    return q - cbase < 64 ? __builtin_amdgcn_readlane(ids, q - cbase) : __builtin_amdgcn_readlane(ids_next, q - cbase - 64);
  };
  auto fetch = [&](int q) -> u32x4 {
    const int pid = q < count ? id_of(q) : -1;
    if (pid < 0 || !loader) return u32x4{0u, 0u, 0u, 0u};
    return ld128(a.kv + (int64_t)pid * page_elems + ld_off);
  };
  // Pages go through LDS in groups of kGroup: one barrier, one softmax rescale and one buffer
  // swap per group.  Group gi sits in tiles[gi & 1]; group gi + 1 waits in registers (ring),
  // its loads issued a whole group earlier.  V rows past kv_len (or of an invalid page) are
  // stored as zeros: they may hold NaN/Inf and meet p = 0.
  u32x4 ring[kGroup];
  auto fetch_group = [&](int gi) {
#pragma unroll
    for (int pp = 0; pp < kGroup; ++pp) ring[pp] = fetch(gi * kGroup + pp);
  };
  auto stage_group = [&](int gi) {
#pragma unroll
    for (int pp = 0; pp < kGroup; ++pp) {
      const int q = gi * kGroup + pp;
      const bool keep = ld_which == 0 || q * kPageSize + ld_row < kv_len;
      if (loader && q < count) st128(&tiles[gi & 1][pp][st_off], keep ? ring[pp] : u32x4{0u, 0u, 0u, 0u});
    }
  };
  const int ngroups = (count + kGroup - 1) / kGroup;
  if (ngroups > 0) {
    fetch_group(0);
    stage_group(0);
    if (ngroups > 1) fetch_group(1);
  }

  float m = -INFINITY, l = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float scale2 = a.sm_scale * kLog2e;

  for (int gi = 0; gi < ngroups; ++gi) {
    const int j0 = gi * kGroup;
    __syncthreads();  // group gi is in tiles[gi & 1]; tiles[(gi + 1) & 1] is free
    if (j0 > 0 && (j0 & 63) == 0) {  // the id window moves on
      cbase += 64;
      ids = ids_next;
      ids_next = cbase + 64 < count ? load_ids(cbase + 64) : -1;
    }
    if (j0 < wcount) {
      f32x4 S[kGroup];
#pragma unroll
      for (int pp = 0; pp < kGroup; ++pp) S[pp] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sk = 0; sk < 4; ++sk)
#pragma unroll
        for (int pp = 0; pp < kGroup; ++pp)
          S[pp] = E::mfma(*reinterpret_cast<const u32x4 *>(&tiles[gi & 1][pp][t * kVStrideP + 32 * sk + 8 * c]),
                          qf[sk], S[pp]);
      float x[kGroup][4];
      float pm = -INFINITY;
      // Below the diagonal of every column and inside kv_len the group needs no element masks
      // (columns past the wave's tokens compute on zero q and are never written).
      bool ok[kGroup];
      bool all_ok = (j0 + kGroup) * kPageSize <= kv_len && (j0 + kGroup) * kPageSize - 1 <= kv_len - qn + tok0;
#pragma unroll
      for (int pp = 0; pp < kGroup; ++pp) {
        ok[pp] = j0 + pp < wcount && id_of(j0 + pp) >= 0;  // an id outside the cache contributes nothing
        all_ok = all_ok && ok[pp];
      }
      if (all_ok) {
#pragma unroll
        for (int pp = 0; pp < kGroup; ++pp)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            x[pp][r] = S[pp][r] * scale2;
            pm = fmaxf(pm, x[pp][r]);
          }
      } else {
#pragma unroll
        for (int pp = 0; pp < kGroup; ++pp)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int tk = (j0 + pp) * kPageSize + 4 * c + r;
            x[pp][r] = (ok[pp] && col_ok && tk <= qpos && tk < kv_len) ? S[pp][r] * scale2 : -INFINITY;
            pm = fmaxf(pm, x[pp][r]);
          }
      }
      const float mn = fmaxf(m, prows4_max(pm));
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float alpha = fast_exp2(m - mref);
      float ps = 0.f;
#pragma unroll
      for (int pp = 0; pp < kGroup; ++pp)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[pp][r] = fast_exp2(x[pp][r] - mref);
          ps += x[pp][r];
        }
      l = l * alpha + prows4_sum(ps);
      m = mn;
      if (__ballot(alpha != 1.f)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float al = shfl(alpha, 4 * c + r);
#pragma unroll
          for (int n = 0; n < 8; ++n) acc[n][r] *= al;
        }
      }
#pragma unroll
      for (int pp = 0; pp < kGroup; ++pp) {
        if (j0 + pp < wcount) {  // later slots may hold a stale or unset tile
          ps4_t pa;
#pragma unroll
          for (int r = 0; r < 4; ++r) pa[r] = M16::pack(x[pp][r]);
          const uint16_t *rd = &tiles[gi & 1][pp][kTile + (4 * c + (t >> 2)) * kVStrideP + 4 * (t & 3)];
#pragma unroll
          for (int n = 0; n < 8; ++n) {
            const ps4_t bv = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ps4_t *)(rd + 16 * n));
            acc[n] = M16::run(pa, bv, acc[n]);
          }
        }
      }
    }
    if (gi + 1 < ngroups) {
      stage_group(gi + 1);
      if (gi + 2 < ngroups) fetch_group(gi + 2);
    }
  }

  // Normalise and write: lane (c, t) holds O[column 4c + r][16n + t].
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int col = 4 * c + r;
    const float L = shfl(l, col);
    const int ctt = col / G, cg = col % G;
    if (col < TW * G && tok0 + ctt < qn) {
      uint16_t *op = a.o + (q0 + tok0 + ctt) * a.o_stride_t + (int64_t)(h * G + cg) * a.o_stride_h + t;
#pragma unroll
      for (int n = 0; n < 8; ++n) op[16 * n] = (uint16_t)E::from_float(L > 0.f ? acc[n][r] / L : 0.f);
    }
  }
  if (a.lse && c == 0 && col_ok)
    a.lse[(q0 + tok0 + tt) * a.hq + h * G + g] = l > 0.f ? (m + log2f(l)) * kLn2 : -INFINITY;
}

template <int DT>
void launch_prefill(const PrefillArgs &a, int G, int max_qo, hipStream_t stream) {
  const int tw = 16 / G;
  const dim3 grid((unsigned)ceil_div(max_qo, (int64_t)tw * kPrefillWaves), a.hkv, a.batch);
  const dim3 block(kPrefillWaves * 64);
  switch (G) {
    case 1: hipLaunchKernelGGL((paged_prefill_kernel<DT, 1>), grid, block, 0, stream, a); break;
    case 2: hipLaunchKernelGGL((paged_prefill_kernel<DT, 2>), grid, block, 0, stream, a); break;
    case 3: hipLaunchKernelGGL((paged_prefill_kernel<DT, 3>), grid, block, 0, stream, a); break;
    case 4: hipLaunchKernelGGL((paged_prefill_kernel<DT, 4>), grid, block, 0, stream, a); break;
    case 5: hipLaunchKernelGGL((paged_prefill_kernel<DT, 5>), grid, block, 0, stream, a); break;
    case 6: hipLaunchKernelGGL((paged_prefill_kernel<DT, 6>), grid, block, 0, stream, a); break;
    case 7: hipLaunchKernelGGL((paged_prefill_kernel<DT, 7>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((paged_prefill_kernel<DT, 8>), grid, block, 0, stream, a); break;
  }
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT int delta_paged_prefill(const void *q, int64_t q_stride_t, int64_t q_stride_h,
                                                const void *kv_cache, int64_t num_pages, const int32_t *qo_indptr,
                                                const int32_t *kv_indptr, const int32_t *kv_indices,
                                                int64_t kv_indices_len, const int32_t *kv_last_page_len, void *o,
                                                int64_t o_stride_t, int64_t o_stride_h, float *lse, int batch,
                                                int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
                                                float sm_scale, int max_qo_len, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_paged_prefill";
  if (batch <= 0 || max_qo_len <= 0) return DELTA_OK;
  if (head_dim != kHeadDim) return set_error(DELTA_ERR_INVALID, "%s: head_dim must be 128", who);
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads)
    return set_error(DELTA_ERR_INVALID, "%s: num_qo_heads must be a multiple of num_kv_heads", who);
  const int G = num_qo_heads / num_kv_heads;
  if (G > kMaxGroup) return set_error(DELTA_ERR_INVALID, "%s: group size %d > %d unsupported", who, G, kMaxGroup);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: bad dtype", who);
  if (!q || !kv_cache || !qo_indptr || !kv_indptr || !kv_indices || !kv_last_page_len || !o)
    return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (((uintptr_t)q | (uintptr_t)kv_cache) & 15u || (q_stride_t % 8) || (q_stride_h % 8))
    return set_error(DELTA_ERR_INVALID, "%s: q and kv_cache 16-byte aligned, q strides multiples of 8", who);
  if (num_pages <= 0 || kv_indices_len < 0) return set_error(DELTA_ERR_INVALID, "%s: empty cache", who);
  PrefillArgs a;
  a.q = (const uint16_t *)q;
  a.q_stride_t = q_stride_t;
  a.q_stride_h = q_stride_h;
  a.kv = (const uint16_t *)kv_cache;
  a.num_pages = num_pages;
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.kv_indices_len = kv_indices_len;
  a.last_page_len = kv_last_page_len;
  a.o = (uint16_t *)o;
  a.o_stride_t = o_stride_t;
  a.o_stride_h = o_stride_h;
  a.lse = lse;
  a.batch = batch;
  a.hq = num_qo_heads;
  a.hkv = num_kv_heads;
  a.sm_scale = sm_scale;
  if (dtype == DELTA_BF16)
    launch_prefill<DELTA_BF16>(a, G, max_qo_len, (hipStream_t)stream);
  else
    launch_prefill<DELTA_FP16>(a, G, max_qo_len, (hipStream_t)stream);
  return check_launch(who);
}
