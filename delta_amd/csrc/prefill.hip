// Causal paged prefill attention for gfx950 (several query tokens per row, GQA).
//
// Replaces FlashInfer's BatchPrefillWithPagedKVCacheWrapper.run with causal=True for rows
// with qo_len > 1 (hoenza/DELTA backend.py:1091-1105, the prompt steps of the engine).  The
// cache already holds the row's new tokens (update_kv runs before attention, model.py:413-418),
// so query i of row b sits at position kv_len_b - qo_len_b + i and attends tokens 0..position.
//
// Work decomposition (flash-attention style, on 32x32 MFMA tiles): a block is kPW waves of one
// (row, kv head) and a run of consecutive query tokens; each wave owns 32 query rows, the
// (token, q head) pairs of TW = 32 / G tokens (rows past TW * G idle when G does not divide
// 32), with its q in registers.  The block sweeps the row's kv tokens 32 at a time (two pages)
// up to its last token's position: each step's K and V (8 KiB each for one head) are loaded
// once per block, 16 bytes per thread, into double-buffered padded LDS tiles (the next step in
// flight in registers) and read by every wave.  Per wave and step:
//   S^T = K Q^T : 8 v_mfma_f32_32x32x16 over d, A = the tile's K rows from LDS
//         (lane%32 = kv token, d in 16 ks + 8 (lane / 32) + [0, 8)), B = the wave's q (same d
//         split, n = lane%32 = query row); D leaves lane l with its row n = l%32 and the 16 kv
//         tokens m_i = 8 (i / 4) + 4 (l / 32) + i % 4;
//   softmax: online per row in the log2 domain, lane-local but for one exchange with lane
//         l ^ 32 (the row's other 16 tokens); causal and kv_len masks only on tiles that need
//         them;
//   O^T += V^T P^T : 8 v_mfma_f32_32x32x16 (4 d tiles x 2 kv chunks), B = the lane's own P in
//         its D order (chunk c = values 8c..8c+7, i.e. kv tokens 16c + 4 (l/32) + {0..3, 8..11}),
//         A = V^T read from the padded tile with ds_read_b64_tr_b16 in that same kv order;
//         lane l accumulates O[row l%32][d = 32 dt + 8 (i / 4) + 4 (l / 32) + i % 4].
// Blocks run heaviest first (the last query tiles attend the most tokens) and blockIdx.x is the
// kv head, so the blocks of one head land on the same XCD (blocks go to the XCDs round robin)
// and share its L2 for that head's K/V.  Page ids are preloaded 64 per register.  No merge.
#include "delta_common.h"

namespace delta {
namespace {

constexpr int kPW = 8;          // waves per block (each 32 query rows)
constexpr int kKvStep = 32;     // kv tokens per step (two pages)
constexpr int kRowP = 136;      // padded LDS tile row (elements): conflict-free 16-byte row reads

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

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short ps4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ps4_t lds_ps4_t;

template <int DT>
struct Mfma32;
template <>
struct Mfma32<DELTA_BF16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma32<DELTA_FP16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};

// max / sum of a value and its copy in lane l ^ 32
__device__ __forceinline__ float halves_max(float v) {
  auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
}
__device__ __forceinline__ float halves_sum(float v) {
  auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(x[0]) + __uint_as_float(x[1]);
}

template <int DT, int G>
__global__ void __launch_bounds__(kPW * 64) paged_prefill_kernel(PrefillArgs a) {
#pragma clang fp contract(off)
  using E = Elem<DT>;
  using MF = Mfma32<DT>;
  constexpr int TW = 32 / G;                  // query tokens per wave
  constexpr int BT = kPW * TW;                // query tokens per block
  constexpr int kTile = kKvStep * kRowP;      // one K or V tile (elements)
  // Two step buffers, each K then V (padded rows), shared by the block's waves.
  __shared__ uint16_t tiles[2][2 * kTile];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hl = lane >> 5, n = lane & 31;
  const int h = blockIdx.x, b = blockIdx.z;
  const int64_t q0 = a.qo_indptr[b], q1 = a.qo_indptr[b + 1];
  const int qn = q1 > q0 ? (int)(q1 - q0) : 0;
  const int tile = (int)gridDim.y - 1 - (int)blockIdx.y;  // heaviest tiles first
  const int btok0 = tile * BT;
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

  // This lane's query row n = (token tt, head g).
  const int tt = n / G, g = n % G;
  const bool row_ok = n < TW * G && tok0 + tt < qn;
  const int qpos = kv_len - qn + tok0 + tt;  // attends tokens 0..qpos
  u32x4 qf[8];  // B operand of S^T = K Q^T: d = 16 ks + 8 hl + [0, 8)
  if (row_ok) {
    const uint16_t *qp = a.q + (q0 + tok0 + tt) * a.q_stride_t + (int64_t)(h * G + g) * a.q_stride_h + 8 * hl;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = ld128(qp + 16 * ks);
  } else {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = u32x4{0u, 0u, 0u, 0u};
  }

  // Steps the block sweeps (up to its last token's position) and the ones this wave needs.
  auto steps_upto = [&](int last_tok) {
    const int pos = kv_len - qn + last_tok;
    const int nt = pos >= 0 ? pos / kKvStep + 1 : 0;
    const int cap = (kv_len + kKvStep - 1) / kKvStep;
    return nt > cap ? cap : nt;
  };
  const int nsteps = steps_upto((btok0 + BT < qn ? btok0 + BT : qn) - 1);
  const int wsteps = tok0 < qn ? steps_upto((tok0 + TW < qn ? tok0 + TW : qn) - 1) : 0;
  // First query position of the wave: steps ending at or below it need no causal mask.
  const int wpos0 = kv_len - qn + tok0;

  const int64_t row_elems = (int64_t)a.hkv * kHeadDim;
  const int64_t page_elems = 2 * kPageSize * row_elems;
  // Cooperative step load: 1024 16-byte chunks (K, then V; 32 rows x 16 chunks), kPW*64 threads.
  constexpr int kChunks = 2 * kKvStep * (kHeadDim / 8);
  constexpr int kPer = kChunks / (kPW * 64);

  // Page ids, 64 per register (lane i: page cbase + i), the next 64 a chunk ahead.
  const int npages = (nsteps * kKvStep + kPageSize - 1) / kPageSize;
  auto load_ids = [&](int base) -> int {
    const int it = base + lane;
    int pid = -1;
    if (it < npages && it < np) pid = a.kv_indices[p0 + it];
    return (pid >= 0 && (int64_t)pid < a.num_pages) ? pid : -1;
  };
  int cbase = 0;
  int ids = npages > 0 ? load_ids(0) : -1;
  int ids_next = npages > 64 ? load_ids(64) : -1;
  auto id_of = [&](int pg) -> int {  // pg in [cbase, cbase + 128)
    return pg - cbase < 64 ? __builtin_amdgcn_readlane(ids, pg - cbase) : __builtin_amdgcn_readlane(ids_next, pg - cbase - 64);
  };
  u32x4 ring[kPer];
  auto fetch = [&](int j) {  // global loads of step j into the ring
    const int pa = 2 * j < npages ? id_of(2 * j) : -1, pb = 2 * j + 1 < npages ? id_of(2 * j + 1) : -1;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int ci = threadIdx.x + r * kPW * 64;
      const int which = ci >> 9, row = (ci >> 4) & 31, c16 = ci & 15;
      const int pid = (row >> 4) ? pb : pa;
      ring[r] = pid >= 0 ? ld128(a.kv + (int64_t)pid * page_elems + (int64_t)(which * kPageSize + (row & 15)) * row_elems +
                                 (int64_t)h * kHeadDim + 8 * c16)
                         : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto stage = [&](int j) {  // the ring (step j) into tiles[j & 1]; V rows past kv_len as zeros
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int ci = threadIdx.x + r * kPW * 64;
      const int which = ci >> 9, row = (ci >> 4) & 31, c16 = ci & 15;
      const bool keep = which == 0 || j * kKvStep + row < kv_len;
      st128(&tiles[j & 1][which * kTile + row * kRowP + 8 * c16], keep ? ring[r] : u32x4{0u, 0u, 0u, 0u});
    }
  };
  if (nsteps > 0) {
    fetch(0);
    stage(0);
    if (nsteps > 1) fetch(1);
  }

  float m = -INFINITY, l = 0.f;
  f32x16 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;
  const float scale2 = a.sm_scale * kLog2e;
  // ds_read_b64_tr_b16 of V^T: 16-lane group q16 = lane / 16, t16 = lane % 16 reads rows
  // (kv) base + t16 / 4 at columns 16 (q16 % 2) + 4 (t16 % 4), and receives its column's four rows.
  const int q16 = lane >> 4, t16 = lane & 15;
  const int vtr_off = kTile + (4 * hl + (t16 >> 2)) * kRowP + 16 * (q16 & 1) + 4 * (t16 & 3);

  for (int j = 0; j < nsteps; ++j) {
    __syncthreads();  // step j is in tiles[j & 1]; tiles[(j + 1) & 1] is free
    if (2 * j >= cbase + 64) {  // the id window moves on (steps cover two pages)
      cbase += 64;
      ids = ids_next;
      ids_next = cbase + 64 < npages ? load_ids(cbase + 64) : -1;
    }
    if (j < wsteps) {
      const uint16_t *tk = &tiles[j & 1][0];
      f32x16 S;
#pragma unroll
      for (int i = 0; i < 16; ++i) S[i] = 0.f;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
        S = MF::run(*reinterpret_cast<const u32x4 *>(tk + n * kRowP + 16 * ks + 8 * hl), qf[ks], S);
      // Masks only where the step crosses the wave's first diagonal, kv_len, or a bad page.
      const int kv0 = j * kKvStep;
      const bool pages_ok = id_of(2 * j) >= 0 && (2 * j + 1 >= np || id_of(2 * j + 1) >= 0);
      const bool full = kv0 + kKvStep - 1 <= wpos0 && kv0 + kKvStep <= kv_len && pages_ok;
      float x[16];
      float pm = -INFINITY;
      if (full) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          x[i] = S[i] * scale2;
          pm = fmaxf(pm, x[i]);
        }
      } else {
        const bool pa_ok = id_of(2 * j) >= 0, pb_ok = 2 * j + 1 < np && id_of(2 * j + 1) >= 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int mm = 8 * (i >> 2) + 4 * hl + (i & 3);
          const int tk_i = kv0 + mm;
          const bool pg = mm < 16 ? pa_ok : pb_ok;
          x[i] = (row_ok && pg && tk_i <= qpos && tk_i < kv_len) ? S[i] * scale2 : -INFINITY;
          pm = fmaxf(pm, x[i]);
        }
      }
      const float mn = fmaxf(m, halves_max(pm));
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float alpha = fast_exp2(m - mref);
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        x[i] = fast_exp2(x[i] - mref);
        ps += x[i];
      }
      l = l * alpha + halves_sum(ps);
      m = mn;
      if (__ballot(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
      }
      // P^T chunks: values 8c .. 8c + 7 of this lane, rounded to the KV dtype.
      u32x4 pc[2];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int w = 0; w < 4; ++w)
          pc[cc][w] = E::from_float(x[8 * cc + 2 * w]) | (E::from_float(x[8 * cc + 2 * w + 1]) << 16);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          const uint16_t *rd = tk + vtr_off + 16 * cc * kRowP + 32 * dt;
          const ps4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ps4_t *)rd);
          const ps4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ps4_t *)(rd + 8 * kRowP));
          u32x4 va;
          va[0] = (uint32_t)(uint16_t)v0[0] | ((uint32_t)(uint16_t)v0[1] << 16);
          va[1] = (uint32_t)(uint16_t)v0[2] | ((uint32_t)(uint16_t)v0[3] << 16);
          va[2] = (uint32_t)(uint16_t)v1[0] | ((uint32_t)(uint16_t)v1[1] << 16);
          va[3] = (uint32_t)(uint16_t)v1[2] | ((uint32_t)(uint16_t)v1[3] << 16);
          acc[dt] = MF::run(va, pc[cc], acc[dt]);
        }
    }
    if (j + 1 < nsteps) {
      stage(j + 1);
      if (j + 2 < nsteps) fetch(j + 2);
    }
  }

  // Normalise and write: lane l holds O[row l%32][32 dt + 8 (i / 4) + 4 hl + i % 4].
  if (row_ok) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t *op = a.o + (q0 + tok0 + tt) * a.o_stride_t + (int64_t)(h * G + g) * a.o_stride_h + 4 * hl;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        uint2 w;
        w.x = E::from_float(acc[dt][4 * q4] * inv) | (E::from_float(acc[dt][4 * q4 + 1] * inv) << 16);
        w.y = E::from_float(acc[dt][4 * q4 + 2] * inv) | (E::from_float(acc[dt][4 * q4 + 3] * inv) << 16);
        *reinterpret_cast<uint2 *>(op + 32 * dt + 8 * q4) = w;
      }
    if (a.lse && hl == 0) a.lse[(q0 + tok0 + tt) * a.hq + h * G + g] = l > 0.f ? (m + log2f(l)) * kLn2 : -INFINITY;
  }
}

template <int DT>
void launch_prefill(const PrefillArgs &a, int G, int max_qo, hipStream_t stream) {
  const int tw = 32 / G;
  const dim3 grid(a.hkv, (unsigned)ceil_div(max_qo, (int64_t)tw * kPW), a.batch);
  const dim3 block(kPW * 64);
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
  if (((uintptr_t)o & 7u) || (o_stride_t % 4) || (o_stride_h % 4))
    return set_error(DELTA_ERR_INVALID, "%s: o 8-byte aligned with strides in multiples of 4", who);
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
