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
// 32), with its q in registers.  The block sweeps the row's kv tokens 64 at a time (four pages,
// two 32-token sub-tiles) up to its last token's position: each step's K and V (16 KiB each for
// one head) are loaded once per block, 16 bytes per thread, into padded LDS tiles (three
// buffers; the next step in flight in registers) and read by every wave.  Waves 0-3 run each
// step whole; waves 4-7, the second wave of each SIMD, run half a step behind (P.V of the
// previous step, then S and softmax of this one, the previous step's V still in its buffer), so
// the two waves of a SIMD are not both in their softmax at once.  Per wave and sub-tile:
//   S^T = K Q^T : 8 v_mfma_f32_32x32x16 over d, A = the tile's K rows from LDS
//         (lane%32 = kv token, d in 16 ks + 8 (lane / 32) + [0, 8)), B = the wave's q (same d
//         split, n = lane%32 = query row); D leaves lane l with its row n = l%32 and the 16 kv
//         tokens m_i = 8 (i / 4) + 4 (l / 32) + i % 4;
//   softmax: online per row in the log2 domain over the step's 32 scores of the lane, one
//         exchange with lane l ^ 32 (the row's other half) for the maximum; the row sum stays
//         per half until the end.  The reference maximum moves only when a score passes it by
//         more than 8 (log2), so the accumulators are rescaled on few steps; causal and kv_len
//         masks only on steps that need them;
//   O^T += V^T P^T : 8 v_mfma_f32_32x32x16 (4 d tiles x 2 kv chunks), B = the lane's own P in
//         its D order (chunk c = values 8c..8c+7, i.e. kv tokens 16c + 4 (l/32) + {0..3, 8..11}),
//         packed by v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32, A = V^T read from the padded tile
//         with ds_read_b64_tr_b16 in that same kv order; lane l accumulates
//         O[row l%32][d = 32 dt + 8 (i / 4) + 4 (l / 32) + i % 4].
// LDS row pitches: K rows are read 16 bytes per lane, 32 rows at once (136 elements = 68 banks
// apart: each 16-lane group covers the 64 banks once); V is read transposed, 4 rows x 16
// columns per 16-lane group and two groups per pass (160 elements: consecutive rows 16 banks
// apart, so a pass covers 64 banks once; at 136 consecutive rows share 4 banks: 2-way conflicts).
// Blocks run heaviest first (the last query tiles attend the most tokens) and blockIdx.x is the
// kv head, so the blocks of one head land on the same XCD (blocks go to the XCDs round robin)
// and share its L2 for that head's K/V.  Page ids are preloaded 64 per register, with a bit
// mask of the invalid ones.  No merge.
#include "delta_common.h"

namespace delta {
namespace {

constexpr int kPW = 8;          // waves per block (each 32 query rows)
constexpr int kSub = 2;         // 32-token sub-tiles per step
constexpr int kKvStep = 32 * kSub;  // kv tokens per step
constexpr int kPgStep = kKvStep / 16;  // pages per step
constexpr int kRowP = 136;      // padded K tile row (elements): conflict-free 16-byte row reads
constexpr int kRowPV = 160;     // padded V tile row (elements), read transposed
constexpr int kBufs = 3;        // LDS step buffers (late waves read a step after the next barrier)

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

// Two floats -> two packed 16-bit values, round to nearest even (one v_cvt_pk_* on gfx950).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float x, float y);
template <>
__device__ __forceinline__ uint32_t pack2<DELTA_BF16>(float x, float y) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{x, y}), b2));
}
template <>
__device__ __forceinline__ uint32_t pack2<DELTA_FP16>(float x, float y) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{x, y}), h2));
}

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
  using MF = Mfma32<DT>;
  constexpr int TW = 32 / G;                  // query tokens per wave
  constexpr int BT = kPW * TW;                // query tokens per block
  constexpr int kTile = kKvStep * kRowP;      // the K tile (elements); the V tile follows
  constexpr int kTileV = kKvStep * kRowPV;
  // Two step buffers, each K then V (padded rows), shared by the block's waves.
  __shared__ uint16_t tiles[kBufs][kTile + kTileV];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hl = lane >> 5, n = lane & 31;
  const int h = blockIdx.x, b = blockIdx.z;
  const int64_t q0 = a.qo_indptr[b], q1 = a.qo_indptr[b + 1];
  const int qn = q1 > q0 ? (int)(q1 - q0) : 0;
  const int tile = (int)gridDim.y - 1 - (int)blockIdx.y;  // heaviest tiles first
  const int btok0 = tile * BT;
  if (btok0 >= qn) return;  // whole block
  // The wave's first query token, read as a scalar: the compiler cannot see that wave (from the
  // thread index) is uniform, and with tok0 scalar the wave's step count and its diagonal test
  // (full / masked step) become scalar branches (8192-token prompt 594 -> 569-585 us).
  const int tok0 = __builtin_amdgcn_readfirstlane(btok0 + wave * TW);

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
    // With a negative scale q's signs are flipped (S of -q is exactly -S; the scale below is then
    // positive).  The xor also makes the loads complete here, before the kv loop.
    const uint32_t flip = a.sm_scale < 0.f ? 0x80008000u : 0u;
    const uint16_t *qp = a.q + (q0 + tok0 + tt) * a.q_stride_t + (int64_t)(h * G + g) * a.q_stride_h + 8 * hl;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = ld128(qp + 16 * ks) ^ u32x4{flip, flip, flip, flip};
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
  const int64_t page_bytes = 2 * kPageSize * row_elems * 2;
  // Cooperative step load: 2 * kKvStep * 16 chunks of 16 bytes (K, then V; rows x 16 chunks) over
  // kPW * 64 threads.  Thread t stages chunk c16 = t % 16 of step rows t / 16 and t / 16 + 32 of
  // K and of V; the 64 lanes of a wave cover four rows of one page, so the page of each of its
  // loads is wave-uniform (page wave / 4 of the step for rows < 32, wave / 4 + 2 above): its id
  // and base address are scalars and the lanes' offsets are fixed for the whole sweep.
  constexpr int kChunks = 2 * kKvStep * (kHeadDim / 8);
  constexpr int kPer = kChunks / (kPW * 64);
  static_assert(kPer == 4 && kKvStep == 64 && kPW * 64 == 2 * kKvStep * 4, "staging layout");
  const int wq = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));  // wave / 4
  const int srow = (int)(threadIdx.x >> 4), c16 = (int)(threadIdx.x & 15);  // srow in [0, 32)
  const uint32_t goff_k = (uint32_t)(((srow & 15) * row_elems + (int64_t)h * kHeadDim + 8 * c16) * 2);
  const uint32_t goff_v = goff_k + (uint32_t)(kPageSize * row_elems * 2);
  int lds_off[kPer];  // elements: K rows srow, srow + 32, then the padded V rows
#pragma unroll
  for (int r = 0; r < kPer; ++r)
    lds_off[r] = (r < 2 ? (srow + 32 * r) * kRowP : kTile + (srow + 32 * (r - 2)) * kRowPV) + 8 * c16;

  // Page ids, 64 per register (lane i: page cbase + i), the next 64 a chunk ahead.
  const int npages = (nsteps * kKvStep + kPageSize - 1) / kPageSize;
  auto load_ids = [&](int base) -> int {
    const int it = base + lane;
    int pid = -1;
    if (it < npages && it < np) pid = a.kv_indices[p0 + it];
    return (pid >= 0 && (int64_t)pid < a.num_pages) ? pid : -1;
  };
  // Invalid page ids (negative or past the cache) of the current window, one bit per page.
  const int lim = npages < np ? npages : np;
  auto bad_of = [&](int id, int base) -> uint64_t { return __ballot(base + lane < lim && id < 0); };
  int cbase = 0;
  int ids = npages > 0 ? load_ids(0) : -1;
  int ids_next = npages > 64 ? load_ids(64) : -1;
  uint64_t bad = bad_of(ids, 0);
  auto id_of = [&](int pg) -> int {  // pg in [cbase, cbase + 128)
    return pg - cbase < 64 ? __builtin_amdgcn_readlane(ids, pg - cbase) : __builtin_amdgcn_readlane(ids_next, pg - cbase - 64);
  };
  u32x4 ring[kPer];  // K rows srow, srow + 32, V rows srow, srow + 32
  auto fetch = [&](int j) {  // global loads of step j into the ring
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int pg = kPgStep * j + wq + 2 * half;
      const int pid = pg < npages ? id_of(pg) : -1;
      if (pid >= 0) {
        const char *pb = reinterpret_cast<const char *>(a.kv) + (int64_t)pid * page_bytes;
        ring[half] = ld128(pb + goff_k);
        ring[2 + half] = ld128(pb + goff_v);
      } else {
        ring[half] = u32x4{0u, 0u, 0u, 0u};
        ring[2 + half] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto stage = [&](int j) {  // the ring (step j) into tiles[j % kBufs]; V rows past kv_len as zeros
    uint16_t *tb = &tiles[j % kBufs][0];
    const bool v_whole = (j + 1) * kKvStep <= kv_len;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      u32x4 v = ring[r];
      if (r >= 2 && !v_whole && j * kKvStep + srow + 32 * (r - 2) >= kv_len) v = u32x4{0u, 0u, 0u, 0u};
      st128(tb + lds_off[r], v);
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
  const float scale2 = fabsf(a.sm_scale) * kLog2e;
  // ds_read_b64_tr_b16 of V^T: 16-lane group q16 = lane / 16, t16 = lane % 16 reads rows
  // (kv) base + t16 / 4 at columns 16 (q16 % 2) + 4 (t16 % 4), and receives its column's four rows.
  const int q16 = lane >> 4, t16 = lane & 15;
  const int vtr_off = kTile + (4 * hl + (t16 >> 2)) * kRowPV + 16 * (q16 & 1) + 4 * (t16 & 3);

  // One step for the wave: S^T = K Q^T, the online softmax (accumulators rescaled when the
  // reference maximum moves) and P^T packed into pc.
  auto score_step = [&](int j, const uint16_t *tk, u32x4 (&pc)[2 * kSub]) {
    f32x16 S[kSub];
#pragma unroll
    for (int sb = 0; sb < kSub; ++sb)
#pragma unroll
      for (int i = 0; i < 16; ++i) S[sb][i] = 0.f;
    // K fragments two k-slices ahead of the MFMAs that use them (one ahead: 2048 tokens ~1 %
    // slower, same registers).
    auto kfrag = [&](int sb, int ks) { return *reinterpret_cast<const u32x4 *>(tk + (32 * sb + n) * kRowP + 16 * ks + 8 * hl); };
    u32x4 kq[3][kSub];  // fragments of k-slices ks, ks + 1, ks + 2
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int sb = 0; sb < kSub; ++sb) kq[s][sb] = kfrag(sb, s);
    // Raised wave priority over each MFMA run: of the SIMD's two waves, the one with MFMAs
    // to issue goes first, which pushes the other into its softmax meanwhile (~1 %).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      if (ks + 2 < 8) {
#pragma unroll
        for (int sb = 0; sb < kSub; ++sb) kq[(ks + 2) % 3][sb] = kfrag(sb, ks + 2);
      }
#pragma unroll
      for (int sb = 0; sb < kSub; ++sb) S[sb] = MF::run(kq[ks % 3][sb], qf[ks], S[sb]);
    }
    __builtin_amdgcn_s_setprio(0);
    // Masks only where the step crosses the wave's first diagonal, kv_len, or a bad page.
    const int kv0 = j * kKvStep;
    const int poff = kPgStep * j - cbase;  // the step's pages: bits poff .. poff + kPgStep - 1
    const bool pages_ok = ((bad >> poff) & ((1ull << kPgStep) - 1)) == 0;
    const bool full = kv0 + kKvStep - 1 <= wpos0 && kv0 + kKvStep <= kv_len && pages_ok;
    // Row maxima on the raw scores (the scale is positive, so it commutes with max), then
    // x = S * scale - m as one fma.  m is the row's reference maximum: it moves only when a
    // score exceeds it by more than 8 (a factor of 2^8), so the exponentials stay <= 256 and the
    // accumulators are rescaled only on those steps.
    constexpr int NX = 16 * kSub;
    float x[NX];
    float pm = -INFINITY;
    if (full) {
#pragma unroll
      for (int i = 0; i < NX; ++i) {
        x[i] = S[i >> 4][i & 15];
        pm = fmaxf(pm, x[i]);
      }
    } else {
      bool pg_ok[kPgStep];
#pragma unroll
      for (int p = 0; p < kPgStep; ++p) pg_ok[p] = ((bad >> (poff + p)) & 1ull) == 0;
#pragma unroll
      for (int i = 0; i < NX; ++i) {
        const int mm = 32 * (i >> 4) + 8 * ((i & 15) >> 2) + 4 * hl + (i & 3);
        const int tk_i = kv0 + mm;
        x[i] = (row_ok && pg_ok[mm >> 4] && tk_i <= qpos && tk_i < kv_len) ? S[i >> 4][i & 15] : -INFINITY;
        pm = fmaxf(pm, x[i]);
      }
    }
    const float smax = halves_max(pm) * scale2;
    float alpha = 1.f;
    if (smax > m + 8.f) {  // also the first finite score of the row (m = -inf)
      alpha = fast_exp2(m - smax);
      m = smax;
    }
    const float nm = m == -INFINITY ? 0.f : -m;
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      x[i] = fast_exp2(fmaf(x[i], scale2, nm));
      ps += x[i];
    }
    l = l * alpha + ps;  // this half's tokens; the halves are summed once at the end
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
    }
    // P^T chunks: values 8c .. 8c + 7 of this lane, rounded to the KV dtype.
#pragma unroll
    for (int cc = 0; cc < 2 * kSub; ++cc)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        pc[cc][w] = pack2<DT>(x[8 * cc + 2 * w], x[8 * cc + 2 * w + 1]);
  };
  // O^T += V^T P^T of a step whose P^T is in pc.
  auto pv_step = [&](const uint16_t *tk, const u32x4 (&pc)[2 * kSub]) {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int cc = 0; cc < 2 * kSub; ++cc) {
        const uint16_t *rd = tk + vtr_off + 16 * cc * kRowPV + 32 * dt;
        const ps4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ps4_t *)rd);
        const ps4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ps4_t *)(rd + 8 * kRowPV));
        u32x4 va;
        va[0] = (uint32_t)(uint16_t)v0[0] | ((uint32_t)(uint16_t)v0[1] << 16);
        va[1] = (uint32_t)(uint16_t)v0[2] | ((uint32_t)(uint16_t)v0[3] << 16);
        va[2] = (uint32_t)(uint16_t)v1[0] | ((uint32_t)(uint16_t)v1[1] << 16);
        va[3] = (uint32_t)(uint16_t)v1[2] | ((uint32_t)(uint16_t)v1[3] << 16);
        acc[dt] = MF::run(va, pc[cc], acc[dt]);
      }
    __builtin_amdgcn_s_setprio(0);
  };

  // Waves 0-3 (one per SIMD) run each step whole; waves 4-7, the SIMDs' second waves, run half
  // a step behind: P.V of the previous step first, then S and the softmax of this one.  So on
  // each SIMD one wave's softmax runs while the other wave's MFMAs do (P.V of one under the
  // other's softmax, S of one under the other's softmax), not both softmaxes at once.  A step's
  // tiles stay in LDS for one more step (three buffers): the late waves read step j - 1 after
  // the barrier of step j.
  const bool late = wave >= kPW / 2;
  u32x4 pcar[2 * kSub];
  for (int j = 0; j <= nsteps; ++j) {
    __syncthreads();  // step j is in tiles[j % 3]; tiles[(j + 1) % 3] is free
    if (j < nsteps && kPgStep * j >= cbase + 64) {  // the id window moves on
      cbase += 64;
      ids = ids_next;
      bad = bad_of(ids, cbase);
      ids_next = cbase + 64 < npages ? load_ids(cbase + 64) : -1;
    }
    if (late) {
      if (j >= 1 && j - 1 < wsteps) pv_step(&tiles[(j - 1) % kBufs][0], pcar);
      if (j < wsteps) score_step(j, &tiles[j % kBufs][0], pcar);
    } else if (j < wsteps) {
      u32x4 pc[2 * kSub];
      score_step(j, &tiles[j % kBufs][0], pc);
      pv_step(&tiles[j % kBufs][0], pc);
    }
    if (j + 1 < nsteps) {
      stage(j + 1);
      if (j + 2 < nsteps) fetch(j + 2);
    }
  }

  // Normalise and write: lane l holds O[row l%32][32 dt + 8 (i / 4) + 4 hl + i % 4].
  l = halves_sum(l);
  if (row_ok) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t *op = a.o + (q0 + tok0 + tt) * a.o_stride_t + (int64_t)(h * G + g) * a.o_stride_h + 4 * hl;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        uint2 w;
        w.x = pack2<DT>(acc[dt][4 * q4] * inv, acc[dt][4 * q4 + 1] * inv);
        w.y = pack2<DT>(acc[dt][4 * q4 + 2] * inv, acc[dt][4 * q4 + 3] * inv);
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
