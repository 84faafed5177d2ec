// Paged decode attention for gfx950 (one query token per row, GQA).
//
// Replaces FlashInfer's paged attention run with qo_len = 1
// (hoenza/DELTA backend.py:461-512, plan at 1091-1105) and the planner layer's
// BatchDumpAttentionWeights logits side-write (backend.py:175-222, 518-585).
//
// Work decomposition
//   block = 16 waves = hb kv heads x R waves each.
//   Page-major (hb = Hkv), grid = (batch * num_splits): a block takes one work unit, a chunk
//   of up to `chunk` pages of one row; a row has clamp(ceil(pages / chunk), 1, num_splits)
//   units and the units are packed row by row at the front of the grid, so ragged rows cost
//   blocks in proportion to their pages (blocks past the last unit exit at once).  Wave w
//   works on kv head w % Hkv and takes every R-th page of the unit, so the Hkv waves of one
//   page slot read all heads of the same page (its K and V are each one contiguous
//   16 * Hkv * 256-byte run).  Head-major (hb = 1), grid = (Hkv, batch): the waves of a
//   (row, kv head) block take its pages round robin, with no split; small batches split
//   head-major blocks too, grid = (batch * num_splits, Hkv), block x = unit (row x / num_splits,
//   split x % num_splits), no packing.  The choice per shape is decode_plan's.
//   Per page and wave (details at decode_split_body): q.K and P.V on MFMA, online
//   softmax in the log2 domain; page ids preloaded 64 per register, the next page's
//   K and V always in flight.
//   The block's waves merge in LDS per head; with num_splits > 1 the block writes an
//   un-normalised partial (acc, m, l) and a merge kernel combines the splits.
//   The ROPE instantiations (decode steps) also rotate q, rotate and append the row's new
//   token to the cache, and take that token's K / V from LDS (mylib::rope and
//   mylib::update_kv of Attention.forward, model.py:413-418, in the same launch).
//
// HBM bytes per launch (algorithmic): K and V of every attended token once,
// q and o once, the page indices once (+ the fp32 logits when dumping).
#include <atomic>
#include <mutex>
#include <type_traits>

#include "delta_common.h"

namespace delta {

namespace {

constexpr int kMaxWaves = 16;  // waves per block (a block never exceeds one CU's 16 slots at <= 128 VGPRs)
constexpr int kHeadMajorWaves = 4;  // waves per block of an unsplit head-major launch (decode_plan)
constexpr int kMergeGroups = 4;     // 128-thread groups of a merge block (16 splits each per round)

// Groups of a merge block for `nsplit` splits: one per 16 splits, at most kMergeGroups.
inline int merge_groups(int nsplit) {
  const int n = (nsplit + 15) / 16;
  return n < 1 ? 1 : (n > kMergeGroups ? kMergeGroups : n);
}

struct DecodeArgs {
  const uint16_t *q;
  int64_t q_stride_b, q_stride_h;
  const uint16_t *kv;
  int64_t num_pages;
  const int32_t *kv_indptr;
  const int32_t *kv_indices;
  int64_t kv_indices_len;
  const int32_t *last_page_len;
  uint16_t *o;
  int64_t o_stride_b, o_stride_h;
  float *lse;
  float *dump;
  int64_t dump_stride_b, dump_stride_h;
  int dump_pages;   // pages per dump row the caller guarantees (max_pages_per_row)
  float *part_acc;  // [row][split][hkv][G][128]   (split < nsplit; a row's units_of splits hold data)
  float *part_ml;   // [row][split][hkv][G][2]     (m in log2 units, l)
  int batch, hq, hkv, nsplit;
  int chunk;        // pages per work unit (split launches)
  int hb;           // kv heads per block (hkv: page-major, 1: head-major)
  int direct;       // split launch whose block x is unit (row x / nsplit, split x % nsplit)
  int bal_w;        // unsplit head-major launch over more (row, kv head) blocks than CUs: rows per
                    // round of the balanced row order (balanced_row); 0 = block y takes row y
  float sm_scale;
  // Decode steps with the new token's RoPE and KV append fused in (the *_append entry
  // points): q is the un-rotated query, row b's new token (k_new, v_new rows b) sits at
  // kv_len_b - 1 of the append CSR (ap_indptr / ap_indices, sharing last_page_len).
  uint16_t *kv_w;   // the cache, writable
  const uint16_t *k_new;
  int64_t k_new_stride;
  const uint16_t *v_new;
  int64_t v_new_stride;
  const int32_t *offsets;  // [batch] the new token's position (rotation angle)
  const int32_t *ap_indptr;
  const int32_t *ap_indices;
  int64_t ap_indices_len;
  float rcp_scale, log2_theta, smooth_a, smooth_b;
  // K-only scorer with the row's logits kept in LDS (TOKMAX): per (row, kv head, token) the
  // largest softmax probability over the head's G q heads, [batch][hkv][tokmax_stride_h].
  float *tokmax;
  int64_t tokmax_stride_b, tokmax_stride_h;
};

struct RowInfo {
  int64_t p0;
  int np;
  int kv_len;
  int last;  // last_page_len clamped to [0, 16]
};

__device__ __forceinline__ RowInfo row_info(const DecodeArgs &a, int b) {
  const int64_t ilen = a.kv_indices_len;
  int64_t p0 = a.kv_indptr[b];
  int64_t p1 = a.kv_indptr[b + 1];
  p0 = p0 < 0 ? 0 : (p0 > ilen ? ilen : p0);
  p1 = p1 < p0 ? p0 : (p1 > ilen ? ilen : p1);
  int last = a.last_page_len[b];
  last = last < 0 ? 0 : (last > kPageSize ? kPageSize : last);
  RowInfo r;
  r.p0 = p0;
  r.np = (int)(p1 - p0);
  r.kv_len = r.np > 0 ? (r.np - 1) * kPageSize + last : 0;
  r.last = last;
  return r;
}

// LDS row of a staged V tile: 128 elements + 8 padding (272 B), so the 16 rows of a
// transposed read start on distinct 4-bank offsets.
constexpr int kVStride = 136;
constexpr int kVTile = kPageSize * kVStride;  // elements per wave

// V rows a lane loads in the register-held P.V path (the planner with on-chip logits): lane
// group c = lane / 16 holds the tokens of its P.V k slots, tok = 2c + v_row(i), i = 0..3.
__device__ __forceinline__ constexpr int v_row(int i) { return 8 * (i >> 1) + (i & 1); }

template <int DT>
struct Mfma16;
template <>
struct Mfma16<DELTA_BF16> {
  typedef short s4 __attribute__((ext_vector_type(4)));
  __device__ __forceinline__ static f32x4 run(s4 a, s4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static short pack(float x) { return __builtin_bit_cast(short, (__bf16)x); }
};
template <>
struct Mfma16<DELTA_FP16> {
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  __device__ __forceinline__ static f32x4 run(s4 a, s4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static short pack(float x) { return __builtin_bit_cast(short, (_Float16)x); }
};

typedef short s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4_t lds_s4_t;

// Work units of a split launch: row b has units_of(b) = clamp(ceil(pages_b / chunk), 1,
// nsplit) of them (its last unit takes any pages past units * chunk, so a row longer than the
// planned maximum is still covered), numbered row by row.
__device__ __forceinline__ int units_of(const DecodeArgs &a, int b) {
  const RowInfo r = row_info(a, b);
  const int n = (r.np + a.chunk - 1) / a.chunk;
  return n < 1 ? 1 : (n > a.nsplit ? a.nsplit : n);
}

// Row of block y of an unsplit head-major launch whose (row, kv head) blocks outnumber the CUs.
// Blocks are dealt to XCDs round robin and each XCD's blocks to its CUs in order, so the blocks
// of rows y, y + bal_w, y + 2 bal_w, ... (bal_w = CUs / Hkv) share CUs and a CU's time is the
// sum of its rows' pages.  Ragged rows are therefore ranked by page count (descending, ties by
// row) and dealt in rounds of bal_w, every other round reversed, so each CU's rows sum to about
// the same.  Config-5 shape (128 rows of 32-256 pages, Hkv = 8): 221.6 us as given, 187.0 us in
// this order, 184.8 us with all rows equal.  Every block ranks all rows itself (B <= 512) on one
// key per row, (pages << 9) | (511 - row), and keeps every row's bounds in LDS, so the chosen
// row's come from there.  `lds` holds 5 B + 1 ints; the block's waves leave in step, so the LDS
// is free afterwards.  Returns the row; *ri gets its bounds.
__device__ int balanced_row(const DecodeArgs &a, int y, int *lds, RowInfo *ri) {
  const int B = a.batch;
  int64_t *p0 = reinterpret_cast<int64_t *>(lds);  // [B] (the dynamic LDS starts 16-byte aligned)
  int *key = lds + 2 * B;                          // [B]
  int *np = lds + 3 * B;                           // [B]
  int *last = lds + 4 * B;                         // [B]
  int *win = lds + 5 * B;
  if (threadIdx.x == 0) *win = y;  // replaced by the ranking below (kept in range regardless)
  for (int r = threadIdx.x; r < B; r += blockDim.x) {
    const RowInfo x = row_info(a, r);
    // Distinct keys (the row in the low bits); page counts past 2^21 - 1 rank as equal.
    key[r] = ((x.np < (1 << 21) ? x.np : (1 << 21) - 1) << 9) | (511 - r);
    np[r] = x.np;
    last[r] = x.last;
    p0[r] = x.p0;
  }
  __syncthreads();
  const int W = a.bal_w;
  const int rnd = y / W;
  const int i = y - rnd * W;
  const int n_r = B - rnd * W < W ? B - rnd * W : W;
  const int want = rnd * W + ((rnd & 1) ? n_r - 1 - i : i);
  for (int r = threadIdx.x; r < B; r += blockDim.x) {
    const int kr = key[r];
    int rank = 0;
    for (int u = 0; u < B; ++u) rank += key[u] > kr ? 1 : 0;
    if (rank == want) *win = r;  // the keys are distinct: exactly one row matches
  }
  __syncthreads();
  int b = uniform(*win);
  b = b < 0 ? 0 : (b >= B ? B - 1 : b);
  RowInfo x;
  x.p0 = p0[b];
  x.np = np[b];
  x.last = last[b];
  x.kv_len = x.np > 0 ? (x.np - 1) * kPageSize + x.last : 0;
  *ri = x;
  __syncthreads();
  return b;
}

// Row, split and unit count of unit u (every wave of the block computes the same answer).
// Units run in two groups: first every row's full units (all but its last, `chunk` pages each),
// numbered row by row, then each row's last unit (at most `chunk` pages unless the row outgrew
// the plan), row b at F + b, F = the number of full units.  Blocks start in grid order, so the
// short last units of a ragged batch fill the launch's tail instead of whole units of the last
// rows.  A running inclusive scan over 64 rows at a time; false past the last unit.
__device__ __forceinline__ bool find_unit(const DecodeArgs &a, int u, int lane, int *row, int *split, int *nu) {
  int base = 0;
  for (int r0 = 0; r0 < a.batch; r0 += 64) {
    const int r = r0 + lane;
    const int n = r < a.batch ? units_of(a, r) - 1 : 0;  // full units of row r
    int incl = n;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off, 64);
      if (lane >= off) incl += v;
    }
    const int total = __shfl(incl, 63, 64);
    if (u < base + total) {
      const uint64_t m = __ballot(base + incl > u);
      const int l = __builtin_ctzll(m);
      const int start = base + __shfl(incl - n, l, 64);
      *row = r0 + l;
      *split = u - start;
      *nu = __shfl(n, l, 64) + 1;
      return true;
    }
    base += total;
  }
  const int b = u - base;  // the last units, one per row
  if (b >= a.batch) return false;
  *row = b;
  *nu = units_of(a, b);
  *split = *nu - 1;
  return true;
}

// Pages of logits a wave stages in LDS before writing them out.  Interleaving the dump's HBM
// writes with the K/V read stream costs far more than their bandwidth share, so the scorer
// (no V tiles in LDS) stages 32 / 16 pages -- a whole split at the usual launch shapes, one
// write burst at the end; the planner (V tiles beside) stages 16 / 8.
template <int G, bool WITH_V>
constexpr int dump_slots() {
  return WITH_V ? (G <= 4 ? 16 : 8) : (G <= 4 ? 32 : 16);
}

// TOKMAX LDS: the waves' (m, l) [16][G][2], 16 floats of per-head lse2, then the logits
// [dump_pages][G][16] (with V, at least 128 pages' worth: the waves' accumulators
// [16][G][128] reuse that space once the logits are consumed), then (ROPE) the token slots.
template <int G>
constexpr int tokmax_lds_header() {
  return kMaxWaves * G * 2 + 16;
}
template <int G, bool WITH_V>
__host__ __device__ inline int64_t tokmax_logit_floats(int dump_pages) {
  constexpr int kAccPages = kMaxWaves * kHeadDim / kPageSize;
  const int64_t pages = (WITH_V && dump_pages < kAccPages) ? kAccPages : dump_pages;
  return pages * G * kPageSize;
}

// The fused append's per-wave token slots (ROPE), in floats from the start of the dynamic LDS:
// past the V tiles and the merge area (attention launches) or past the larger of the merge
// area and the V tiles plus the dump staging (planner launches).
template <int G, bool WITH_V, bool WITH_DUMP>
__host__ __device__ constexpr int rope_lds_offset(int nw) {
  return WITH_DUMP ? (nw * G * (2 + kHeadDim) > nw * kVTile / 2 + nw * dump_slots<G, WITH_V>() * G * kPageSize
                          ? nw * G * (2 + kHeadDim)
                          : nw * kVTile / 2 + nw * dump_slots<G, WITH_V>() * G * kPageSize)
                   : nw * kVTile / 2 + nw * G * (2 + kHeadDim);
}

// max / sum over the four 16-lane rows (lanes l, l^16, l^32, l^48) with the gfx950 permlane swaps.
__device__ __forceinline__ float rows4_max(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows4_sum(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// One (row, split, group of hb kv heads) per block; R = blockDim/64/hb waves per head take the
// split's pages round robin.
//   q.K : v_mfma_f32_16x16x32, one per (8-token half f, 64-d half sp) of the page.  A row
//         i = 2u + e is token 8f + u restricted to d in 64 sp + 32 e + [0, 32): lane (c, t)
//         loads K[8f + t/2][64 sp + 32 (t%2) + 8c, +8), so one load instruction covers 8 token
//         rows x 128 contiguous bytes (whole cache lines; a 16-row x 64-byte pattern costs
//         ~10% of HBM bandwidth).  B column g < 8 holds q_g[64 sp + 8c, +8) and column 8 + g
//         holds q_g[64 sp + 32 + 8c, +8), so D[2u][g] + D[2u + 1][8 + g] = q_g . K[8f + u]
//         over the 64 d of sp: one DPP row rotate by 8 joins the two halves.  Lane (c, g)
//         ends with tokens tok(r) = 8 (r/2) + 2c + r%2, r = 0..3, of head g.
//   softmax: per lane 4 tokens of one head; row reductions are 3 in-lane ops + 2 permlane swaps.
//   P.V : v_mfma_f32_16x16x16 -- A = P (row g = lane%16, k = 4c + r <-> token tok(r)),
//         B = V from a padded LDS tile whose row 4c + r holds token tok(r), read with
//         ds_read_b64_tr_b16 (lane (c, j) gets tile rows 4c..4c+3 at d = 16n + j),
//         D = O[g = 4c + r][d = 16n + lane%16].
// TOKMAX (head-major, unsplit, the row's logits fit in LDS): every page's logits stay in LDS
// ([page][g][16], past a small merge header); once the block's waves have merged, the block
// knows each head's final lse and writes, per token, max_g 2^(x_g log2 e - lse2_g) --
// del3_legacy_softmax's per-token max over this kv head's q heads -- instead of a logits dump.
// Without V it is the K-only scorer; with V (the planner) P.V takes V from registers instead
// of LDS tiles, which leaves the LDS to the logits: lane (c, j) loads V[tok(i)][8j, 8j + 8)
// for its four k slots and MFMA n takes element n of each (two v_perm_b32), so
// D = O[g = 4c + r][d = 8 lane%16 + n].
// Store of a split partial.  AGENT (the subset launches): agent-scope (sc1) stores, which
// measured 2-3 % faster on the small split subset launches at configs 2 and 4 (15.9 -> 15.6 and
// 12.6 -> 12.2 us with their merge launch, interleaved A/B) but slower on the larger split
// full-attention launches (config 4 88.1 -> 90.9 us), which keep plain stores.
template <bool AGENT>
__device__ __forceinline__ void part_store(float *p, float v) {
  if constexpr (AGENT)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *p = v;
}

template <int DT, int G, bool WITH_V, bool WITH_DUMP, bool ROPE, bool TOKMAX = false, bool AGENT_PARTS = false>
__device__ __forceinline__ void decode_split_body(const DecodeArgs &a, float *smem) {
  // No FMA contraction: every instantiation (with or without the dump) rounds the softmax
  // arguments identically, so P -- rounded to the KV dtype for the P.V MFMA -- is the same.
#pragma clang fp contract(off)
  static_assert(!TOKMAX || (!WITH_DUMP && (WITH_V || !ROPE)), "TOKMAX: the K-only scorer or the on-chip planner");
  constexpr bool REGV = TOKMAX && WITH_V;  // P.V with V in registers (no V tiles)
  using E = Elem<DT>;
  using M16 = Mfma16<DT>;

  const int nw = blockDim.x >> 6;
  const int hb = a.hb;
  const int R = nw / hb;  // waves per kv head
  // Head group: blockIdx.y of a split launch (blockIdx.x = work unit), blockIdx.x otherwise.
  const int head0 = (a.nsplit > 1 ? (int)blockIdx.y : (int)blockIdx.x) * hb;
  const int wave = uniform(threadIdx.x >> 6);
  const int h = head0 + wave % hb;
  const int rslot = wave / hb;
  const int lane = threadIdx.x & 63;
  const int c = lane >> 4;
  const int t = lane & 15;

  int b, split = 0, j0 = 0, j1;
  RowInfo ri;
  const int unit = blockIdx.x;
  if (a.nsplit > 1) {
    int nu;
    if (a.direct) {
      // Every row owns nsplit block slots: the row is known from the block index, so its bounds,
      // q and page ids load with no scan before them; slots past the row's units exit.
      b = uniform(unit / a.nsplit);
      split = uniform(unit - b * a.nsplit);
      ri = row_info(a, b);
      nu = (ri.np + a.chunk - 1) / a.chunk;
      nu = nu < 1 ? 1 : (nu > a.nsplit ? a.nsplit : nu);
      if (split >= nu) return;  // whole block
    } else {
      if (!find_unit(a, unit, lane, &b, &split, &nu)) return;  // past the last unit: whole block
      ri = row_info(a, b);
    }
    j0 = split * a.chunk;
    j1 = split == nu - 1 ? ri.np : min(ri.np, j0 + a.chunk);
  } else {
    if (a.bal_w > 0) {
      b = balanced_row(a, blockIdx.y, reinterpret_cast<int *>(smem), &ri);
    } else {
      b = blockIdx.y;
      ri = row_info(a, b);
    }
    j1 = ri.np;
  }
  // A split launch's partial slot (row, split), and whether this is the row's first split;
  // both wave-uniform, so kept in scalar registers across the page loop.
  const int pslot = uniform(b * a.nsplit + split);
  const bool split0 = uniform(split) == 0;
  // (ROPE) The append CSR's row bounds, requested with the row's own bounds: the slot's page
  // id below then needs no round trip of its own before the page stream starts.  Scalar loads:
  // their waits (lgkmcnt) never wait for page data, as a pending vector load before the page
  // loop would make each page's test against the slot wait for all of its K and V.
  int64_t ap_q0 = 0, ap_q1 = 0;
  if (ROPE) {
    const int bu = uniform(b);
    ap_q0 = ld_scalar(a.ap_indptr, bu);
    ap_q1 = ld_scalar(a.ap_indptr, bu + 1);
  }

  // Query fragments (B operand of q.K) for the two 64-d halves sp: column t holds head t % 8
  // at d = 64 sp + 32 (t / 8) + 8c + [0, 8); zero for heads past the group.
  u32x4 qf[2];
  if ((t & 7) < G) {
    const uint16_t *qp = a.q + (int64_t)b * a.q_stride_b + (int64_t)(h * G + (t & 7)) * a.q_stride_h +
                         32 * (t >> 3) + 8 * c;
    qf[0] = ld128(qp);
    qf[1] = ld128(qp + 64);
  } else {
    qf[0] = qf[1] = u32x4{0u, 0u, 0u, 0u};
  }

  // Fused RoPE + append of the row's new token (ROPE), with no block barrier: every wave
  // loads the token's k and v pair `lane` of its kv head and its position before the page
  // stream starts (independent of it), and the append slot right after its page ids; lane i
  // computes pair i's (cos, sin), rotates q (ds_bpermute hands each lane the pairs of its
  // fragments) and k, and keeps the rotated k and the v in an LDS slot of the wave's own,
  // from which the wave that attends the token's page takes that row.  The cache slot is
  // written at the end of the kernel: no wave reads it.
  int ap_pid = -1, ap_slot = 0;
  uint32_t kraw = 0u, vraw = 0u;
  float rpos = 0.f;
  if (ROPE) {
    kraw = reinterpret_cast<const uint32_t *>(a.k_new + (int64_t)b * a.k_new_stride + (int64_t)h * kHeadDim)[lane];
    vraw = reinterpret_cast<const uint32_t *>(a.v_new + (int64_t)b * a.v_new_stride + (int64_t)h * kHeadDim)[lane];
    rpos = (float)a.offsets[b];
  }
  // The waves' LDS slots for the token: [64] rotated k pairs, then [64] v pairs, per wave.
  auto rope_slots = [&]() -> uint32_t * {
    return reinterpret_cast<uint32_t *>(
        smem + (TOKMAX ? tokmax_lds_header<G>() + (int)tokmax_logit_floats<G, WITH_V>(a.dump_pages)
                       : rope_lds_offset<G, WITH_V, WITH_DUMP>(nw)));
  };
  uint32_t *const tok_lds = rope_slots() + wave * kHeadDim;

  const int64_t row_elems = (int64_t)a.hkv * kHeadDim;
  const int64_t page_elems = 2 * kPageSize * row_elems;
  const int64_t k_off = (int64_t)(t >> 1) * row_elems + 32 * (t & 1) + 8 * c;  // + k_step(s)
  // K fragment s covers tokens 8 (s / 2) + [0, 8) and d half sp = s % 2.
  auto k_step = [&](int s) -> int64_t { return (int64_t)(s >> 1) * 8 * row_elems + 64 * (s & 1); };
  // V row i of a lane: token c + 4i (V tiles) or 2c + v_row(i) (registers).
  const int64_t v_off = kPageSize * row_elems + (int64_t)(REGV ? 2 * c : c) * row_elems + 8 * t;
  auto v_step = [&](int i) -> int64_t { return (int64_t)(REGV ? v_row(i) : 4 * i) * row_elems; };
  uint16_t *vt = reinterpret_cast<uint16_t *>(smem) + wave * kVTile;           // this wave's V tile
  // Logits staged per wave for a window of kDumpSlots pages, then written out together
  // (flush_window) at the end of the window's last iteration.
  constexpr int kDumpSlots = dump_slots<G, WITH_V>();
  float *dbuf = reinterpret_cast<float *>(smem + (WITH_V ? nw * kVTile / 2 : 0)) + wave * (kDumpSlots * G * kPageSize);

  float m = -INFINITY, l = 0.f;  // running stats of head g = t
  f32x4 acc[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const float sm_scale = a.sm_scale;
  const int first = j0 + rslot;
  const int count = first < j1 ? (j1 - first + R - 1) / R : 0;

  // Page ids of this wave's pages, 64 per register: lane i holds iteration 64 * chunk + i
  // (-1 marks an id outside the cache).  Loading them ahead keeps the page loop free of
  // dependent index loads; each page address comes from one readlane.
  auto load_ids = [&](int it0) -> int {
    const int it = it0 + lane;
    int pid = -1;
    if (it < count) pid = a.kv_indices[ri.p0 + first + (int64_t)R * it];
    return (pid >= 0 && (int64_t)pid < a.num_pages) ? pid : -1;
  };
  auto page_ptr = [&](int pid) -> const uint16_t * {
    return a.kv + (int64_t)(pid < 0 ? 0 : pid) * page_elems + (int64_t)h * kHeadDim;
  };

  // Chunks of up to 64 pages: one id load per chunk, the next chunk's ids loaded a chunk ahead.
  // The next page's K and V are always in flight; the wave's last page issues no load (a
  // repeated streaming load would miss and cost a page of HBM traffic).
  // Staged logits of one window: 4 lanes per (page, head) run of 16 logits, whole pages only
  // (positions past kv_len hold -inf, as the reference's -inf-filled buffer does).
  uint32_t okmask = 0;  // window slots holding a valid page
  // Lane roles in a flush: one (slot, head, quarter) f32x4 per store instruction, kSpi slots
  // per instruction; only two lane-constant 32-bit offsets stay live across the page loop.
  constexpr int kSpi = 64 / (4 * G);                      // slots per store instruction
  constexpr int kFlushInstr = (kDumpSlots + kSpi - 1) / kSpi;
  const int f_sl = lane / (4 * G);                        // slot within an instruction
  const int f_g = (lane % (4 * G)) >> 2, f_qq = lane & 3;
  const bool f_lane = f_sl < kSpi;
  const uint32_t f_lds = (uint32_t)(((f_sl * G + f_g) * kPageSize + 4 * f_qq) * sizeof(float));
  const uint32_t f_dst = (uint32_t)(((int64_t)f_g * a.dump_stride_h + (int64_t)f_sl * R * kPageSize + 4 * f_qq) *
                                    sizeof(float));
  float *const dump_row = WITH_DUMP ? a.dump + (int64_t)b * a.dump_stride_b + (int64_t)h * G * a.dump_stride_h
                                    : nullptr;
  auto flush_window = [&](int gi0, int nslots) {
#pragma unroll
    for (int q = 0; q < kFlushInstr; ++q) {
      const int sl = q * kSpi + f_sl;
      const int jp = first + R * (gi0 + sl);
      if (f_lane && sl < nslots && ((okmask >> sl) & 1u) && jp < a.dump_pages) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const char *>(dbuf) + f_lds +
                                                         q * kSpi * G * kPageSize * sizeof(float));
        // uniform part: first page of instruction q's slots
        const int jq = first + R * (gi0 + q * kSpi);
        float *dst = reinterpret_cast<float *>(reinterpret_cast<char *>(dump_row + (int64_t)jq * kPageSize) + f_dst);
        // Agent-scope (sc1) store through a buffer resource over the block's dump rows (offsets
        // below 2^31, checked on the host): against nontemporal stores the same bytes, the planner
        // 114 -> 109 us at config 4 and planner + score kernel 2001 -> 1913 us at config 5.
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(dump_row, (short)0, 0x7fffffff, kBufferRsrcWord3);
        const int off = (int)(reinterpret_cast<const char *>(dst) - reinterpret_cast<const char *>(dump_row));
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, off, 0, kCpolSc1);
      }
    }
    okmask = 0;
  };

  // RoPE of q and of the token's k (lane i holds pair i's (cos, sin); q pair 32 sp + 16 (t / 8)
  // + 4c + w sits in qf[sp][w], zero for heads past the group).  It needs only the token's
  // position, k and v, not the append slot, so it never waits on the slot's dependent loads.
  auto rope_prologue = [&]() {
    float cs_sn[2];
    rope_cos_sin(lane, rpos, a.rcp_scale, a.log2_theta, a.smooth_a, a.smooth_b, cs_sn);
#pragma unroll
    for (int sp = 0; sp < 2; ++sp)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int j = 32 * sp + 16 * (t >> 3) + 4 * c + w;
        const float cw[2] = {shfl(cs_sn[0], j), shfl(cs_sn[1], j)};
        qf[sp][w] = rope_rotate<DT>(qf[sp][w], cw);
      }
    tok_lds[lane] = rope_rotate<DT>(kraw, cs_sn);
    tok_lds[kHeadDim / 2 + lane] = vraw;
    // Only this wave reads the slot back, in order after these stores.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  // Attention launches run it while their first page is in flight; planner launches (more
  // live registers: the dump staging) here, before their page ids are requested.
  constexpr bool kRopeUnderFirstPage = !WITH_DUMP;
  if (ROPE && !kRopeUnderFirstPage) rope_prologue();
  int ids = count > 0 ? load_ids(0) : -1;
  if (ROPE && kRopeUnderFirstPage) {
    // The token's k, v and position were requested before the page ids: settle them here
    // (the wait leaves the ids in flight), so that no wait in the RoPE prologue, which runs
    // under the first page's loads, also waits for that page.
    asm volatile("" ::"v"(kraw), "v"(vraw), "v"(rpos));
  }
  if (ROPE) {
    // The append slot, with delta_append_kv's checks (a row without a valid slot appends
    // nothing; last_page_len is shared with the attention CSR).  Its page id, a dependent
    // load, goes out right after the page ids: the first page's loads wait only for those.
    __builtin_amdgcn_sched_barrier(0);
    if (ap_q0 >= 0 && ap_q1 > ap_q0 && ap_q1 <= a.ap_indices_len) {
      const int tp = (int)(ap_q1 - ap_q0 - 1) * kPageSize + uniform(ri.last) - 1;  // the new token's position
      if (tp >= 0) {
        ap_pid = ld_scalar(a.ap_indices, ap_q0 + tp / kPageSize);
        ap_slot = tp % kPageSize;
      }
    }
  }
  // One page of the wave (index gi in its page list, id pidc, data in kr / vr): q.K, the logits
  // (dump / on-chip staging), the online softmax and, with V, P.V.  When `more`, the load of
  // page pidn into kr / vr is issued right after kr's last use, so it is in flight while the
  // rest of this page (and any other page in between) is processed.
  auto page_body = [&](int gi, u32x4 (&kr)[4], u32x4 (&vr)[4], int pidc, int pidn, bool more) {
    const int j = first + R * gi;
    const bool ok = pidc >= 0;
    if (ROPE && ok && pidc == ap_pid) {
      // The new token's row of this page (a wave-uniform branch, taken once): K lanes with
      // t / 2 == slot % 8 in steps 2 (slot / 8) + sp, V lanes with c == slot % 4 in tile row
      // group slot / 4.
      if ((t >> 1) == (ap_slot & 7)) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if ((s >> 1) == (ap_slot >> 3))
            kr[s] = *reinterpret_cast<const u32x4 *>(tok_lds + 32 * (s & 1) + 16 * (t & 1) + 4 * c);
      }
      // (register-held V: lanes with 2c == slot % 8 - slot % 2, row i = 2 (slot / 8) + slot % 2)
      if (WITH_V && c == (REGV ? (ap_slot & 7) >> 1 : ap_slot & 3)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (i == (REGV ? 2 * (ap_slot >> 3) + (ap_slot & 1) : ap_slot >> 2))
            vr[i] = *reinterpret_cast<const u32x4 *>(tok_lds + kHeadDim / 2 + 4 * t);
      }
    }

    if (WITH_V && !REGV) {
      // Stage this page's V (loaded one iteration ago) before anything else, so the wait at
      // the top of the iteration is the only one on loaded data and the registers are free
      // for the next page's V below.  Rows past kv_len (and all rows of an invalid page) are
      // zeroed by mask, since they may hold NaN/Inf and meet p = 0.  Token 4i + c goes to
      // tile row 8 (i % 2) + 4 (c / 2) + 2 (i / 2) + c % 2, the row whose k slot holds its p.
      const int vlim = ok ? ri.kv_len - j * kPageSize : 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t keep = 4 * i + c < vlim ? 0xffffffffu : 0u;
        const u32x4 w = vr[i] & u32x4{keep, keep, keep, keep};
        const int trow = 8 * (i & 1) + 4 * (c >> 1) + 2 * (i >> 1) + (c & 1);
        st128(vt + trow * kVStride + 8 * t, w);
      }
    }
    f32x4 S0 = {0.f, 0.f, 0.f, 0.f}, S1 = {0.f, 0.f, 0.f, 0.f};
    S0 = E::mfma(kr[0], qf[0], S0);
    S1 = E::mfma(kr[2], qf[0], S1);
    S0 = E::mfma(kr[1], qf[1], S0);
    S1 = E::mfma(kr[3], qf[1], S1);
    if (more) {
      const uint16_t *nbase = page_ptr(pidn);
#pragma unroll
      for (int s = 0; s < 4; ++s) kr[s] = ld128_stream(nbase + k_off + k_step(s));
      if (WITH_V && !REGV) {
#pragma unroll
        for (int i = 0; i < 4; ++i) vr[i] = ld128_stream(nbase + v_off + v_step(i));
      }
    }

    // Join the d halves: q_g . K[tok(r)] = D[rows 2u, 2u + 1] of columns g and 8 + g.
    const float S[4] = {S0[0] + dpp_f<0x128>(S0[1]), S0[2] + dpp_f<0x128>(S0[3]),
                        S1[0] + dpp_f<0x128>(S1[1]), S1[2] + dpp_f<0x128>(S1[3])};
    const int tok0 = j * kPageSize + 2 * c;  // tok(r) = tok0 + 8 (r / 2) + r % 2
    float x[4], p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      x[r] = (ok && tok0 + 8 * (r >> 1) + (r & 1) < ri.kv_len) ? S[r] * sm_scale : -INFINITY;
    const int slot = gi % kDumpSlots;
    if (TOKMAX && t < G && j < a.dump_pages) {
      float *dl = smem + tokmax_lds_header<G>() + (j * G + t) * kPageSize + 2 * c;
      *reinterpret_cast<float2 *>(dl) = float2{x[0], x[1]};
      *reinterpret_cast<float2 *>(dl + 8) = float2{x[2], x[3]};
    }
    if (WITH_DUMP) {
      // Logits staged in LDS, one slot per page of a kDumpSlots-page window.
      if (t < G) {
        float *dl = dbuf + (slot * G + t) * kPageSize + 2 * c;
        *reinterpret_cast<float2 *>(dl) = float2{x[0], x[1]};
        *reinterpret_cast<float2 *>(dl + 8) = float2{x[2], x[3]};
      }
      okmask |= (ok ? 1u : 0u) << slot;
    }
    float pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] *= kLog2e;
      pm = fmaxf(pm, x[r]);
    }
    const float mn = fmaxf(m, rows4_max(pm));
    const float mref = mn == -INFINITY ? 0.f : mn;
    const float alpha = fast_exp2(m - mref);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = fast_exp2(x[r] - mref);
      ps += p[r];
    }
    l = l * alpha + rows4_sum(ps);
    m = mn;

    if (WITH_V) {
      // Rescale the accumulators only when some head's running max moved.
      if (__ballot(alpha != 1.f)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float al = shfl(alpha, 4 * c + r);
#pragma unroll
          for (int n = 0; n < 8; ++n) acc[n][r] *= al;
        }
      }
      s4_t pa;
#pragma unroll
      for (int r = 0; r < 4; ++r) pa[r] = t < G ? M16::pack(p[r]) : (short)0;
      if (REGV) {
        // This page's V rows (loaded one iteration ago): element n of each row for MFMA n.
        // Rows past kv_len (and all rows of an invalid page) are zeroed by mask, since they
        // may hold NaN/Inf and meet p = 0.  Then the next page's V goes into vr.
        const int vlim = ok ? ri.kv_len - j * kPageSize : 0;
        uint32_t keep[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) keep[i] = 2 * c + v_row(i) < vlim ? 0xffffffffu : 0u;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          // low (n even) or high (n odd) halves of word n / 2: rows 0, 1 and rows 2, 3
          const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
          const uint32_t lo = __builtin_amdgcn_perm(vr[1][n >> 1] & keep[1], vr[0][n >> 1] & keep[0], sel);
          const uint32_t hi = __builtin_amdgcn_perm(vr[3][n >> 1] & keep[3], vr[2][n >> 1] & keep[2], sel);
          acc[n] = M16::run(pa, __builtin_bit_cast(s4_t, (uint2){lo, hi}), acc[n]);
        }
        if (more) {
          const uint16_t *nbase = page_ptr(pidn);
#pragma unroll
          for (int i = 0; i < 4; ++i) vr[i] = ld128_stream(nbase + v_off + v_step(i));
        }
      } else {
        const uint16_t *rd = vt + (4 * c + (t >> 2)) * kVStride + 4 * (t & 3);
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const s4_t bv = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t *)(rd + 16 * n));
          acc[n] = M16::run(pa, bv, acc[n]);
        }
      }
    }
    // Last page of a window (or of the wave): write the window's staged logits.  The
    // stores go out after the next page's loads, which therefore never wait behind them.
    if (WITH_DUMP && (slot == kDumpSlots - 1 || gi + 1 == count)) flush_window(gi - slot, slot + 1);
  };

  auto issue = [&](int pidc, u32x4 (&kr)[4], u32x4 (&vr)[4]) {
    const uint16_t *base = page_ptr(pidc);
    // Issue order K then V, as in the page body, so the waits can stay partial.
#pragma unroll
    for (int s = 0; s < 4; ++s) kr[s] = ld128_stream(base + k_off + k_step(s));
    __builtin_amdgcn_sched_barrier(0);
    if (WITH_V) {
#pragma unroll
      for (int i = 0; i < 4; ++i) vr[i] = ld128_stream(base + v_off + v_step(i));
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Page ids of the wave's pages gi in [cb, cb + 128): lanes of `ids` (chunk cb) and `ids_nx`.
  int cb = 0;
  int ids_nx = count > 64 ? load_ids(64) : -1;
  auto id_at = [&](int gi) -> int {
    const int o = gi - cb;
    return o < 64 ? __builtin_amdgcn_readlane(ids, o) : __builtin_amdgcn_readlane(ids_nx, o - 64);
  };
  auto advance_chunk = [&](int gi) {  // gi reached the next chunk of 64: shift the id registers
    if (gi - cb >= 64) {
      cb += 64;
      ids = ids_nx;
      ids_nx = cb + 64 < count ? load_ids(cb + 64) : -1;
    }
  };

  // The new token's rotated k and v go into its cache slot from the LDS copy of the first wave
  // of each kv head (rslot 0: 32 lanes, one 16-byte chunk each), once per (row, kv head) (split 0
  // of a split row), as soon as that wave's page loop is done: the stores overlap the block's
  // merge instead of following it.  (Issued inside the loop they cost more: stores share vmcnt
  // with the page loads, so the next page's wait would also wait for them.)  No wave of the
  // launch reads the slot's bytes from the cache (the waves attending that page take the row
  // from LDS).
  auto write_own_slot = [&]() {
    if (ROPE && rslot == 0 && lane < 32 && ap_pid >= 0 && (int64_t)ap_pid < a.num_pages &&
        (a.nsplit == 1 || split0)) {
      const int which = lane >> 4, r = lane & 15;  // 0 = K, 1 = V; 16-byte chunk r
      uint16_t *dst = a.kv_w + (((int64_t)ap_pid * 2 + which) * kPageSize + ap_slot) * (int64_t)a.hkv * kHeadDim +
                      (int64_t)h * kHeadDim + 8 * r;
      st128(dst, *reinterpret_cast<const u32x4 *>(tok_lds + which * (kHeadDim / 2) + 4 * r));
    }
  };
  u32x4 kf[4], vf[4];
  if (WITH_V) {
    // Attention: one page in flight (K and V) while the current one is processed.
    int pid = id_at(0);
    if (count > 0) issue(pid, kf, vf);
    if (ROPE && kRopeUnderFirstPage) rope_prologue();
    for (int gi = 0; gi < count; ++gi) {
      advance_chunk(gi);
      const bool more = gi + 1 < count;
      const int pidn = more ? id_at(gi + 1) : -1;
      page_body(gi, kf, vf, pid, pidn, more);
      pid = pidn;
    }
    if (ROPE) write_own_slot();
  } else {
    // K-only scorer: no V tiles or accumulators, so two pages of K are in flight -- pages
    // alternate between the register sets kf and kg, each reloaded two pages ahead.
    u32x4 kg[4];
    int pa = id_at(0), pb = count > 1 ? id_at(1) : -1;
    if (count > 0) issue(pa, kf, vf);
    if (count > 1) issue(pb, kg, vf);
    for (int gi = 0; gi < count; gi += 2) {
      advance_chunk(gi);
      const int p2 = gi + 2 < count ? id_at(gi + 2) : -1;
      page_body(gi, kf, vf, pa, p2, gi + 2 < count);
      pa = p2;
      if (gi + 1 < count) {
        const int p3 = gi + 3 < count ? id_at(gi + 3) : -1;
        page_body(gi + 1, kg, vf, pb, p3, gi + 3 < count);
        pb = p3;
      }
    }
  }

  // Per-token maxima of the row's logits in LDS (TOKMAX): max_g 2^(x_g log2 e - lse2_g).
  auto write_tokmax = [&]() {
    const float *lse2 = smem + tokmax_lds_header<G>() - 16;
    const float *lg = smem + tokmax_lds_header<G>();
    float *outp = a.tokmax + (int64_t)b * a.tokmax_stride_b + (int64_t)head0 * a.tokmax_stride_h;
    const int np_out = ri.np < a.dump_pages ? ri.np : a.dump_pages;
    // Four consecutive tokens per thread: one 16-byte LDS read per head, one 16-byte store.
    for (int tq = threadIdx.x; tq < np_out * (kPageSize / 4); tq += blockDim.x) {
      const int j = tq >> 2, tok = 4 * (tq & 3);
      f32x4 mx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (lse2[g] != -INFINITY) {
          const f32x4 x = *reinterpret_cast<const f32x4 *>(lg + (j * G + g) * kPageSize + tok);
#pragma unroll
          for (int e = 0; e < 4; ++e) mx[e] = fmaxf(mx[e], fast_exp2(x[e] * kLog2e - lse2[g]));
        }
      }
      __builtin_nontemporal_store(mx, reinterpret_cast<f32x4 *>(outp) + tq);
    }
  };

  if constexpr (REGV) {
    // The planner with on-chip logits (head-major, unsplit: one kv head h per block).  The
    // waves' (m, l) give each head's final lse; the logits become per-token maxima; then the
    // waves' accumulators are merged through the logits' space.
    float *const s_ml = smem;                                // [16][G][2]
    float *const lse2 = smem + tokmax_lds_header<G>() - 16;  // [G]
    float *const s_acc = smem + tokmax_lds_header<G>();      // [16][G][128], over the logits
    if (c == 0 && t < G) {
      s_ml[(wave * G + t) * 2 + 0] = m;
      s_ml[(wave * G + t) * 2 + 1] = l;
    }
    __syncthreads();
    if (threadIdx.x < G) {
      const int g = threadIdx.x;
      float M = -INFINITY, L = 0.f;
      for (int w = 0; w < nw; ++w) M = fmaxf(M, s_ml[(w * G + g) * 2]);
      const float Mr = M == -INFINITY ? 0.f : M;
      for (int w = 0; w < nw; ++w) L = fmaf(s_ml[(w * G + g) * 2 + 1], fast_exp2(s_ml[(w * G + g) * 2] - Mr), L);
      lse2[g] = L > 0.f ? M + log2f(L) : -INFINITY;
      if (a.lse != nullptr) a.lse[(int64_t)b * a.hq + h * G + g] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
    }
    __syncthreads();
    write_tokmax();
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int g = 4 * c + r;
      if (g < G) {
#pragma unroll
        for (int n = 0; n < 8; ++n) s_acc[(wave * G + g) * kHeadDim + 8 * t + n] = acc[n][r];
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * kHeadDim; idx += blockDim.x) {
      const int g = idx / kHeadDim, dd = idx % kHeadDim;
      float M = -INFINITY, L = 0.f, A = 0.f;
      for (int w = 0; w < nw; ++w) M = fmaxf(M, s_ml[(w * G + g) * 2]);
      const float Mr = M == -INFINITY ? 0.f : M;
      for (int w = 0; w < nw; ++w) {
        const float sc = fast_exp2(s_ml[(w * G + g) * 2] - Mr);
        L = fmaf(s_ml[(w * G + g) * 2 + 1], sc, L);
        A = fmaf(s_acc[(w * G + g) * kHeadDim + dd], sc, A);
      }
      const float ov = L > 0.f ? A / L : 0.f;
      a.o[(int64_t)b * a.o_stride_b + (int64_t)(h * G + g) * a.o_stride_h + dd] = (uint16_t)E::from_float(ov);
    }
    return;
  }

  // One-wave blocks of a split attention launch (small batches) store their partial straight
  // from registers: lane (c, t) holds O[g = 4c + r][d = 16 n + t] in acc[n][r], lanes c = 0, t < G
  // hold (m, l) of head t.  No block merge, no barrier.
  if constexpr (WITH_V && !WITH_DUMP && !TOKMAX) {
    if (nw == 1 && a.nsplit > 1) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int g = 4 * c + r;
        if (g < G) {
          const int64_t pidx = ((int64_t)pslot * a.hkv + h) * G + g;
#pragma unroll
          for (int n = 0; n < 8; ++n) part_store<AGENT_PARTS>(&a.part_acc[pidx * kHeadDim + 16 * n + t], acc[n][r]);
        }
      }
      if (c == 0 && t < G) {
        const int64_t pidx = ((int64_t)pslot * a.hkv + h) * G + t;
        part_store<AGENT_PARTS>(&a.part_ml[pidx * 2 + 0], m);
        part_store<AGENT_PARTS>(&a.part_ml[pidx * 2 + 1], l);
      }
      return;
    }
  }

  // Merge the block's waves in LDS.  Attention launches have a merge area of their own past
  // the V tiles, so each wave stores its (m, l, acc) as soon as it leaves the loop; the dump
  // launches reuse the V tiles' space once every wave left it.
  constexpr bool kOwnMerge = WITH_V && !WITH_DUMP;
  float *const s_ml = smem + (kOwnMerge ? nw * kVTile / 2 : 0);  // [nw][G][2]
  float *const s_acc = s_ml + nw * G * 2;                                                          // [nw][G][128]
  if (!kOwnMerge) __syncthreads();
  if (c == 0 && t < G) {
    s_ml[(wave * G + t) * 2 + 0] = m;
    s_ml[(wave * G + t) * 2 + 1] = l;
  }
  if (WITH_V) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int g = 4 * c + r;
      if (g < G) {
#pragma unroll
        for (int n = 0; n < 8; ++n) s_acc[(wave * G + g) * kHeadDim + 16 * n + t] = acc[n][r];
      }
    }
  }
  __syncthreads();

  // One output per (kv head, group row, d): combine the R waves of that head.
  const int n_out = hb * (WITH_V ? G * kHeadDim : G);
  for (int idx = threadIdx.x; idx < n_out; idx += blockDim.x) {
    const int hl = WITH_V ? idx / (G * kHeadDim) : idx / G;  // head within the block
    const int hh = head0 + hl;
    const int g = WITH_V ? (idx / kHeadDim) % G : idx % G;
    const int dd = WITH_V ? idx % kHeadDim : 0;
    float M = -INFINITY, L = 0.f, A = 0.f;
    // R waves per head unrolled (head-major launches: 16, or 4 when unsplit), so all the LDS
    // reads issue together (same sums in the same order as the loop below).
    auto unrolled = [&](auto rw) {
      constexpr int RW = decltype(rw)::value;
      float mw[RW], lw[RW], aw[RW];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int w = r * hb + hl;
        mw[r] = s_ml[(w * G + g) * 2];
        lw[r] = s_ml[(w * G + g) * 2 + 1];
        aw[r] = s_acc[(w * G + g) * kHeadDim + dd];
      }
#pragma unroll
      for (int r = 0; r < RW; ++r) M = fmaxf(M, mw[r]);
      const float Mr = M == -INFINITY ? 0.f : M;
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const float sc = fast_exp2(mw[r] - Mr);
        L = fmaf(lw[r], sc, L);
        A = fmaf(aw[r], sc, A);
      }
    };
    if (kOwnMerge && R == kMaxWaves) {
      unrolled(std::integral_constant<int, kMaxWaves>());
    } else if (kOwnMerge && R == kHeadMajorWaves) {
      unrolled(std::integral_constant<int, kHeadMajorWaves>());
    } else {
      for (int r = 0; r < R; ++r) M = fmaxf(M, s_ml[((r * hb + hl) * G + g) * 2]);
      const float Mr = M == -INFINITY ? 0.f : M;
      for (int r = 0; r < R; ++r) {
        const int w = r * hb + hl;
        const float sc = fast_exp2(s_ml[(w * G + g) * 2] - Mr);
        L = fmaf(s_ml[(w * G + g) * 2 + 1], sc, L);
        if (WITH_V) A = fmaf(s_acc[(w * G + g) * kHeadDim + dd], sc, A);
      }
    }
    const int hq = hh * G + g;
    if (a.nsplit == 1) {
      if (WITH_V) {
        const float ov = L > 0.f ? A / L : 0.f;
        a.o[(int64_t)b * a.o_stride_b + (int64_t)hq * a.o_stride_h + dd] = (uint16_t)E::from_float(ov);
      }
      if (dd == 0 && a.lse != nullptr)
        a.lse[(int64_t)b * a.hq + hq] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
      if (TOKMAX) smem[tokmax_lds_header<G>() - 16 + g] = L > 0.f ? M + log2f(L) : -INFINITY;
    } else {
      const int64_t pidx = ((int64_t)pslot * a.hkv + hh) * G + g;
      if (WITH_V) part_store<AGENT_PARTS>(&a.part_acc[pidx * kHeadDim + dd], A);
      if (dd == 0) {
        part_store<AGENT_PARTS>(&a.part_ml[pidx * 2 + 0], M);
        part_store<AGENT_PARTS>(&a.part_ml[pidx * 2 + 1], L);
      }
    }
  }
  if (TOKMAX) {
    __syncthreads();
    write_tokmax();
  }
}

// Named entry kernels, one per reference op, so profiles separate them:
//   full  = target_decode (full CSR), subset = target_subset_decode (selected
//   pages), plan = target_decode_plan (full CSR + logits dump),
//   score = the standalone K-only scorer.
//   ROPE = the new decode token's RoPE and KV append fused in (the *_append entry points).
template <int DT, int G, bool ROPE>
__global__ void __launch_bounds__(kMaxWaves * 64) paged_decode_full_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_split_body<DT, G, true, false, ROPE>(a, smem);
}
template <int DT, int G, bool ROPE>
__global__ void __launch_bounds__(kMaxWaves * 64) paged_decode_subset_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_split_body<DT, G, true, false, ROPE, false, true>(a, smem);
}
template <int DT, int G, bool ROPE>
__global__ void __launch_bounds__(kMaxWaves * 64) paged_decode_plan_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_split_body<DT, G, true, true, ROPE>(a, smem);
}
template <int DT, int G>
__global__ void __launch_bounds__(kMaxWaves * 64) page_score_kv_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_split_body<DT, G, false, true, false>(a, smem);
}
template <int DT, int G>
__global__ void __launch_bounds__(kMaxWaves * 64) page_score_tokmax_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_split_body<DT, G, false, false, false, true>(a, smem);
}
// The planner with the row's logits kept on chip: attention + per-token maxima, no dump.
template <int DT, int G, bool ROPE>
__global__ void __launch_bounds__(kMaxWaves * 64) paged_decode_plan_tokmax_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_split_body<DT, G, true, false, ROPE, true>(a, smem);
}

// Combines the split partials of one (row, q head): thread d of a 128-thread group computes
//   M = max_s m_s,  o[d] = sum_s A_s[d] 2^(m_s - M) / sum_s l_s 2^(m_s - M),
//   lse = (M + log2 sum_s l_s 2^(m_s - M)) ln 2
// over the row's units_of splits.  A block holds ngrp = merge_groups(nsplit) groups (up to 4):
// group q merges the batches of 16 splits that start at 16 q, 16 (q + ngrp), ..., and the
// groups' sums then combine through LDS, so up to 64 splits cost one round of loads.  Partials
// sit at (row, split), so each group's first batch issues its loads with the row bounds, not
// after them (splits the row does not have weigh nothing).
template <int DT>
__global__ void __launch_bounds__(kMergeGroups * kHeadDim) decode_merge_kernel(DecodeArgs a, int G) {
  using E = Elem<DT>;
  __shared__ float s_m[kMergeGroups], s_l[kMergeGroups], s_a[kMergeGroups][kHeadDim];
  const int b = blockIdx.x / a.hq;
  const int hq = blockIdx.x % a.hq;
  const int h = hq / G, g = hq % G;
  const int dd = threadIdx.x % kHeadDim;
  const int grp = threadIdx.x / kHeadDim;
  const int ngrp = blockDim.x / kHeadDim;
  const int nu = units_of(a, b);
  const int64_t stride = (int64_t)a.hkv * G;  // partial rows per split
  const int64_t p0 = ((int64_t)b * a.nsplit * a.hkv + h) * G + g;
  // Batches of 16 splits whose loads all issue together (weight 0 past the row's last split;
  // a group's first batch reads min(16, nsplit - 16 q) slots regardless of the row's count); the
  // running sums move to a new maximum between batches.
  float M = -INFINITY, L = 0.f, A = 0.f;
  auto merge16 = [&](int s0, int lim) {
    float mv[16], lv[16], av[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t pidx = p0 + (int64_t)(s0 + (i < lim ? i : 0)) * stride;
      mv[i] = a.part_ml[pidx * 2];
      lv[i] = a.part_ml[pidx * 2 + 1];
      av[i] = a.part_acc[pidx * kHeadDim + dd];
    }
    float cm = M;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (s0 + i < nu) cm = fmaxf(cm, mv[i]);
    const float cmr = cm == -INFINITY ? 0.f : cm;
    const float al = fast_exp2(M - cmr);  // 0 while nothing is merged (M = -inf)
    L *= al;
    A *= al;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (s0 + i < nu) {
        const float sc = fast_exp2(mv[i] - cmr);
        L = fmaf(lv[i], sc, L);
        A = fmaf(av[i], sc, A);
      }
    }
    M = cm;
  };
  const int first = 16 * grp;  // < nsplit: merge_groups gives no group past the last split
  merge16(first, a.nsplit - first < 16 ? a.nsplit - first : 16);
  for (int s0 = first + 16 * ngrp; s0 < nu; s0 += 16 * ngrp) merge16(s0, nu - s0);
  if (ngrp > 1) {
    if (dd == 0) {
      s_m[grp] = M;
      s_l[grp] = L;
    }
    s_a[grp][dd] = A;
    __syncthreads();
    if (grp != 0) return;
    float MM = -INFINITY;
    for (int q = 0; q < ngrp; ++q) MM = fmaxf(MM, s_m[q]);
    const float Mr = MM == -INFINITY ? 0.f : MM;
    L = 0.f;
    A = 0.f;
    for (int q = 0; q < ngrp; ++q) {
      const float sc = fast_exp2(s_m[q] - Mr);
      L = fmaf(s_l[q], sc, L);
      A = fmaf(s_a[q][dd], sc, A);
    }
    M = MM;
  }
  a.o[(int64_t)b * a.o_stride_b + (int64_t)hq * a.o_stride_h + dd] = (uint16_t)E::from_float(L > 0.f ? A / L : 0.f);
  if (dd == 0 && a.lse != nullptr) a.lse[(int64_t)b * a.hq + hq] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
}

// lse-only merge (scorer path without V): one 64-lane wave per (row, q head), lanes over units.
__global__ void __launch_bounds__(256) decode_merge_lse_kernel(DecodeArgs a, int G) {
  const int idx = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (idx >= a.batch * a.hq) return;
  const int b = idx / a.hq;
  const int hq = idx % a.hq;
  const int nu = units_of(a, b);
  const int64_t stride = (int64_t)a.hkv * G;
  const int64_t p0 = ((int64_t)b * a.nsplit * a.hkv + hq / G) * G + hq % G;
  // The first 64 splits' (m, l) load with the row bounds (lane s holds split s); further ones
  // (rows of more than 64 splits) after them.
  const bool have0 = lane < a.nsplit;
  const int64_t q0 = p0 + (int64_t)(have0 ? lane : 0) * stride;
  const float m0 = a.part_ml[q0 * 2], l0 = a.part_ml[q0 * 2 + 1];
  float M = lane < nu ? m0 : -INFINITY;
  for (int s = lane + 64; s < nu; s += 64) M = fmaxf(M, a.part_ml[(p0 + s * stride) * 2]);
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, shfl_xor(M, off));
  const float Mr = M == -INFINITY ? 0.f : M;
  float L = lane < nu ? l0 * fast_exp2(m0 - Mr) : 0.f;
  for (int s = lane + 64; s < nu; s += 64) {
    const int64_t pidx = p0 + s * stride;
    L = fmaf(a.part_ml[pidx * 2 + 1], fast_exp2(a.part_ml[pidx * 2] - Mr), L);
  }
  for (int off = 32; off > 0; off >>= 1) L += shfl_xor(L, off);
  if (lane == 0) a.lse[idx] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
}

enum Mode { kAttn = 0, kAttnDump = 1, kScoreOnly = 2, kAttnSubset = 3, kScoreTokmax = 4, kAttnTokmax = 5 };

template <int DT, int G>
void launch_split(const DecodeArgs &a, int waves, int mode, hipStream_t stream) {
  dim3 grid = a.nsplit > 1 ? dim3(a.batch * a.nsplit, a.hkv / a.hb) : dim3(a.hkv / a.hb, a.batch);
  dim3 block(64 * waves);
  const bool rope = a.k_new != nullptr;
  const size_t merge = (size_t)waves * G * (2 + kHeadDim) * sizeof(float);
  const size_t tiles = (size_t)waves * kVTile * sizeof(uint16_t);
  const size_t dumps = (size_t)waves * dump_slots<G, true>() * G * kPageSize * sizeof(float);
  const size_t dumps_score = (size_t)waves * dump_slots<G, false>() * G * kPageSize * sizeof(float);
  // Attention launches: V tiles, then their own merge area; planner launches: the merge reuses
  // the V tiles and the dump staging.  The fused append's token slots (512 bytes per wave) sit
  // past everything else, at rope_lds_offset.
  const size_t rope_lds = (size_t)waves * kHeadDim * sizeof(uint32_t);
  const size_t sm_attn = rope ? (size_t)rope_lds_offset<G, true, false>(waves) * sizeof(float) + rope_lds
                              : tiles + merge;
  const size_t sm_plan = rope ? (size_t)rope_lds_offset<G, true, true>(waves) * sizeof(float) + rope_lds
                              : (merge > tiles + dumps ? merge : tiles + dumps);
  const size_t sm_score = dumps_score > (size_t)waves * G * 2 * sizeof(float) ? dumps_score : (size_t)waves * G * 2 * sizeof(float);
  // balanced_row's row tables (5 B + 1 ints at the start of the LDS) fit in every launch's LDS.
  const size_t bal = a.bal_w > 0 ? (size_t)(5 * a.batch + 1) * sizeof(int) : 0;
  auto lds = [bal](size_t sm) { return sm > bal ? sm : bal; };
  switch (mode) {
    case kAttn:
      if (rope)
        hipLaunchKernelGGL((paged_decode_full_kernel<DT, G, true>), grid, block, lds(sm_attn), stream, a);
      else
        hipLaunchKernelGGL((paged_decode_full_kernel<DT, G, false>), grid, block, lds(sm_attn), stream, a);
      break;
    case kAttnSubset:
      if (rope)
        hipLaunchKernelGGL((paged_decode_subset_kernel<DT, G, true>), grid, block, lds(sm_attn), stream, a);
      else
        hipLaunchKernelGGL((paged_decode_subset_kernel<DT, G, false>), grid, block, lds(sm_attn), stream, a);
      break;
    case kAttnDump:
      if (rope)
        hipLaunchKernelGGL((paged_decode_plan_kernel<DT, G, true>), grid, block, lds(sm_plan), stream, a);
      else
        hipLaunchKernelGGL((paged_decode_plan_kernel<DT, G, false>), grid, block, lds(sm_plan), stream, a);
      break;
    case kScoreTokmax:
      hipLaunchKernelGGL((page_score_tokmax_kernel<DT, G>), grid, block,
                         lds((size_t)(tokmax_lds_header<G>() + a.dump_pages * G * kPageSize) * sizeof(float)), stream, a);
      break;
    case kAttnTokmax: {
      const size_t sm = lds((size_t)(tokmax_lds_header<G>() + tokmax_logit_floats<G, true>(a.dump_pages)) *
                                sizeof(float) + (rope ? rope_lds : 0));
      if (rope)
        hipLaunchKernelGGL((paged_decode_plan_tokmax_kernel<DT, G, true>), grid, block, sm, stream, a);
      else
        hipLaunchKernelGGL((paged_decode_plan_tokmax_kernel<DT, G, false>), grid, block, sm, stream, a);
      break;
    }
    default:
      hipLaunchKernelGGL((page_score_kv_kernel<DT, G>), grid, block, lds(sm_score), stream, a);
      break;
  }
}


template <int DT>
void launch_split_g(const DecodeArgs &a, int G, int waves, int mode, hipStream_t stream) {
  switch (G) {
    case 1: launch_split<DT, 1>(a, waves, mode, stream); break;
    case 2: launch_split<DT, 2>(a, waves, mode, stream); break;
    case 3: launch_split<DT, 3>(a, waves, mode, stream); break;
    case 4: launch_split<DT, 4>(a, waves, mode, stream); break;
    case 5: launch_split<DT, 5>(a, waves, mode, stream); break;
    case 6: launch_split<DT, 6>(a, waves, mode, stream); break;
    case 7: launch_split<DT, 7>(a, waves, mode, stream); break;
    default: launch_split<DT, 8>(a, waves, mode, stream); break;
  }
}

}  // namespace

// Launch shape for a (batch, kv heads, max pages) problem, from its arguments only (so a
// captured graph keeps a valid shape).  A block holds R waves per kv head over hb heads:
// one wave per SIMD for unsplit head-major launches (4 waves) and for small ones whose waves
// take at most 8 pages per unit, and R = max(1, 4 / Hkv) waves per head for page-major ones,
// with split counts sized for 16-wave blocks.  Fewer waves per block
// shorten the block's closing merge and the prologue every wave repeats, and a CU keeps
// enough pages in flight regardless (a bare gather streams at full rate from 4 waves of one
// page each):
//   page-major (hb = Hkv): the Hkv waves of one page slot read all heads of a page
//     together (whole 32 KiB K and V runs: ~5.9 TB/s on MI355X), and the split count
//     brings a 16-wave plan to 4096 waves (4 per SIMD on 256 CUs), never below 2 pages per
//     wave; splits cost a merge launch (~5 us).  Run with one wave per head at Hkv = 8
//     (config-3 full 166.6 -> 163.4 us, planner with dump 192.9 -> 185.1 us, config-2
//     planner 99.9 -> 94.3 us);
//   head-major (hb = 1) when the (row, kv head) pairs alone give >= 256 blocks and the
//     launch reads at most kHeadMajorPageHeads page-heads (8 KiB each, ~2 GB): no split and
//     no merge launch (config-3 full attention 170.6 -> 159.6 us against page-major units
//     and their merge).  Past that size, where a ragged batch's longest rows would leave
//     most blocks idle at the end, page-major work units balance better (config 5 full
//     attention 1545 us page-major, 1739 us head-major; 1508 us with the full units
//     first).  These blocks hold 4 waves (one per SIMD): 32 KiB of pages in flight per CU
//     already stream at full rate (a bare gather of the
//     config-3 subset pages: 41.4 us with 4 waves of one page each, 42.0 with 8, 42.2 with
//     16), while the block's closing merge of its waves' partials and the fused RoPE
//     prologue, which every wave repeats, shrink with the wave count (subset launch 44.8 ->
//     44.4 -> 43.6 us for 16 -> 8 -> 4 waves);
//   head-major with splits (grid (units, Hkv)) for attention launches of fewer than 256
//     pairs (small batches): the launch still reaches 256 blocks, and each unit's partials
//     cover one kv head, so the partials and the merge's reads are 1/Hkv of page-major's
//     (config 4 subset: 20.6 -> 15.5 us); 4-wave blocks take 4 pages per wave at config 4
//     (14.8 -> 14.1 us against 16 waves of one page; twice the splits: 16.2).
//     Dump launches (planner, scorer) keep page-major, which measured faster for them.
//   Work units hold at most kMaxChunk pages (128 per wave at Hkv = 8), so a ragged batch is cut
//   into many equal units instead of one share per row sized by its longest row.
constexpr int kHeadMajorPairs = 256;
constexpr int kBalanceMaxRows = 512;  // balanced_row ranks every row in each block
constexpr int kBalanceMinPages = 32;  // shorter rows: the ranking would cost more than the balance gains

// Compute units of the current device (256 on MI355X), cached per device.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}
constexpr int64_t kHeadMajorPageHeads = 262144;
constexpr int kMaxChunk = 128;

void decode_plan(int batch, int hkv, int max_pages, bool dump, int *nsplit, int *waves, int *hb, int *chunk) {
  const bool unsplit = (int64_t)batch * hkv >= kHeadMajorPairs &&
                       (int64_t)batch * hkv * max_pages <= kHeadMajorPageHeads;
  const bool small = !dump && (int64_t)batch * hkv < kHeadMajorPairs;
  const int h = (unsplit || small) ? 1 : hkv;
  int R = h > 0 ? kMaxWaves / h : 1;
  if (R < 1) R = 1;
  const int w = h * R;  // the split count is sized for 16-wave blocks
  const int groups = h > 0 ? hkv / h : 1;
  int64_t ns = 1;
  if (batch > 0 && max_pages > 0) {
    ns = ceil_div(256 * 4 * 4, (int64_t)batch * groups * w);
    int64_t cap = max_pages / ((small ? 1 : 2) * R);
    if (cap < 1) cap = 1;
    if (ns > cap) ns = cap;
    if (ns < 1) ns = 1;
    if (ns > 1024) ns = 1024;
  }
  if (unsplit) {
    R = kHeadMajorWaves;
    ns = 1;
  } else if (!small) {
    R = kHeadMajorWaves / h > 1 ? kHeadMajorWaves / h : 1;
  }
  int64_t ch = max_pages > 0 ? ceil_div(max_pages, ns) : 1;
  if (ns > 1 && ch > kMaxChunk) {
    ch = kMaxChunk;
    ns = ceil_div(max_pages, ch);
  }
  // Small launches whose units give each of 4 waves at most 8 pages (the config 2 and 4 subset
  // launches) run 4-wave blocks; when they split and 4x their split count still fits one 16-split
  // merge batch (config 2: 4 -> 16 splits) they run one-wave blocks with 4x the splits instead
  // (an unsplit launch keeps its blocks: no merge launch), each wave
  // storing its partial from registers with no closing block merge (config-2 subset 17.4 -> 16.6
  // us; at config 4, 16 -> 64 splits, the merge's 4x partials cost more than the block merge
  // saves: 13.6 -> 14.2 us).  Others keep 16 waves (the config-4 full attention, 128-page units:
  // with 4 waves its full-cache engine step ran 5.4-5.6 -> 5.9-6.0 ms, though a launch timed alone
  // was unchanged).
  if (small && ceil_div(ch, (int64_t)kHeadMajorWaves) <= 8) {
    R = kHeadMajorWaves;
    if (ns > 1 && ns * kHeadMajorWaves <= 16 && ns * kHeadMajorWaves <= max_pages) {
      ns *= kHeadMajorWaves;
      ch = ceil_div(max_pages, ns);
      R = 1;
    }
  }
  *nsplit = (int)ns;
  *waves = h * R;
  *hb = h;
  *chunk = (int)(ch < 1 ? 1 : ch);
}

// The K-only scorer keeps the row's logits in LDS (no dump, no merge launch) when a head-major
// unsplit launch fills the GPU (>= 256 (row, kv head) blocks) and max_pages * G * 16 logits fit
// beside the merge header in 160 KiB.
bool tokmax_fits(int batch, int hkv, int G, int max_pages) {
  const int64_t lds = ((int64_t)kMaxWaves * G * 2 + 16 + (int64_t)max_pages * G * kPageSize) * (int64_t)sizeof(float);
  return (int64_t)batch * hkv >= kHeadMajorPairs && lds <= 160 * 1024;
}

// The planner keeps the row's logits in LDS (no dump) under the same conditions, with room for
// the waves' accumulators (at least 128 pages' worth of logits) and the append's token slots.
bool plan_tokmax_fits(int batch, int hkv, int G, int max_pages, bool rope) {
  const int64_t floats = kMaxWaves * G * 2 + 16 + (max_pages < 128 ? 128 : (int64_t)max_pages) * G * kPageSize;
  const int64_t lds = floats * (int64_t)sizeof(float) + (rope ? kMaxWaves * kHeadDim * 4 : 0);
  return (int64_t)batch * hkv >= kHeadMajorPairs && max_pages > 0 && lds <= 160 * 1024;
}

int decode_num_splits(int batch, int hkv, int max_pages) {
  int ns, w, hb, ch, ns_dump;
  decode_plan(batch, hkv, max_pages, false, &ns, &w, &hb, &ch);
  decode_plan(batch, hkv, max_pages, true, &ns_dump, &w, &hb, &ch);
  return ns > ns_dump ? ns : ns_dump;
}

// Workspace of a split launch: (m, l) for every (row, split, q head), then acc: batch * nsplit
// slots, of which each row uses its units_of.
size_t decode_workspace_bytes(int batch, int hq, int nsplit, bool with_acc) {
  if (nsplit <= 1) return 0;
  const size_t per = (with_acc ? kHeadDim : 0) + 2;
  return ((size_t)batch * hq * nsplit * per * sizeof(float) + 255) & ~(size_t)255;
}

// Shared validation + launch used by the attention and the scorer entry points.
int run_decode(const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *kv_cache,
               int64_t num_pages, const int32_t *kv_indptr, const int32_t *kv_indices,
               int64_t kv_indices_len, const int32_t *kv_last_page_len, void *o,
               int64_t o_stride_b, int64_t o_stride_h, float *lse, float *dump,
               int64_t dump_stride_b, int64_t dump_stride_h, int batch, int hq, int hkv,
               int head_dim, int dtype, float sm_scale, int max_pages, int mode,
               void *workspace, size_t workspace_bytes, hipStream_t stream, const char *who,
               const delta_decode_append_t *ap) {
  clear_error();
  if (batch <= 0) return DELTA_OK;
  if (head_dim != kHeadDim) return set_error(DELTA_ERR_INVALID, "%s: head_dim must be 128 (got %d)", who, head_dim);
  if (hkv <= 0 || hq <= 0 || hq % hkv != 0)
    return set_error(DELTA_ERR_INVALID, "%s: num_qo_heads (%d) must be a multiple of num_kv_heads (%d)", who, hq, hkv);
  const int G = hq / hkv;
  if (G > kMaxGroup) return set_error(DELTA_ERR_INVALID, "%s: group size %d > %d unsupported", who, G, kMaxGroup);
  if (hkv > kMaxWaves) return set_error(DELTA_ERR_INVALID, "%s: num_kv_heads %d > %d unsupported", who, hkv, kMaxWaves);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: dtype must be bf16 or fp16", who);
  if (!q || !kv_cache || !kv_indptr || !kv_indices || !kv_last_page_len)
    return set_error(DELTA_ERR_INVALID, "%s: null input pointer", who);
  // `dump` is the [batch][hkv][stride_h] per-token maxima output of the TOKMAX modes
  const bool tokmax = mode == kScoreTokmax || mode == kAttnTokmax;
  if (mode != kScoreOnly && mode != kScoreTokmax && !o) return set_error(DELTA_ERR_INVALID, "%s: null output pointer", who);
  if ((mode == kAttnDump || mode == kScoreOnly || tokmax) && !dump)
    return set_error(DELTA_ERR_INVALID, "%s: null logits dump", who);
  if (mode == kScoreTokmax && !tokmax_fits(batch, hkv, G, max_pages))
    return set_error(DELTA_ERR_INVALID, "%s: this shape does not fit the LDS scorer", who);
  if (mode == kAttnTokmax && !plan_tokmax_fits(batch, hkv, G, max_pages, ap != nullptr))
    return set_error(DELTA_ERR_INVALID, "%s: this shape does not fit the on-chip planner", who);
  if (((uintptr_t)q | (uintptr_t)kv_cache) & 15u)
    return set_error(DELTA_ERR_INVALID, "%s: q and kv_cache must be 16-byte aligned", who);
  if ((q_stride_h % 8) || (q_stride_b % 8))
    return set_error(DELTA_ERR_INVALID, "%s: q strides must be multiples of 8 elements", who);
  if (num_pages <= 0 || kv_indices_len < 0) return set_error(DELTA_ERR_INVALID, "%s: empty cache", who);
  // The dump writer addresses a (row, kv head) block of G dump rows with offsets below 2^31 bytes.
  if (dump && (dump_stride_b < 0 || dump_stride_h < 0 || (int64_t)(G - 1) * dump_stride_h > (int64_t)1 << 28 ||
               (int64_t)(max_pages > 0 ? max_pages : 1) * kPageSize > (int64_t)1 << 28 || ((uintptr_t)dump & 3u)))
    return set_error(DELTA_ERR_INVALID, "%s: logits dump strides must be non-negative, 4-byte aligned, "
                     "(G - 1) * stride_h <= 2^28 and max_pages * 16 <= 2^28", who);
  if (max_pages <= 0) max_pages = 1;

  DecodeArgs a;
  a.q = (const uint16_t *)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.kv = (const uint16_t *)kv_cache;
  a.num_pages = num_pages;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.kv_indices_len = kv_indices_len;
  a.last_page_len = kv_last_page_len;
  a.o = (uint16_t *)o;
  a.o_stride_b = o_stride_b;
  a.o_stride_h = o_stride_h;
  a.lse = lse;
  a.dump = tokmax ? nullptr : dump;
  a.dump_stride_b = dump_stride_b;
  a.dump_stride_h = dump_stride_h;
  a.dump_pages = max_pages;
  a.tokmax = tokmax ? dump : nullptr;
  a.tokmax_stride_b = dump_stride_b;
  a.tokmax_stride_h = dump_stride_h;
  a.batch = batch;
  a.hq = hq;
  a.hkv = hkv;
  int waves;
  decode_plan(batch, hkv, max_pages, dump != nullptr, &a.nsplit, &waves, &a.hb, &a.chunk);
  if (tokmax) {  // head-major, unsplit: each block ends with its head's final lse
    // 4 waves (one per SIMD), as the other unsplit head-major launches: config-3 planner
    // 176.1 -> 169.7 us and K-only scorer 92.2 -> 88.5 us against 16 waves (8 waves: 173.3 /
    // 91.7).
    a.nsplit = 1;
    a.hb = 1;
    waves = kHeadMajorWaves;
    a.chunk = max_pages;
  }
  // Head-major split launches (small batches: fewer than 256 (row, kv head) pairs) map blocks to
  // units directly; page-major ones pack a ragged batch's units at the front of the grid.
  a.direct = a.nsplit > 1 && a.hb == 1;
  // Unsplit head-major launches with more blocks than CUs deal ragged rows to CUs evenly.
  const int cus = device_cus();
  a.bal_w = (a.nsplit == 1 && a.hb == 1 && (int64_t)batch * hkv > cus && batch <= kBalanceMaxRows &&
             max_pages >= kBalanceMinPages)
                ? (cus / hkv > 0 ? cus / hkv : 1)
                : 0;
  a.sm_scale = sm_scale;
  a.part_acc = nullptr;
  a.part_ml = nullptr;
  a.kv_w = nullptr;
  a.k_new = a.v_new = nullptr;
  a.k_new_stride = a.v_new_stride = 0;
  a.offsets = a.ap_indptr = a.ap_indices = nullptr;
  a.ap_indices_len = 0;
  a.rcp_scale = a.log2_theta = a.smooth_a = a.smooth_b = 0.f;
  if (ap) {
    if (mode == kScoreOnly || mode == kScoreTokmax)
      return set_error(DELTA_ERR_INVALID, "%s: the scorer takes no append", who);
    if (!ap->k || !ap->v || !ap->offsets || !ap->kv_indptr || !ap->kv_indices)
      return set_error(DELTA_ERR_INVALID, "%s: null append pointer", who);
    if ((((uintptr_t)ap->k | (uintptr_t)ap->v) & 3u) || (ap->k_stride % 2) || (ap->v_stride % 2) ||
        ap->k_stride < 0 || ap->v_stride < 0 || ap->kv_indices_len < 0)
      return set_error(DELTA_ERR_INVALID, "%s: append k/v must be 4-byte aligned with even row strides", who);
    if (!(ap->rope_scale > 0.f) || !(ap->rope_theta > 0.f))
      return set_error(DELTA_ERR_INVALID, "%s: bad rope params", who);
    a.kv_w = (uint16_t *)kv_cache;
    a.k_new = (const uint16_t *)ap->k;
    a.k_new_stride = ap->k_stride;
    a.v_new = (const uint16_t *)ap->v;
    a.v_new_stride = ap->v_stride;
    a.offsets = ap->offsets;
    a.ap_indptr = ap->kv_indptr;
    a.ap_indices = ap->kv_indices;
    a.ap_indices_len = ap->kv_indices_len;
    a.rcp_scale = 1.0f / ap->rope_scale;
    a.log2_theta = log2f(ap->rope_theta);
    if (ap->llama31) {
      if (!(ap->high_freq_factor > ap->low_freq_factor) || !(ap->low_freq_factor > 0.f))
        return set_error(DELTA_ERR_INVALID, "%s: bad llama3.1 frequency factors", who);
      const float two_pi = 6.283185307179586f;
      a.smooth_a = ap->old_context_len / (two_pi * ap->high_freq_factor - two_pi * ap->low_freq_factor);
      a.smooth_b = -1.0f / (ap->high_freq_factor / ap->low_freq_factor - 1.0f);
    }
  }

  if (a.hb < 1 || a.hkv % a.hb != 0)
    return set_error(DELTA_ERR_INVALID, "%s: launch planned with %d of %d kv heads per block", who, a.hb, a.hkv);
  const bool with_acc = mode != kScoreOnly && mode != kScoreTokmax;
  const size_t need = decode_workspace_bytes(batch, hq, a.nsplit, with_acc);
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return set_error(DELTA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who, need, workspace_bytes);
    if ((uintptr_t)workspace & 255u) return set_error(DELTA_ERR_INVALID, "%s: workspace must be 256-byte aligned", who);
    float *ws = (float *)workspace;
    a.part_ml = ws;
    a.part_acc = ws + (size_t)batch * hq * a.nsplit * 2;
  }
  if (mode == kScoreOnly && !lse && a.nsplit > 1)
    return set_error(DELTA_ERR_INVALID, "%s: scorer needs an lse buffer", who);

  if (dtype == DELTA_BF16)
    launch_split_g<DELTA_BF16>(a, G, waves, mode, stream);
  else
    launch_split_g<DELTA_FP16>(a, G, waves, mode, stream);
  int rc = check_launch(who);
  if (rc || a.nsplit == 1) return rc;
  if (with_acc) {
    if (dtype == DELTA_BF16)
      hipLaunchKernelGGL(decode_merge_kernel<DELTA_BF16>, dim3(batch * hq), dim3(kHeadDim * merge_groups(a.nsplit)), 0,
                         stream, a, G);
    else
      hipLaunchKernelGGL(decode_merge_kernel<DELTA_FP16>, dim3(batch * hq), dim3(kHeadDim * merge_groups(a.nsplit)), 0,
                         stream, a, G);
  } else {
    const int n = batch * hq;
    hipLaunchKernelGGL(decode_merge_lse_kernel, dim3((n + 3) / 4), dim3(256), 0, stream, a, G);
  }
  return check_launch(who);
}

}  // namespace delta

extern "C" DELTA_EXPORT int delta_decode_num_splits(int batch, int num_kv_heads, int max_pages_per_row) {
  return delta::decode_num_splits(batch, num_kv_heads, max_pages_per_row);
}

extern "C" DELTA_EXPORT size_t delta_paged_decode_workspace_bytes(int batch, int num_qo_heads, int num_kv_heads,
                                                                  int max_pages_per_row) {
  const int ns = delta::decode_num_splits(batch, num_kv_heads, max_pages_per_row);
  return delta::decode_workspace_bytes(batch, num_qo_heads, ns, true);
}

extern "C" DELTA_EXPORT int delta_paged_decode(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                               const void *kv_cache, int64_t num_pages, const int32_t *kv_indptr,
                                               const int32_t *kv_indices, int64_t kv_indices_len,
                                               const int32_t *kv_last_page_len, void *o, int64_t o_stride_b,
                                               int64_t o_stride_h, float *lse, float *logits_dump,
                                               int64_t dump_stride_b, int64_t dump_stride_h, int batch,
                                               int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
                                               float sm_scale, int max_pages_per_row, void *workspace,
                                               size_t workspace_bytes, delta_stream_t stream) {
  const int mode = logits_dump ? delta::kAttnDump : delta::kAttn;
  return delta::run_decode(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices, kv_indices_len,
                           kv_last_page_len, o, o_stride_b, o_stride_h, lse, logits_dump, dump_stride_b,
                           dump_stride_h, batch, num_qo_heads, num_kv_heads, head_dim, dtype, sm_scale,
                           max_pages_per_row, mode, workspace, workspace_bytes, (hipStream_t)stream,
                           "delta_paged_decode", nullptr);
}

extern "C" DELTA_EXPORT int delta_paged_decode_subset(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                                      const void *kv_cache, int64_t num_pages,
                                                      const int32_t *kv_indptr, const int32_t *kv_indices,
                                                      int64_t kv_indices_len, const int32_t *kv_last_page_len, void *o,
                                                      int64_t o_stride_b, int64_t o_stride_h, float *lse, int batch,
                                                      int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
                                                      float sm_scale, int max_pages_per_row, void *workspace,
                                                      size_t workspace_bytes, delta_stream_t stream) {
  return delta::run_decode(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices, kv_indices_len,
                           kv_last_page_len, o, o_stride_b, o_stride_h, lse, nullptr, 0, 0, batch, num_qo_heads,
                           num_kv_heads, head_dim, dtype, sm_scale, max_pages_per_row, delta::kAttnSubset, workspace,
                           workspace_bytes, (hipStream_t)stream, "delta_paged_decode_subset", nullptr);
}

extern "C" DELTA_EXPORT int delta_paged_decode_append(const delta_decode_append_t *append, const void *q,
                                                      int64_t q_stride_b, int64_t q_stride_h, void *kv_cache,
                                                      int64_t num_pages, const int32_t *kv_indptr,
                                                      const int32_t *kv_indices, int64_t kv_indices_len,
                                                      const int32_t *kv_last_page_len, void *o, int64_t o_stride_b,
                                                      int64_t o_stride_h, float *lse, float *logits_dump,
                                                      int64_t dump_stride_b, int64_t dump_stride_h, int batch,
                                                      int num_qo_heads, int num_kv_heads, int head_dim, int dtype,
                                                      float sm_scale, int max_pages_per_row, void *workspace,
                                                      size_t workspace_bytes, delta_stream_t stream) {
  if (!append) return delta::set_error(DELTA_ERR_INVALID, "delta_paged_decode_append: null append");
  const int mode = logits_dump ? delta::kAttnDump : delta::kAttn;
  return delta::run_decode(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices, kv_indices_len,
                           kv_last_page_len, o, o_stride_b, o_stride_h, lse, logits_dump, dump_stride_b,
                           dump_stride_h, batch, num_qo_heads, num_kv_heads, head_dim, dtype, sm_scale,
                           max_pages_per_row, mode, workspace, workspace_bytes, (hipStream_t)stream,
                           "delta_paged_decode_append", append);
}

extern "C" DELTA_EXPORT int delta_paged_decode_subset_append(const delta_decode_append_t *append, const void *q,
                                                             int64_t q_stride_b, int64_t q_stride_h, void *kv_cache,
                                                             int64_t num_pages, const int32_t *kv_indptr,
                                                             const int32_t *kv_indices, int64_t kv_indices_len,
                                                             const int32_t *kv_last_page_len, void *o,
                                                             int64_t o_stride_b, int64_t o_stride_h, float *lse,
                                                             int batch, int num_qo_heads, int num_kv_heads,
                                                             int head_dim, int dtype, float sm_scale,
                                                             int max_pages_per_row, void *workspace,
                                                             size_t workspace_bytes, delta_stream_t stream) {
  if (!append) return delta::set_error(DELTA_ERR_INVALID, "delta_paged_decode_subset_append: null append");
  return delta::run_decode(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices, kv_indices_len,
                           kv_last_page_len, o, o_stride_b, o_stride_h, lse, nullptr, 0, 0, batch, num_qo_heads,
                           num_kv_heads, head_dim, dtype, sm_scale, max_pages_per_row, delta::kAttnSubset, workspace,
                           workspace_bytes, (hipStream_t)stream, "delta_paged_decode_subset_append", append);
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the split partials live in a file-scope device array instead of a
// caller workspace, for callers that cannot allocate (graph capture, serving loops that forbid
// hipMalloc).  Each GPU holds its own copy of the array until the process ends; its device
// address is looked up once per device, with that device current, and only that address is
// handed to kernels (the array's name is a host-side stand-in, not a device address).
// ---------------------------------------------------------------------------
namespace delta {
namespace {

constexpr size_t kScratchBytes = (size_t)64 << 20;  // 64 MiB: every BASELINE shape needs <= 46 MB
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {nullptr};

// The current device's copy of `scratch` (null, with the error set, on failure).
void *scratch_for_current_device(const char *who) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error(DELTA_ERR_HIP, "%s: no usable current device (%d)", who, dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error(DELTA_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT int delta_paged_decode_noalloc(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                                       const void *kv_cache, int64_t num_pages,
                                                       const int32_t *kv_indptr, const int32_t *kv_indices,
                                                       int64_t kv_indices_len, const int32_t *kv_last_page_len,
                                                       void *o, int64_t o_stride_b, int64_t o_stride_h, float *lse,
                                                       float *logits_dump, int64_t dump_stride_b,
                                                       int64_t dump_stride_h, int batch, int num_qo_heads,
                                                       int num_kv_heads, int head_dim, int dtype, float sm_scale,
                                                       int max_pages_per_row, delta_stream_t stream) {
  const char *who = "delta_paged_decode_noalloc";
  delta::clear_error();
  if (batch <= 0) return DELTA_OK;
  if (num_kv_heads <= 0 || num_qo_heads <= 0)
    return delta::set_error(DELTA_ERR_INVALID, "%s: head counts must be positive", who);
  const size_t need = delta_paged_decode_workspace_bytes(batch, num_qo_heads, num_kv_heads,
                                                         max_pages_per_row > 0 ? max_pages_per_row : 1);
  if (need > delta::kScratchBytes)
    return delta::set_error(DELTA_ERR_INVALID,
                            "%s: this shape needs %zu bytes of split scratch, more than the %zu-byte static "
                            "scratch; use delta_paged_decode with a workspace",
                            who, need, delta::kScratchBytes);
  void *ws = delta::scratch_for_current_device(who);
  if (!ws) return DELTA_ERR_HIP;
  const int mode = logits_dump ? delta::kAttnDump : delta::kAttn;
  return delta::run_decode(q, q_stride_b, q_stride_h, kv_cache, num_pages, kv_indptr, kv_indices, kv_indices_len,
                           kv_last_page_len, o, o_stride_b, o_stride_h, lse, logits_dump, dump_stride_b,
                           dump_stride_h, batch, num_qo_heads, num_kv_heads, head_dim, dtype, sm_scale,
                           max_pages_per_row, mode, ws, delta::kScratchBytes, (hipStream_t)stream, who, nullptr);
}
