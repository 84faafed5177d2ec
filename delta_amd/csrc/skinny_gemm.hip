// Decode-batch GEMM for gfx950: out[m, n] = sum_k x[m, k] * W[n, k] (+ bias[n]), M <= 32.
//
// The projections of a decode step (model.py:412 wqkv, 432 wo, 509-514 w1/w3/w2, 328 lm_head;
// nn.Linear layout, W is [N, K] row-major) multiply a handful of token rows by a large weight,
// so they are weight-streaming: 2 bytes of W per 2 * M flops.  At M = 32 hipBLASLt streams the
// smaller weights at 1.7-3.7 TB/s (few, large tiles); this kernel is built to stream W once at
// HBM rate:
//
//   grid = (N / (8 * NB), ceil(M / (8 TG))), block = 8 waves splitting K; wave w owns k in
//   [w * kper, (w + 1) * kper) for the block's 8 * NB output columns and 8 TG token rows
//   (TG = 1 at M <= 8, else 4), with 1 or 2 k steps of loads in flight.
//   Per 64-wide k step and 8-column block, one v_mfma_f32_16x16x32 per 8 token rows:
//     A = W: row i = 2u + e is column n0 + u restricted to k in 32 e + [0, 32); lane (c, t)
//         loads W[n0 + t/2][k + 32 (t%2) + 8c, +8), so one load instruction covers 8 weight
//         rows x 128 contiguous bytes (whole cache lines, streaming hint);
//     B = x^T: column j = 8 e' + v is token v of the group restricted to the same k slice e';
//     D[2u + e][8 e' + v] is a partial dot product only when e == e', so
//     out(u, v) = D[2u][v] + D[2u + 1][8 + v] -- one DPP row rotate by 8, done once at the end
//     (the join is linear, so the accumulators stay raw over all k steps).
//   The 8 waves' partials meet in LDS and the block writes bf16/fp16 rows (fp32 sum, bias
//   added before the one rounding).
//
// HBM bytes per launch (algorithmic): W once (N * K * 2) + x and out (small).  Measured on
// MI355X against hipBLASLt (x @ W.T, graph replays over rotating weights): at M = 4 this kernel
// streams the Llama-3-8B projections at 4.5-6.0 TB/s (hipBLASLt 2.1-4.7) and the Qwen2.5-7B ones at
// 3.3-6.6 TB/s (hipBLASLt 2.1-5.1; merged w1|w3 41 vs 53 us).  At M = 32 it is faster standalone
// for weights up to ~48 MB (wo: 12.5 vs 19.7 us) and slower for the large ones: every block
// re-reads the x fragments of its k range (as many load instructions as for W), which costs
// most inside a decode step, where x was just written across all 8 XCDs' L2s.
#include "delta_common.h"

namespace delta {
namespace {

constexpr int kGemmWaves = 8;  // 2-3 blocks per CU overlap one block's reduction with another's loads

struct GemmArgs {
  const uint16_t *x;
  int64_t ldx;
  const uint16_t *w;
  int64_t ldw;
  const uint16_t *bias;
  uint16_t *out;
  int64_t ldo;
  int M, N, K, kper;
  int inter;  // GLU: W = [gate rows; up rows], out [M][inter]
};

// TG groups of 8 token rows per block (TG = 1 for M <= 8, else 4); each wave keeps D k steps of
// W and x in flight (a ring of D fragment sets), so the launch has enough bytes in flight to
// stream W at HBM rate even when the N / 16 blocks barely cover the CUs.
// GLU (FeedForward's gate/up GEMM and SiLU-mul, model.py:509-514): column groups nb < NB / 2 are
// gate columns n0 + 8 nb, the others the matching up columns inter + n0 + 8 (nb - NB / 2); the
// block writes dtype(dtype(silu(g)) * u) of its 4 NB columns, g and u rounded to the dtype first.
template <int DT, int NB, int TG, int D, bool GLU = false>
__global__ void __launch_bounds__(kGemmWaves * 64) gemm_skinny_kernel(GemmArgs a) {
  using E = Elem<DT>;
  extern __shared__ float red[];  // [wave][8 TG token rows][8 NB columns]
  constexpr int kCols = 8 * NB;
  constexpr int kRows = 8 * TG;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane >> 4, t = lane & 15;
  const int n0 = blockIdx.x * (GLU ? kCols / 2 : kCols);
  // row offset of column group nb in W
  auto grp = [&](int nb) -> int64_t {
    return GLU && nb >= NB / 2 ? (int64_t)a.inter + 8 * (nb - NB / 2) : (int64_t)8 * nb;
  };
  const int m0 = blockIdx.y * kRows;
  const int kb = wave * a.kper;
  const int ke = min(a.K, kb + a.kper);
  const int S = ke > kb ? (ke - kb) / 64 : 0;  // this wave's k steps

  const uint16_t *wp = a.w + (int64_t)(n0 + (t >> 1)) * a.ldw + 32 * (t & 1) + 8 * c + kb;
  const uint16_t *xp[TG];
  bool xok[TG];
#pragma unroll
  for (int tg = 0; tg < TG; ++tg) {
    const int r = m0 + 8 * tg + (t & 7);
    xok[tg] = r < a.M;
    xp[tg] = a.x + (int64_t)(xok[tg] ? r : 0) * a.ldx + 32 * (t >> 3) + 8 * c + kb;
  }

  f32x4 acc[NB][TG];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) acc[nb][tg] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 wf[D][NB], xf[D][TG];
  auto load = [&](int d, int s) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) wf[d][nb] = ld128_stream(wp + grp(nb) * a.ldw + 64 * s);
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) xf[d][tg] = xok[tg] ? ld128(xp[tg] + 64 * s) : u32x4{0u, 0u, 0u, 0u};
  };
  auto step = [&](int d) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int tg = 0; tg < TG; ++tg) acc[nb][tg] = E::mfma(wf[d][nb], xf[d][tg], acc[nb][tg]);
  };
  // Step s lives in slot s % D.  Prologue: the first D steps; steady state: use slot d, refill
  // it D steps ahead (no branch while 2 D steps remain); then the last 1..2 D steps.
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < S) load(d, d);
  int s0 = 0;
  for (; s0 + 2 * D <= S; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      step(d);
      load(d, s0 + d + D);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    if (s0 + d < S) {
      step(d);
      if (s0 + d + D < S) load(d, s0 + d + D);
    }
  }
  s0 += D;
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (s0 + d < S) step(d);

  // Join the k slices and park this wave's partials: lane (c, v < 8) holds columns
  // n0 + 8 nb + 2c + {0, 1} of token row 8 tg + v.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) {
      const float s0v = acc[nb][tg][0] + dpp_f<0x128>(acc[nb][tg][1]);
      const float s1v = acc[nb][tg][2] + dpp_f<0x128>(acc[nb][tg][3]);
      if (t < 8) {
        float *r = red + ((int64_t)wave * kRows + 8 * tg + t) * kCols + 8 * nb + 2 * c;
        r[0] = s0v;
        r[1] = s1v;
      }
    }
  __syncthreads();
  if (GLU) {
    constexpr int kOut = kCols / 2;
    for (int idx = threadIdx.x; idx < kRows * kOut; idx += kGemmWaves * 64) {
      const int row = idx / kOut, col = idx % kOut;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < kGemmWaves; ++w) {
        g += red[(w * kRows + row) * kCols + col];
        u += red[(w * kRows + row) * kCols + kOut + col];
      }
      if (m0 + row < a.M) {
        const float gr = E::lo(E::from_float(g)), ur = E::lo(E::from_float(u));
        const float h = E::lo(E::from_float(gr / (1.f + expf(-gr))));
        a.out[(int64_t)(m0 + row) * a.ldo + n0 + col] = (uint16_t)E::from_float(h * ur);
      }
    }
    return;
  }
  for (int idx = threadIdx.x; idx < kRows * kCols; idx += kGemmWaves * 64) {
    const int row = idx / kCols, col = idx % kCols;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kGemmWaves; ++w) sum += red[(w * kRows + row) * kCols + col];
    if (m0 + row < a.M) {
      if (a.bias) sum += (float)E::lo(a.bias[n0 + col]);
      a.out[(int64_t)(m0 + row) * a.ldo + n0 + col] = (uint16_t)E::from_float(sum);
    }
  }
}

template <int DT, int NB, int TG, int D>
void launch_nb(const GemmArgs &a, hipStream_t stream) {
  const dim3 grid(a.N / (8 * NB), (a.M + 8 * TG - 1) / (8 * TG));
  hipLaunchKernelGGL((gemm_skinny_kernel<DT, NB, TG, D>), grid, dim3(kGemmWaves * 64),
                     kGemmWaves * 8 * TG * 8 * NB * sizeof(float), stream, a);
}

// At M <= 8 a wave keeps two k steps in flight when the launch has at most one block per CU
// (the bytes in flight must come from depth there), one otherwise.  Measured at 4 token rows
// (graph replays, rotating weights): Qwen2.5-7B w2 30.7 -> 22.8 us, wo 8.3 -> 6.5 us; a depth
// of 4 or 8 was slower again, and so was depth 2 with more than 256 blocks.
template <int DT>
int launch_gemm(const GemmArgs &a, int nb, hipStream_t stream) {
  if (a.M <= 8) {
    const bool deep = a.N / (8 * nb) <= 256;
    if (nb == 4) deep ? launch_nb<DT, 4, 1, 2>(a, stream) : launch_nb<DT, 4, 1, 1>(a, stream);
    else deep ? launch_nb<DT, 2, 1, 2>(a, stream) : launch_nb<DT, 2, 1, 1>(a, stream);
  } else {
    if (nb == 4) launch_nb<DT, 4, 4, 1>(a, stream);
    else launch_nb<DT, 2, 4, 1>(a, stream);
  }
  return check_launch("delta_gemm_skinny");
}

// ---------------------------------------------------------------------------------------------
// Decode GEMM at up to 32 token rows: x staged in LDS once per block and shared by its 8 waves.
//
// The kernel above splits K across the waves of a block, so every wave reads its own slice of
// x, as many load instructions as for W at 32 rows.  Here the 8 waves of a block own different
// columns (8 NB each, 64 NB per block) over the same k range, and the block stages x through
// LDS in chunks of kChunk k, already in MFMA fragment order (lane l of (k step, token group)
// at 16 l bytes: conflict-free 16-byte reads).  Enough blocks come from splitting K across the
// grid's y dimension (S splits); with S > 1 every split writes fp32 partials [S][M][N] that the
// consumer sums (bias added by split 0), with S = 1 the block writes the rounded output.
//   A = W as in gemm_skinny_kernel (8 weight rows x 128 contiguous bytes per load, streaming);
//   B = x^T token group tg (rows 8 tg + v), read from LDS; D joined by one DPP rotate.
// W keeps four k steps in flight per wave; a load past the block's last step is pointed at x
// (resident in L2) and never used, so the ring's waits stay static.  Measured at 32 rows
// (graph replays, rotating weights) against hipBLASLt: Llama-3-8B wo 9.5 vs 14.0 us, w2 24.6 vs
// 32.8, wqkv 13.7 vs 15.3, merged w1|w3 45.4 vs 45.6 (its transposed layout); depth 2 left
// HBM idle (wo 11.1, w2 31.9) and depth 8 spilled.
constexpr int kChunk = 512;                   // k per staged x chunk
constexpr int kChunkSteps = kChunk / 64;      // 64-wide k steps per chunk
constexpr int kXFrag = kChunkSteps * 4 * 64;  // u32x4 fragments per chunk buffer (32 rows)
static_assert(kChunkSteps % 4 == 0, "the W ring's slots follow the chunk's steps");

struct SplitArgs {
  const uint16_t *x;
  int64_t ldx;
  const uint16_t *w;
  int64_t ldw;
  const uint16_t *bias;
  uint16_t *out;    // S == 1
  int64_t ldo;
  float *part;      // S > 1: [S][M][N]
  int M, N, K, ksplit;  // ksplit: k per split (multiple of 64)
  int inter;        // GLU: out [M][inter] = silu(gate) * up of W = [gate rows; up rows]
};

// GLU (the merged w1|w3 GEMM and SiLU-mul, FeedForward model.py:509-514): NB = 1, unsplit; waves
// 0-3 of block b own gate columns 32 b + [0, 32), waves 4-7 the up columns inter + 32 b + [0, 32),
// and the block writes dtype(dtype(silu(g)) * u) with g and u rounded to the dtype first (what
// the GEMM and then delta_silu_mul compute).
template <int DT, int NB, bool GLU>
__global__ void __launch_bounds__(kGemmWaves * 64) gemm_rows32_kernel(SplitArgs a) {
  using E = Elem<DT>;
  __shared__ u32x4 xs[2][kXFrag];  // 2 x 32 KiB
  constexpr int D = 4;  // k steps of W in flight per wave (8 slots spill, 2 leave HBM idle)
  static_assert(!GLU || NB == 1, "the GLU epilogue pairs one 8-column group per wave");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane >> 4, t = lane & 15;
  const int ncol = GLU ? (wave >= 4 ? a.inter : 0) + blockIdx.x * 32 + (wave & 3) * 8
                       : blockIdx.x * (64 * NB) + wave * (8 * NB);
  const int kb = blockIdx.y * a.ksplit;
  const int ke = min(a.K, kb + a.ksplit);
  const int total = ke > kb ? (ke - kb) / 64 : 0;  // k steps of this split
  const int nchunks = (total + kChunkSteps - 1) / kChunkSteps;

  // x staging: thread i moves 16-byte units u = i + 512 j of the chunk: row u / 64, k8 u % 64.
  u32x4 xr[4];
  auto load_chunk = [&](int ch) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = threadIdx.x + 512 * j;
      const int row = u >> 6, k8 = u & 63;
      const int k = kb + ch * kChunk + 8 * k8;
      xr[j] = (row < a.M && k < ke) ? ld128(a.x + (int64_t)row * a.ldx + k) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = threadIdx.x + 512 * j;
      const int row = u >> 6, k8 = u & 63;
      const int s = k8 >> 3, half = (k8 >> 2) & 1, cc = k8 & 3;
      const int l = 16 * cc + (row & 7) + 8 * half;
      xs[buf][(s * 4 + (row >> 3)) * 64 + l] = xr[j];
    }
  };

  const uint16_t *wp = a.w + (int64_t)(ncol + (t >> 1)) * a.ldw + 32 * (t & 1) + 8 * c + kb;
  u32x4 wf[D][NB];
  auto load_w = [&](int d, int g) {
    const bool in = g < total;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      wf[d][nb] = ld128_stream(in ? wp + (int64_t)nb * 8 * a.ldw + 64 * g : a.x);
  };

  f32x4 acc[NB][4];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int tg = 0; tg < 4; ++tg) acc[nb][tg] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (nchunks > 0) {
    load_chunk(0);
    store_chunk(0);
    if (nchunks > 1) load_chunk(1);
  }
#pragma unroll
  for (int d = 0; d < D; ++d) load_w(d, d);
  __syncthreads();

  for (int ch = 0; ch < nchunks; ++ch) {
    const int buf = ch & 1;
    const int steps = min(kChunkSteps, total - ch * kChunkSteps);
    auto step = [&](int d, int sl) {
      u32x4 xf[4];
#pragma unroll
      for (int tg = 0; tg < 4; ++tg) xf[tg] = xs[buf][(sl * 4 + tg) * 64 + lane];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int tg = 0; tg < 4; ++tg) acc[nb][tg] = E::mfma(wf[d][nb], xf[tg], acc[nb][tg]);
    };
    // Slot d holds step g with g % D == d (a chunk's kChunkSteps is a multiple of D).
    int s0 = 0;
    for (; s0 + D <= steps; s0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        step(d, s0 + d);
        load_w(d, ch * kChunkSteps + s0 + d + D);
      }
    }
    for (int d = 0; s0 + d < steps; ++d) step(d, s0 + d);  // the split's last steps
    if (ch + 1 < nchunks) {
      store_chunk(buf ^ 1);  // its last reader was chunk ch - 1, behind the barrier below
      if (ch + 2 < nchunks) load_chunk(ch + 2);
      __syncthreads();
    }
  }

  // Join the k slices: lane (c, v < 8) holds columns ncol + 8 nb + 2c + {0, 1} of row 8 tg + v.
  if (GLU) {
    // Up waves park dtype(up) in LDS ([32 rows][32 columns], the x buffers are free once every
    // wave left the loop); gate waves finish silu(g) * u and write the block's 32 columns.
    float *upv = reinterpret_cast<float *>(&xs[0][0]);
    __syncthreads();
#pragma unroll
    for (int tg = 0; tg < 4; ++tg) {
      const float s0v = acc[0][tg][0] + dpp_f<0x128>(acc[0][tg][1]);
      const float s1v = acc[0][tg][2] + dpp_f<0x128>(acc[0][tg][3]);
      if (wave >= 4 && t < 8) {
        float *u = upv + (8 * tg + t) * 32 + (wave & 3) * 8 + 2 * c;
        u[0] = E::lo(E::from_float(s0v));
        u[1] = E::lo(E::from_float(s1v));
      }
    }
    __syncthreads();
    if (wave < 4) {
#pragma unroll
      for (int tg = 0; tg < 4; ++tg) {
        const float s0v = acc[0][tg][0] + dpp_f<0x128>(acc[0][tg][1]);
        const float s1v = acc[0][tg][2] + dpp_f<0x128>(acc[0][tg][3]);
        const int row = 8 * tg + t;
        if (t < 8 && row < a.M) {
          const float *u = upv + row * 32 + wave * 8 + 2 * c;
          const float g0 = E::lo(E::from_float(s0v)), g1 = E::lo(E::from_float(s1v));
          const float h0 = E::lo(E::from_float(g0 / (1.f + expf(-g0))));
          const float h1 = E::lo(E::from_float(g1 / (1.f + expf(-g1))));
          const uint32_t pk = E::from_float(h0 * u[0]) | (E::from_float(h1 * u[1]) << 16);
          *reinterpret_cast<uint32_t *>(a.out + (int64_t)row * a.ldo + ncol + 2 * c) = pk;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int tg = 0; tg < 4; ++tg) {
      const float s0v = acc[nb][tg][0] + dpp_f<0x128>(acc[nb][tg][1]);
      const float s1v = acc[nb][tg][2] + dpp_f<0x128>(acc[nb][tg][3]);
      const int row = 8 * tg + t;
      const int col = ncol + 8 * nb + 2 * c;
      if (t < 8 && row < a.M) {
        float v0 = s0v, v1 = s1v;
        if (a.bias && blockIdx.y == 0) {
          v0 += (float)E::lo(a.bias[col]);
          v1 += (float)E::lo(a.bias[col + 1]);
        }
        if (gridDim.y == 1) {
          const uint32_t pk = E::from_float(v0) | (E::from_float(v1) << 16);
          *reinterpret_cast<uint32_t *>(a.out + (int64_t)row * a.ldo + col) = pk;
        } else {
          float *pp = a.part + ((int64_t)blockIdx.y * a.M + row) * a.N + col;
          *reinterpret_cast<float2 *>(pp) = float2{v0, v1};
        }
      }
    }
}

// Splits of a 32-row launch: enough blocks for every CU (N / 64 NB column blocks times S), S a
// divisor of K / 64 so every split holds whole k steps.  Two column groups per wave for the very
// wide (lm_head) and the deep (w2: K >= 8192) weights.
void rows32_plan(int N, int K, int *nb, int *splits) {
  *nb = (N % 128 == 0 && (N / 128 >= 256 || K >= 8192)) ? 2 : 1;
  const int cblocks = N / (64 * *nb);
  const int steps = K / 64;
  int s = 1;
  while (cblocks * s < 256 && s < 16 && steps % (2 * s) == 0) s *= 2;
  *splits = s;
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT int delta_gemm_skinny(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                              const void *bias, void *out, int64_t ldo, int M, int N, int K,
                                              int dtype, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_gemm_skinny";
  if (M <= 0 || N <= 0) return DELTA_OK;
  if (!x || !w || !out) return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: dtype must be bf16 or fp16", who);
  if (K <= 0 || K % 64) return set_error(DELTA_ERR_INVALID, "%s: K (%d) must be a positive multiple of 64", who, K);
  if (N % 16) return set_error(DELTA_ERR_INVALID, "%s: N (%d) must be a multiple of 16", who, N);
  if (ldx < K || ldw < K || ldo < N) return set_error(DELTA_ERR_INVALID, "%s: leading dimensions too small", who);
  if ((ldx % 8) || (ldw % 8) || (((uintptr_t)x | (uintptr_t)w) & 15u))
    return set_error(DELTA_ERR_INVALID, "%s: x and W rows must be 16-byte aligned", who);
  GemmArgs a;
  a.x = (const uint16_t *)x;
  a.ldx = ldx;
  a.w = (const uint16_t *)w;
  a.ldw = ldw;
  a.bias = (const uint16_t *)bias;
  a.out = (uint16_t *)out;
  a.ldo = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  a.kper = (int)(ceil_div(K / 64, kGemmWaves) * 64);
  a.inter = 0;
  // 32 columns per block when that still gives every CU a block, else 16.
  const int nb = (N % 32 == 0 && N / 32 >= 256) ? 4 : 2;
  return dtype == DELTA_BF16 ? launch_gemm<DELTA_BF16>(a, nb, (hipStream_t)stream)
                             : launch_gemm<DELTA_FP16>(a, nb, (hipStream_t)stream);
}

extern "C" DELTA_EXPORT int delta_gemm_rows32_splits(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 || N % 64) return 0;
  int nb, sp;
  delta::rows32_plan(N, K, &nb, &sp);
  return sp;
}

extern "C" DELTA_EXPORT int delta_gemm_rows32(const void *x, int64_t ldx, const void *w, int64_t ldw,
                                              const void *bias, void *out, int64_t ldo, float *partials,
                                              int M, int N, int K, int dtype, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_gemm_rows32";
  if (M <= 0 || N <= 0) return DELTA_OK;
  if (!x || !w) return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (M > 32) return set_error(DELTA_ERR_INVALID, "%s: M (%d) must be <= 32", who, M);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: dtype must be bf16 or fp16", who);
  if (K <= 0 || K % 64) return set_error(DELTA_ERR_INVALID, "%s: K (%d) must be a positive multiple of 64", who, K);
  if (N % 64) return set_error(DELTA_ERR_INVALID, "%s: N (%d) must be a multiple of 64", who, N);
  if (ldx < K || ldw < K) return set_error(DELTA_ERR_INVALID, "%s: leading dimensions too small", who);
  if ((ldx % 8) || (ldw % 8) || (((uintptr_t)x | (uintptr_t)w) & 15u))
    return set_error(DELTA_ERR_INVALID, "%s: x and W rows must be 16-byte aligned", who);
  int nb, sp;
  rows32_plan(N, K, &nb, &sp);
  if (sp == 1) {
    if (!out || ldo < N || (ldo % 2) || ((uintptr_t)out & 3u))
      return set_error(DELTA_ERR_INVALID, "%s: out must be [M, >= N] with 4-byte aligned rows", who);
  } else if (!partials || ((uintptr_t)partials & 7u)) {
    return set_error(DELTA_ERR_INVALID, "%s: this shape needs fp32 partials [%d][M][N] (8-byte aligned)", who, sp);
  }
  SplitArgs a;
  a.x = (const uint16_t *)x;
  a.ldx = ldx;
  a.w = (const uint16_t *)w;
  a.ldw = ldw;
  a.bias = (const uint16_t *)bias;
  a.out = (uint16_t *)out;
  a.ldo = ldo;
  a.part = partials;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ksplit = K / sp;
  a.inter = 0;
  const dim3 grid(N / (64 * nb), sp), block(kGemmWaves * 64);
  if (dtype == DELTA_BF16) {
    if (nb == 2) hipLaunchKernelGGL((gemm_rows32_kernel<DELTA_BF16, 2, false>), grid, block, 0, (hipStream_t)stream, a);
    else hipLaunchKernelGGL((gemm_rows32_kernel<DELTA_BF16, 1, false>), grid, block, 0, (hipStream_t)stream, a);
  } else {
    if (nb == 2) hipLaunchKernelGGL((gemm_rows32_kernel<DELTA_FP16, 2, false>), grid, block, 0, (hipStream_t)stream, a);
    else hipLaunchKernelGGL((gemm_rows32_kernel<DELTA_FP16, 1, false>), grid, block, 0, (hipStream_t)stream, a);
  }
  return check_launch(who);
}

extern "C" DELTA_EXPORT int delta_gemm_rows32_silu(const void *x, int64_t ldx, const void *w13, int64_t ldw, void *out,
                                                   int64_t ldo, int M, int inter, int K, int dtype,
                                                   delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_gemm_rows32_silu";
  if (M <= 0 || inter <= 0) return DELTA_OK;
  if (!x || !w13 || !out) return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (M > 32) return set_error(DELTA_ERR_INVALID, "%s: M (%d) must be <= 32", who, M);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: dtype must be bf16 or fp16", who);
  if (K <= 0 || K % 64) return set_error(DELTA_ERR_INVALID, "%s: K (%d) must be a positive multiple of 64", who, K);
  if (inter % 32) return set_error(DELTA_ERR_INVALID, "%s: inter (%d) must be a multiple of 32", who, inter);
  if (ldx < K || ldw < K || ldo < inter || (ldo % 2) || ((uintptr_t)out & 3u))
    return set_error(DELTA_ERR_INVALID, "%s: leading dimensions too small or out rows not 4-byte aligned", who);
  if ((ldx % 8) || (ldw % 8) || (((uintptr_t)x | (uintptr_t)w13) & 15u))
    return set_error(DELTA_ERR_INVALID, "%s: x and W rows must be 16-byte aligned", who);
  SplitArgs a;
  a.x = (const uint16_t *)x;
  a.ldx = ldx;
  a.w = (const uint16_t *)w13;
  a.ldw = ldw;
  a.bias = nullptr;
  a.out = (uint16_t *)out;
  a.ldo = ldo;
  a.part = nullptr;
  a.M = M;
  a.N = 2 * inter;
  a.K = K;
  a.ksplit = K;
  a.inter = inter;
  const dim3 grid(inter / 32, 1), block(kGemmWaves * 64);
  if (dtype == DELTA_BF16)
    hipLaunchKernelGGL((gemm_rows32_kernel<DELTA_BF16, 1, true>), grid, block, 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((gemm_rows32_kernel<DELTA_FP16, 1, true>), grid, block, 0, (hipStream_t)stream, a);
  return check_launch(who);
}

extern "C" DELTA_EXPORT int delta_gemm_skinny_silu(const void *x, int64_t ldx, const void *w13, int64_t ldw, void *out,
                                                   int64_t ldo, int M, int inter, int K, int dtype,
                                                   delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_gemm_skinny_silu";
  if (M <= 0 || inter <= 0) return DELTA_OK;
  if (!x || !w13 || !out) return set_error(DELTA_ERR_INVALID, "%s: null pointer", who);
  if (M > 8) return set_error(DELTA_ERR_INVALID, "%s: M (%d) must be <= 8", who, M);
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16) return set_error(DELTA_ERR_INVALID, "%s: dtype must be bf16 or fp16", who);
  if (K <= 0 || K % 64) return set_error(DELTA_ERR_INVALID, "%s: K (%d) must be a positive multiple of 64", who, K);
  if (inter % 16) return set_error(DELTA_ERR_INVALID, "%s: inter (%d) must be a multiple of 16", who, inter);
  if (ldx < K || ldw < K || ldo < inter) return set_error(DELTA_ERR_INVALID, "%s: leading dimensions too small", who);
  if ((ldx % 8) || (ldw % 8) || (((uintptr_t)x | (uintptr_t)w13) & 15u))
    return set_error(DELTA_ERR_INVALID, "%s: x and W rows must be 16-byte aligned", who);
  GemmArgs a;
  a.x = (const uint16_t *)x;
  a.ldx = ldx;
  a.w = (const uint16_t *)w13;
  a.ldw = ldw;
  a.bias = nullptr;
  a.out = (uint16_t *)out;
  a.ldo = ldo;
  a.M = M;
  a.N = 2 * inter;
  a.K = K;
  a.kper = (int)(ceil_div(K / 64, kGemmWaves) * 64);
  a.inter = inter;
  // 16 gate + 16 up columns per block, one k step in flight (the launch has inter / 16 blocks)
  const dim3 grid(inter / 16, 1), block(kGemmWaves * 64);
  const size_t lds = kGemmWaves * 8 * 32 * sizeof(float);
  if (dtype == DELTA_BF16)
    hipLaunchKernelGGL((gemm_skinny_kernel<DELTA_BF16, 4, 1, 1, true>), grid, block, lds, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<DELTA_FP16, 4, 1, 1, true>), grid, block, lds, (hipStream_t)stream, a);
  return check_launch(who);
}
