// Dense decode-step helpers for the captured gfx950 decode step.
//
// The dense half of a decode layer (model.py:330-359, 495-532) is torch ops in the
// reference; here the element-wise chains between the GEMMs are single kernels so a
// captured step is not dominated by ~16 tiny launches per layer:
//   add_rmsnorm : h = x + r (bf16), y = bf16(bf16(h * rsqrt(mean(h^2) + eps)) * w)
//                 -- RMSNorm.forward (model.py:527-532) fused with the residual add
//                    of TransformerBlock.forward (model.py:338-341);
//   silu_mul    : y = bf16(bf16(silu(g)) * u) -- FeedForward w2's input (model.py:509-514);
//   argmax_rows : torch.argmax(logits, -1) of _finalize_logits (model.py:320-323), two
//                 passes (row chunks, then per row), no memset.
// Each kernel rounds where the reference's bf16 tensor ops round.
#include <type_traits>

#include "delta_common.h"

namespace delta {
namespace {

constexpr int kNormThreads = 256;

// PS > 0: the residual is the sum of PS fp32 partials (a split-K GEMM's, [PS][rows][dim] with
// split stride ps), rounded to the dtype once -- the value the unsplit GEMM would have written.
// All PS loads of a chunk are issued before the first add (one round trip, not PS).
template <int DT, int PS>
__global__ void __launch_bounds__(kNormThreads)
    add_rmsnorm_kernel(const uint16_t *x, int64_t xs, const uint16_t *r, int64_t rs, const uint16_t *w,
                       float eps, uint16_t *h_out, int64_t hs, uint16_t *y, int64_t ys, int dim,
                       const float *part, int64_t ps) {
  // No contraction: every product is rounded where the reference's ops round it (a fused
  // multiply-round would also differ between the instantiations).
#pragma clang fp contract(off)
  constexpr bool PART = PS > 0;
  using E = Elem<DT>;
  __shared__ float red[kNormThreads / 64];
  const int row = blockIdx.x;
  const uint16_t *xr = x + (int64_t)row * xs;
  const uint16_t *rr = PART ? nullptr : (r ? r + (int64_t)row * rs : nullptr);
  const float *pr = PART ? part + (int64_t)row * dim : nullptr;
  constexpr int kMaxChunks = 4;  // 8 elements per chunk -> dim <= 8192
  float hv[kMaxChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxChunks; ++k) {
    const int c0 = (threadIdx.x + k * kNormThreads) * 8;
    if (c0 < dim) {
      const u32x4 a = ld128(xr + c0);
      u32x4 o;
      if (PART) {
        f32x4 pv[PS > 0 ? PS : 1][2];
#pragma unroll
        for (int sp = 0; sp < PS; ++sp) {
          pv[sp][0] = *reinterpret_cast<const f32x4 *>(pr + sp * ps + c0);
          pv[sp][1] = *reinterpret_cast<const f32x4 *>(pr + sp * ps + c0 + 4);
        }
        float rs8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) rs8[e] = 0.f;
#pragma unroll
        for (int sp = 0; sp < PS; ++sp)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            rs8[e] += pv[sp][0][e];
            rs8[4 + e] += pv[sp][1][e];
          }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float r0 = E::lo(E::from_float(rs8[2 * q])), r1 = E::lo(E::from_float(rs8[2 * q + 1]));
          const uint32_t lo = E::from_float(E::lo(a[q]) + r0);
          const uint32_t hi = E::from_float(E::hi(a[q]) + r1);
          o[q] = lo | (hi << 16);
        }
      } else if (rr) {
        const u32x4 bb = ld128(rr + c0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = E::from_float(E::lo(a[q]) + E::lo(bb[q]));
          const uint32_t hi = E::from_float(E::hi(a[q]) + E::hi(bb[q]));
          o[q] = lo | (hi << 16);
        }
      } else {
        o = a;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        hv[k][2 * q] = E::lo(o[q]);
        hv[k][2 * q + 1] = E::hi(o[q]);
        ss = fmaf(hv[k][2 * q], hv[k][2 * q], ss);
        ss = fmaf(hv[k][2 * q + 1], hv[k][2 * q + 1], ss);
      }
      if (h_out && (PART || rr)) st128(h_out + (int64_t)row * hs + c0, o);
    }
  }
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
  const float inv = rsqrtf(tot / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < kMaxChunks; ++k) {
    const int c0 = (threadIdx.x + k * kNormThreads) * 8;
    if (c0 < dim) {
      const u32x4 wv = ld128(w + c0);
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // h * inv is rounded to fp32 and then to the dtype, as the reference's fp32 RMSNorm
        // followed by type_as does; the empty asm keeps the fp16 conversion from being folded
        // into one mixed-precision fma (a single rounding, taken for some elements only).
        float m0 = hv[k][2 * q] * inv, m1 = hv[k][2 * q + 1] * inv;
        asm volatile("" : "+v"(m0), "+v"(m1));
        const float n0 = E::lo(E::from_float(m0));
        const float n1 = E::lo(E::from_float(m1));
        o[q] = E::from_float(n0 * E::lo(wv[q])) | (E::from_float(n1 * E::hi(wv[q])) << 16);
      }
      st128(y + (int64_t)row * ys + c0, o);
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint16_t *gu, int64_t gs, uint16_t *y, int64_t ys,
                                                        int inter) {
  using E = Elem<DT>;
  const int row = blockIdx.y;
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c0 >= inter) return;
  const u32x4 g = ld128(gu + (int64_t)row * gs + c0);
  const u32x4 u = ld128(gu + (int64_t)row * gs + inter + c0);
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float g0 = E::lo(g[q]), g1 = E::hi(g[q]);
    const float s0 = E::lo(E::from_float(g0 / (1.f + expf(-g0))));
    const float s1 = E::lo(E::from_float(g1 / (1.f + expf(-g1))));
    o[q] = E::from_float(s0 * E::lo(u[q])) | (E::from_float(s1 * E::hi(u[q])) << 16);
  }
  st128(y + (int64_t)row * ys + c0, o);
}

// (value desc, index asc); NaN ranks highest (torch.argmax treats NaN as the maximum).
__device__ __forceinline__ bool better(float v1, int i1, float v2, int i2) {
  const bool n1 = v1 != v1, n2 = v2 != v2;
  if (n1 != n2) return n1;
  if (!n1 && v1 != v2) return v1 > v2;
  return i1 < i2;
}

__device__ __forceinline__ void block_best(float &best, int &bi, float *s_val, int *s_idx) {
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(bi, off);
    if (better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_val[wave] = best;
    s_idx[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int nw = (blockDim.x + 63) >> 6;
    for (int w = 1; w < nw; ++w)
      if (better(s_val[w], s_idx[w], best, bi)) {
        best = s_val[w];
        bi = s_idx[w];
      }
  }
}

constexpr int kArgChunks = 32;

template <int DT>
__global__ void __launch_bounds__(256) argmax_chunk_kernel(const uint16_t *logits, int64_t stride, int cols,
                                                            float *ws_val, int *ws_idx) {
  using E = Elem<DT>;
  __shared__ float s_val[4];
  __shared__ int s_idx[4];
  const int r = blockIdx.y;
  const int per = (cols + kArgChunks - 1) / kArgChunks;
  const int c_beg = blockIdx.x * per;
  const int c_end = min(cols, c_beg + per);
  const uint16_t *row = logits + (int64_t)r * stride;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int c = c_beg + threadIdx.x; c < c_end; c += 256) {
    const float v = E::lo(row[c]);
    if (bi == 0x7fffffff || better(v, c, best, bi)) {
      best = v;
      bi = c;
    }
  }
  block_best(best, bi, s_val, s_idx);
  if (threadIdx.x == 0) {
    ws_val[r * kArgChunks + blockIdx.x] = best;
    ws_idx[r * kArgChunks + blockIdx.x] = bi;
  }
}

__global__ void __launch_bounds__(64) argmax_final_kernel(const float *ws_val, const int *ws_idx, int64_t *out,
                                                           int64_t out_stride) {
  const int r = blockIdx.x;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  if (threadIdx.x < kArgChunks) {
    best = ws_val[r * kArgChunks + threadIdx.x];
    bi = ws_idx[r * kArgChunks + threadIdx.x];
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(bi, off);
    if (better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  if (threadIdx.x == 0) out[(int64_t)r * out_stride] = bi == 0x7fffffff ? 0 : bi;
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT size_t delta_argmax_workspace_bytes(int rows) {
  return (size_t)rows * delta::kArgChunks * (sizeof(float) + sizeof(int));
}

extern "C" DELTA_EXPORT int delta_argmax_rows(const void *logits, int64_t row_stride, int rows, int cols,
                                              int dtype, int64_t *out, int64_t out_stride, void *workspace,
                                              size_t workspace_bytes, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  if (rows <= 0) return DELTA_OK;
  if (!logits || !out || cols <= 0) return set_error(DELTA_ERR_INVALID, "delta_argmax_rows: bad arguments");
  if (dtype != DELTA_BF16 && dtype != DELTA_FP16)
    return set_error(DELTA_ERR_INVALID, "delta_argmax_rows: dtype must be bf16 or fp16");
  const size_t need = delta_argmax_workspace_bytes(rows);
  if (!workspace || workspace_bytes < need)
    return set_error(DELTA_ERR_WORKSPACE, "delta_argmax_rows: workspace of %zu bytes needed", need);
  float *wv = (float *)workspace;
  int *wi = (int *)((char *)workspace + (size_t)rows * kArgChunks * sizeof(float));
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(kArgChunks, rows);
  if (dtype == DELTA_BF16)
    hipLaunchKernelGGL(argmax_chunk_kernel<DELTA_BF16>, grid, dim3(256), 0, st, (const uint16_t *)logits,
                       row_stride, cols, wv, wi);
  else
    hipLaunchKernelGGL(argmax_chunk_kernel<DELTA_FP16>, grid, dim3(256), 0, st, (const uint16_t *)logits,
                       row_stride, cols, wv, wi);
  int rc = check_launch("delta_argmax_rows");
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, st, wv, wi, out, out_stride);
  return check_launch("delta_argmax_rows");
}

extern "C" DELTA_EXPORT int delta_add_rmsnorm(const void *x, int64_t x_stride, const void *residual,
                                              int64_t r_stride, const void *weight, float eps, void *sum_out,
                                              int64_t s_stride, void *out, int64_t out_stride, int rows, int dim,
                                              int dtype, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  if (rows <= 0) return DELTA_OK;
  if (!x || !weight || !out || dim <= 0 || dim % 8 || dim > 8 * 4 * kNormThreads)
    return set_error(DELTA_ERR_INVALID, "delta_add_rmsnorm: bad arguments (dim %% 8 == 0, dim <= 8192)");
  if (((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)residual | (uintptr_t)sum_out) & 15u ||
      (x_stride | r_stride | s_stride | out_stride) & 7)
    return set_error(DELTA_ERR_INVALID, "delta_add_rmsnorm: 16-byte aligned rows required");
  if (dtype == DELTA_BF16)
    hipLaunchKernelGGL((add_rmsnorm_kernel<DELTA_BF16, 0>), dim3(rows), dim3(kNormThreads), 0, (hipStream_t)stream,
                       (const uint16_t *)x, x_stride, (const uint16_t *)residual, r_stride,
                       (const uint16_t *)weight, eps, (uint16_t *)sum_out, s_stride, (uint16_t *)out, out_stride,
                       dim, nullptr, 0);
  else if (dtype == DELTA_FP16)
    hipLaunchKernelGGL((add_rmsnorm_kernel<DELTA_FP16, 0>), dim3(rows), dim3(kNormThreads), 0, (hipStream_t)stream,
                       (const uint16_t *)x, x_stride, (const uint16_t *)residual, r_stride,
                       (const uint16_t *)weight, eps, (uint16_t *)sum_out, s_stride, (uint16_t *)out, out_stride,
                       dim, nullptr, 0);
  else
    return set_error(DELTA_ERR_INVALID, "delta_add_rmsnorm: bad dtype");
  return check_launch("delta_add_rmsnorm");
}

extern "C" DELTA_EXPORT int delta_silu_mul(const void *gate_up, int64_t gu_stride, void *out, int64_t out_stride,
                                           int rows, int inter, int dtype, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  if (rows <= 0) return DELTA_OK;
  if (!gate_up || !out || inter <= 0 || inter % 8) return set_error(DELTA_ERR_INVALID, "delta_silu_mul: bad arguments");
  if (((uintptr_t)gate_up | (uintptr_t)out) & 15u || (gu_stride | out_stride) & 7)
    return set_error(DELTA_ERR_INVALID, "delta_silu_mul: 16-byte aligned rows required");
  dim3 grid((unsigned)ceil_div(inter, 256 * 8), rows);
  if (dtype == DELTA_BF16)
    hipLaunchKernelGGL(silu_mul_kernel<DELTA_BF16>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)gate_up, gu_stride, (uint16_t *)out, out_stride, inter);
  else if (dtype == DELTA_FP16)
    hipLaunchKernelGGL(silu_mul_kernel<DELTA_FP16>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)gate_up, gu_stride, (uint16_t *)out, out_stride, inter);
  else
    return set_error(DELTA_ERR_INVALID, "delta_silu_mul: bad dtype");
  return check_launch("delta_silu_mul");
}

extern "C" DELTA_EXPORT int delta_add_rmsnorm_partials(const void *x, int64_t x_stride, const float *partials,
                                                       int nsplit, const void *weight, float eps, void *sum_out,
                                                       int64_t s_stride, void *out, int64_t out_stride, int rows,
                                                       int dim, int dtype, delta_stream_t stream) {
  using namespace delta;
  clear_error();
  const char *who = "delta_add_rmsnorm_partials";
  if (rows <= 0) return DELTA_OK;
  if (!x || !partials || !weight || !out || dim <= 0 || dim % 8 || dim > 8 * 4 * kNormThreads)
    return set_error(DELTA_ERR_INVALID, "%s: bad arguments (dim %% 8 == 0, dim <= 8192)", who);
  if (nsplit != 2 && nsplit != 4 && nsplit != 8 && nsplit != 16)
    return set_error(DELTA_ERR_INVALID, "%s: nsplit must be 2, 4, 8 or 16 (delta_gemm_rows32's splits)", who);
  if (((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)sum_out | (uintptr_t)partials) & 15u ||
      (x_stride | s_stride | out_stride) & 7)
    return set_error(DELTA_ERR_INVALID, "%s: 16-byte aligned rows required", who);
  const int64_t ps = (int64_t)rows * dim;
  auto launch = [&](auto dt_tag, auto ps_tag) {
    constexpr int DT = decltype(dt_tag)::value, PSN = decltype(ps_tag)::value;
    hipLaunchKernelGGL((add_rmsnorm_kernel<DT, PSN>), dim3(rows), dim3(kNormThreads), 0, (hipStream_t)stream,
                       (const uint16_t *)x, x_stride, nullptr, 0, (const uint16_t *)weight, eps, (uint16_t *)sum_out,
                       s_stride, (uint16_t *)out, out_stride, dim, partials, ps);
  };
  auto by_splits = [&](auto dt_tag) {
    switch (nsplit) {
      case 2: launch(dt_tag, std::integral_constant<int, 2>{}); break;
      case 4: launch(dt_tag, std::integral_constant<int, 4>{}); break;
      case 8: launch(dt_tag, std::integral_constant<int, 8>{}); break;
      default: launch(dt_tag, std::integral_constant<int, 16>{}); break;
    }
  };
  if (dtype == DELTA_BF16) by_splits(std::integral_constant<int, DELTA_BF16>{});
  else if (dtype == DELTA_FP16) by_splits(std::integral_constant<int, DELTA_FP16>{});
  else return set_error(DELTA_ERR_INVALID, "%s: bad dtype", who);
  return check_launch(who);
}
