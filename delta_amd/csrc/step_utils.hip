// Per-row argmax for the graph-captured decode step.
//
// Replaces torch.argmax(logits, -1) of _finalize_logits (hoenza/DELTA
// model.py:320-323) inside the decode hipGraph: one block per row, the first
// index of the maximum (torch.argmax's rule), NaN counted as the maximum.  A
// plain single-pass kernel, so the captured step records no memset node.
#include "delta_common.h"

namespace delta {
namespace {

template <int DT>
__global__ void __launch_bounds__(1024) argmax_rows_kernel(const uint16_t *logits, int64_t stride, int cols,
                                                             int64_t *out, int64_t out_stride) {
  using E = Elem<DT>;
  __shared__ float s_val[16];
  __shared__ int s_idx[16];
  const int r = blockIdx.x;
  const uint16_t *row = logits + (int64_t)r * stride;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    const uint32_t w = row[c];
    const float v = E::lo(w);
    const bool take = (v != v) ? !(best != best) : (v > best);  // first NaN wins, else strictly greater
    if (take || (bi == 0x7fffffff)) {
      best = v;
      bi = c;
    }
  }
  // (value desc, index asc) reduction; NaN ranks highest.
  auto better = [](float v1, int i1, float v2, int i2) {
    const bool n1 = v1 != v1, n2 = v2 != v2;
    if (n1 != n2) return n1;
    if (!n1 && v1 != v2) return v1 > v2;
    return i1 < i2;
  };
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
    out[(int64_t)r * out_stride] = bi == 0x7fffffff ? 0 : bi;
  }
}

}  // namespace
}  // namespace delta

extern "C" DELTA_EXPORT int delta_argmax_rows(const void *logits, int64_t row_stride, int rows, int cols,
                                              int dtype, int64_t *out, int64_t out_stride,
                                              delta_stream_t stream) {
  using namespace delta;
  clear_error();
  if (rows <= 0) return DELTA_OK;
  if (!logits || !out || cols <= 0) return set_error(DELTA_ERR_INVALID, "delta_argmax_rows: bad arguments");
  if (dtype == DELTA_BF16)
    hipLaunchKernelGGL(argmax_rows_kernel<DELTA_BF16>, dim3(rows), dim3(1024), 0, (hipStream_t)stream,
                       (const uint16_t *)logits, row_stride, cols, out, out_stride);
  else if (dtype == DELTA_FP16)
    hipLaunchKernelGGL(argmax_rows_kernel<DELTA_FP16>, dim3(rows), dim3(1024), 0, (hipStream_t)stream,
                       (const uint16_t *)logits, row_stride, cols, out, out_stride);
  else
    return set_error(DELTA_ERR_INVALID, "delta_argmax_rows: dtype must be bf16 or fp16");
  return check_launch("delta_argmax_rows");
}
