// Shared device helpers for the gfx950 selective-KV decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/delta_hip.h"

#define DELTA_EXPORT __attribute__((visibility("default")))

namespace delta {

constexpr int kPageSize = 16;
constexpr int kHeadDim = 128;
constexpr int kMaxGroup = 8;  // largest q-heads-per-kv-head the decode kernels instantiate
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Error reporting (thread local), implemented in capi.hip.
int set_error(int code, const char *fmt, ...);
void clear_error();
int check_launch(const char *what);

// ---------------------------------------------------------------------------
// Raw 16-byte vectors and the two MFMA flavours.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ u32x4 ld128(const void *p) {
  return *reinterpret_cast<const u32x4 *>(p);
}
__device__ __forceinline__ void st128(void *p, u32x4 v) { *reinterpret_cast<u32x4 *>(p) = v; }

// Buffer resources for raw buffer stores: linear addressing (stride 0), 32-bit data format in the
// fourth word; cache-policy operand sc1 (agent scope) as the compiler encodes it for gfx950.
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kCpolSc1 = 16;
// Streaming 16-byte load (nontemporal hint): for data read exactly once, such as the K/V
// pages of a decode step.  On MI355X a page gather issued this way sustains ~6.6 TB/s against
// ~5.8 TB/s for plain loads of the same addresses.
__device__ __forceinline__ u32x4 ld128_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// Element conversions for a packed 32-bit pair of 16-bit floats.
template <int DT>
struct Elem;

template <>
struct Elem<DELTA_BF16> {
  __device__ __forceinline__ static float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ __forceinline__ static float hi(uint32_t w) {
    return __uint_as_float(w & 0xffff0000u);
  }
  // IEEE round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
  __device__ __forceinline__ static uint32_t from_float(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  }
  __device__ __forceinline__ static f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Elem<DELTA_FP16> {
  __device__ __forceinline__ static float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  __device__ __forceinline__ static float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  __device__ __forceinline__ static uint32_t from_float(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ __forceinline__ static f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// ---------------------------------------------------------------------------
// Cross-lane reductions inside one 16-lane row of a wave64 (DPP, no LDS).
// quad_perm [1,0,3,2] and [2,3,0,1], then half-row mirror, then row mirror:
// after the four steps every lane holds the reduction of its 16-lane row.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float shfl(float v, int src_lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(v)));
}
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  int lane = __lane_id();
  return shfl(v, lane ^ mask);
}
__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
// Scalar (s_load) read of a word the kernel never writes, at a wave-uniform index: the constant
// address space makes the compiler use the scalar data cache path, whose waits (lgkmcnt) are
// independent of the vector loads in flight.
__device__ __forceinline__ int ld_scalar(const int32_t *p, int64_t i) {
  typedef const __attribute__((address_space(4))) int32_t *cptr;
  return ((cptr)p)[i];
}
__device__ __forceinline__ float ld_scalar(const float *p, int64_t i) {
  typedef const __attribute__((address_space(4))) float *cptr;
  return ((cptr)p)[i];
}

// Wave-wide inclusive prefix sum of a 0/1 flag via ballot (wave64).
__device__ __forceinline__ int wave_prefix_exclusive(bool flag, int *total) {
  uint64_t m = __ballot(flag);
  int lane = __lane_id();
  uint64_t below = lane == 0 ? 0ull : (m & ((~0ull) >> (64 - lane)));
  *total = __popcll(m);
  return __popcll(below);
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Interleaved RoPE (FlashInfer apply_rope / apply_llama31_rope, interleave=True):
// pair (2j, 2j+1) of a head rotates by pos * f_j, f_j = theta^(-2j/128) / rope_scale, or
// for Llama 3.1 the blend (1 - s) f_j / rope_scale + s f_j with
// s = clamp(f_j * smooth_a + smooth_b, 0, 1).  Every kernel that rotates (the RoPE kernels
// and the fused decode attention) calls these two, with contraction off, so each product
// and sum rounds the same way everywhere and the launches agree bit for bit.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rope_cos_sin(int j, float pos, float rcp_scale, float log2_theta, float smooth_a,
                                             float smooth_b, float *cs_sn) {
#pragma clang fp contract(off)
  float f = exp2f(-(2.0f * (float)j / (float)kHeadDim) * log2_theta);  // theta^(-2j/d)
  const float s = fminf(fmaxf(f * smooth_a + smooth_b, 0.f), 1.f);
  f = (1.f - s) * (f * rcp_scale) + s * f;
  float sn, cs;
  sincosf(pos * f, &sn, &cs);
  cs_sn[0] = cs;
  cs_sn[1] = sn;
}

// Rotates one packed pair by (cos, sin) = (cs_sn[0], cs_sn[1]); fp32 math, one rounding.
template <int DT>
__device__ __forceinline__ uint32_t rope_rotate(uint32_t pr, const float *cs_sn) {
#pragma clang fp contract(off)
  using E = Elem<DT>;
  const float cs = cs_sn[0], sn = cs_sn[1];
  const float x0 = E::lo(pr), x1 = E::hi(pr);
  const float y0 = x0 * cs - x1 * sn;
  const float y1 = x1 * cs + x0 * sn;
  return E::from_float(y0) | (E::from_float(y1) << 16);
}

}  // namespace delta
