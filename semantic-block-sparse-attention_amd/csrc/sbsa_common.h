// Shared device helpers for the gfx950 kernels of libsbsa.
//
// bf16 values are carried as raw uint16_t bit patterns; conversions are
// explicit (round to nearest even, as torch's .to(torch.bfloat16), in hardware).  MFMA
// operands use clang's __bf16 vector types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sbsa.h"

typedef uint16_t bf16_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

#define SBSA_WAVE 64

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// gfx950 converts with v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN.
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ bf16_t f2bf(float f) {
  __bf16 b = (__bf16)f;
  bf16_t r;
  __builtin_memcpy(&r, &b, 2);
  return r;
}

// fp32 -> bf16 -> fp32 (the value a bf16 tensor would hold).
__device__ __forceinline__ float round_bf16(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ uint32_t pack2bf(float a, float b) {
  bf16x2_t v = __builtin_convertvector(f32x2_t{a, b}, bf16x2_t);
  uint32_t r;
  __builtin_memcpy(&r, &v, 4);
  return r;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  bf16x8_t r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ long long wave_sum_i64(long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// ---- cross-lane reductions on the DPP paths (no LDS round trip) -------------
// Every one of these must run with all 64 lanes of the wave active.
// dpp controls: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_ror:4 = 0x124, row_ror:8 = 0x128, row_shr:n = 0x110 + n.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// max / min / integer sum over a wave; the result is uniform
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  v = fmaxf(v, dpp_f<0x128>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ float wave_min_dpp(float v) {
  v = fminf(v, dpp_f<0xB1>(v));
  v = fminf(v, dpp_f<0x4E>(v));
  v = fminf(v, dpp_f<0x124>(v));
  v = fminf(v, dpp_f<0x128>(v));
  return fminf(fminf(readlane_f(v, 0), readlane_f(v, 16)), fminf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ int wave_sum_i32_dpp(int v) {
  v += dpp_i<0xB1>(v);
  v += dpp_i<0x4E>(v);
  v += dpp_i<0x124>(v);
  v += dpp_i<0x128>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
// float sum over a wave, rows of 16 first, then the four rows in order
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x124>(v);
  v += dpp_f<0x128>(v);
  return ((readlane_f(v, 0) + readlane_f(v, 16)) + readlane_f(v, 32)) + readlane_f(v, 48);
}
// three independent integer sums over a wave, interleaved
__device__ __forceinline__ void wave_sum3_i32_dpp(int& x, int& y, int& z) {
  x += dpp_i<0xB1>(x); y += dpp_i<0xB1>(y); z += dpp_i<0xB1>(z);
  x += dpp_i<0x4E>(x); y += dpp_i<0x4E>(y); z += dpp_i<0x4E>(z);
  x += dpp_i<0x124>(x); y += dpp_i<0x124>(y); z += dpp_i<0x124>(z);
  x += dpp_i<0x128>(x); y += dpp_i<0x128>(y); z += dpp_i<0x128>(z);
  x = (__builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16)) +
      (__builtin_amdgcn_readlane(x, 32) + __builtin_amdgcn_readlane(x, 48));
  y = (__builtin_amdgcn_readlane(y, 0) + __builtin_amdgcn_readlane(y, 16)) +
      (__builtin_amdgcn_readlane(y, 32) + __builtin_amdgcn_readlane(y, 48));
  z = (__builtin_amdgcn_readlane(z, 0) + __builtin_amdgcn_readlane(z, 16)) +
      (__builtin_amdgcn_readlane(z, 32) + __builtin_amdgcn_readlane(z, 48));
}
// three independent integer sums over a wave, the same in every lane: rows of
// 16 by DPP, the two halves by a lane swap, then two rows read out
__device__ __forceinline__ void wave_sum3_i32_swap(int& x, int& y, int& z) {
  x += dpp_i<0xB1>(x); y += dpp_i<0xB1>(y); z += dpp_i<0xB1>(z);
  x += dpp_i<0x4E>(x); y += dpp_i<0x4E>(y); z += dpp_i<0x4E>(z);
  x += dpp_i<0x124>(x); y += dpp_i<0x124>(y); z += dpp_i<0x124>(z);
  x += dpp_i<0x128>(x); y += dpp_i<0x128>(y); z += dpp_i<0x128>(z);
  const auto sx = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
  const auto sy = __builtin_amdgcn_permlane32_swap((uint32_t)y, (uint32_t)y, false, false);
  const auto sz = __builtin_amdgcn_permlane32_swap((uint32_t)z, (uint32_t)z, false, false);
  x = (int)(sx[0] + sx[1]);
  y = (int)(sy[0] + sy[1]);
  z = (int)(sz[0] + sz[1]);
  x = __builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16);
  y = __builtin_amdgcn_readlane(y, 0) + __builtin_amdgcn_readlane(y, 16);
  z = __builtin_amdgcn_readlane(z, 0) + __builtin_amdgcn_readlane(z, 16);
}
// the smallest integer count that reaches a budget: a count c below 2^24 (exact
// in fp32) satisfies (float)c >= budget exactly when c >= ceil(budget)
__device__ __forceinline__ int budget_count(float budget) {
  return (int)ceilf(fminf(budget, 16777216.f));
}
// inclusive prefix sum over the wave (row scans by row_shr, then row carries)
__device__ __forceinline__ int wave_incl_scan_dpp(int v) {
  v += dpp_i<0x111>(v);
  v += dpp_i<0x112>(v);
  v += dpp_i<0x114>(v);
  v += dpp_i<0x118>(v);
  const int r0 = __builtin_amdgcn_readlane(v, 15);
  const int r1 = __builtin_amdgcn_readlane(v, 31);
  const int r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// One prefill work item, 32 bytes: written by the work-list builder and read
// by the attention kernel.  For a cluster item (c >= 0) the builder resolves
// everything the attention needs from the reverse index, so an item costs the
// kernel one load: nkeys = visible rows of the cluster, entry0 = first partial
// slot of the item (rev_indptr + qb), row0 = first packed row of the run.  A
// local item (c < 0) leaves the last three at 0.
struct __attribute__((aligned(32))) PrefillItem {
  int h, c, qb, qn;
  int nkeys, entry0, row0, pad;
};

#define SBSA_CHECK_LAUNCH()                                 \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return SBSA_ERR_LAUNCH; \
  } while (0)
