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

#define SBSA_CHECK_LAUNCH()                                 \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return SBSA_ERR_LAUNCH; \
  } while (0)
