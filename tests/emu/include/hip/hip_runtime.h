// A CPU stand-in for the part of the HIP runtime and of the gfx950 builtins that
// libsbsa's kernels use, so that the library's own .hip sources (after the
// mechanical rewrite of tests/emu/transform.py) compile for the host and run
// there.  Test infrastructure only: the product library is built with hipcc.
//
// Execution model: a launch runs its blocks one after another; each block's
// threads are host threads.  Cross-lane operations (readfirstlane, DPP, MFMA,
// transposing LDS reads, ...) are collective over the 64 lanes of a wave.
// Loads straight into LDS are queued per wave and land only when a s_waitcnt
// lets the wave's count of outstanding vector-memory operations drop, so a
// missing or too loose wait shows up as stale LDS data.  Every buffer-resource
// and LDS-DMA access is checked against the allocations the address sanitizer
// knows (when the library is built with it), as a GPU memory fault would be.
#pragma once

#include <stdint.h>
#include <cmath>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>
#include <tuple>

// ---------------------------------------------------------------- qualifiers
#define __global__
#define __device__
#define __host__
#define __forceinline__ inline __attribute__((always_inline))
#define __launch_bounds__(...)
#define __shared__ static
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) ((const void*)&(x))

typedef int hipError_t;
typedef void* hipStream_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1 };
enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 16 };
enum hipMemcpyKind { hipMemcpyHostToHost = 0, hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2,
                     hipMemcpyDeviceToDevice = 3, hipMemcpyDefault = 4 };

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct emu_uint3 {
  unsigned x, y, z;
};
extern thread_local emu_uint3 threadIdx, blockIdx, blockDim, gridDim;

typedef __attribute__((ext_vector_type(4))) short emu_s16x4_t;

namespace emu {

// ---- the collective primitives (emu_runtime.cpp) ----------------------------
int lane();
int wave();
// all 64 lanes post `bytes` of `in`; `fn(get)` runs in every lane after the
// rendezvous, get(l) giving lane l's bytes; a second rendezvous follows
void wave_exchange(const void* in, int bytes, void* all_out /* [64][bytes] */);
void block_barrier();
int block_or(int v);
void* dyn_lds();
// a static LDS array of the kernel: filled with stale bytes once per block
void shared_var(const void* p, size_t bytes);
// vector-memory queue
void buffer_load_lds(uint32_t rsrc[4], uint32_t lds_addr, uint32_t voffset, int size);
void global_load_lds(const void* gptr, const void* lds_ptr, int size, int offset);
void buffer_store(uint32_t rsrc[4], int voffset, const void* data, int size);
void waitcnt(unsigned imm);
void check_global(const void* p, size_t n, const char* what);
void fail(const char* fmt, ...);

// every lane's posted value, read in place from the wave's slot bank (stable
// until every lane has moved on to the operation after the next)
const unsigned char* wave_post(const void* in, int bytes);
constexpr int kSlotBytes = 128;
template <class T>
struct LaneView {
  const unsigned char* base;
  T operator[](int l) const {
    T v;
    memcpy(&v, base + (size_t)l * kSlotBytes, sizeof(T));
    return v;
  }
};
template <class T>
__forceinline__ LaneView<T> gather(const T& v) {
  static_assert(sizeof(T) <= kSlotBytes, "wave slot");
  return LaneView<T>{wave_post(&v, sizeof(T))};
}
template <class T>
__forceinline__ void gather(const T& v, T (&all)[64]) {
  const LaneView<T> view = gather(v);
  for (int l = 0; l < 64; ++l) all[l] = view[l];
}

// a rendezvous of the wave's 64 lanes: the emulation's stand-in for the
// lockstep execution a wave has on the GPU (where the builtin only orders the
// compiler's memory operations), at points where lanes hand data to each other
// through LDS
__forceinline__ void wave_sync() {
  const int d = 0;
  wave_post(&d, sizeof(int));
}

template <class T>
__forceinline__ T readfirstlane(T v) {
  return gather(v)[0];
}
template <class T>
__forceinline__ T readlane(T v, int l) {
  return gather(v)[l & 63];
}
__forceinline__ unsigned long long ballot(bool p) {
  const auto all = gather((int)p);
  unsigned long long m = 0;
  for (int l = 0; l < 64; ++l)
    if (all[l]) m |= 1ull << l;
  return m;
}
template <class T>
__forceinline__ T shfl(T v, int src, int width = 64) {
  const auto all = gather(v);
  const int l = lane();
  const int base = l - l % width;
  return all[base + ((src % width) + width) % width];
}
template <class T>
__forceinline__ T shfl_xor(T v, int m, int width = 64) {
  const auto all = gather(v);
  const int l = lane();
  const int s = l ^ m;
  return (s / width == l / width) ? all[s] : v;
}
template <class T>
__forceinline__ T shfl_up(T v, unsigned d, int width = 64) {
  const auto all = gather(v);
  const int l = lane();
  const int s = l - (int)d;
  return (s >= l - l % width) ? all[s] : v;
}
// DPP: quad_perm (ctrl < 0x100), row_shl (0x101-0x10F), row_shr (0x111-0x11F),
// row_ror (0x121-0x12F); the source lane outside the row reads `old`, or 0
// with bound_ctrl; row_mask / bank_mask are all ones in this library
__forceinline__ int update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
  if (row_mask != 0xf || bank_mask != 0xf) fail("update_dpp: partial masks are not emulated");
  const auto all = gather(src);
  const int l = lane();
  const int row = l & ~15, i = l & 15;
  int s = -1;
  if (ctrl < 0x100) {
    s = (l & ~3) + ((ctrl >> (2 * (l & 3))) & 3);
  } else if (ctrl >= 0x101 && ctrl <= 0x10F) {
    const int n = ctrl - 0x100;
    s = (i + n < 16) ? row + i + n : -1;
  } else if (ctrl >= 0x111 && ctrl <= 0x11F) {
    const int n = ctrl - 0x110;
    s = (i - n >= 0) ? row + i - n : -1;
  } else if (ctrl >= 0x121 && ctrl <= 0x12F) {
    const int n = ctrl - 0x120;
    s = row + ((i - n) & 15);
  } else {
    fail("update_dpp: control 0x%x is not emulated", ctrl);
  }
  if (s < 0) return bound_ctrl ? 0 : old;
  return all[s];
}
// v_permlane32_swap: (vdst, vsrc) -> lanes 32..63 of vdst swapped with lanes 0..31 of vsrc
struct u32pair {
  uint32_t v[2];
  uint32_t operator[](int i) const { return v[i]; }
};
__forceinline__ u32pair permlane32_swap(uint32_t vdst, uint32_t vsrc, bool, bool) {
  struct Two {
    uint32_t v[2];
  } both{{vdst, vsrc}};
  const auto all = gather(both);
  const int l = lane();
  u32pair r;
  if (l < 32) {
    r.v[0] = all[l].v[0];
    r.v[1] = all[l + 32].v[0];
  } else {
    r.v[0] = all[l - 32].v[1];
    r.v[1] = all[l].v[1];
  }
  return r;
}
// ds_read_b64_tr_b16: lane 16 g + i receives element i % 4 of the 64-bit words
// addressed by lanes 16 g + i / 4 + 4 e, e = 0..3
__forceinline__ emu_s16x4_t ds_read_tr16_b64(const void* p) {
  const auto all = gather(p);
  const int l = lane();
  const int g = l >> 4, i = l & 15;
  emu_s16x4_t r;
  for (int e = 0; e < 4; ++e) {
    const int16_t* w = reinterpret_cast<const int16_t*>(all[16 * g + i / 4 + 4 * e]);
    r[e] = w[i % 4];
  }
  return r;
}
float bf16_to_float(uint16_t h);
// MFMA 32x32x16 bf16: A lane l = row l % 32, k 8 (l / 32) ..; B lane l = column
// l % 32, k 8 (l / 32) ..; D lane l, r = row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32
template <class V8, class V16>
__forceinline__ V16 mfma32x32x16(V8 a, V8 b, V16 c) {
  struct In {
    uint16_t a[8], b[8];
  } in;
  __builtin_memcpy(in.a, &a, 16);
  __builtin_memcpy(in.b, &b, 16);
  const auto all = gather(in);
  const int l = lane();
  const int col = l % 32;
  float bcol[16];
  for (int kh = 0; kh < 2; ++kh) {
    const In x = all[col + 32 * kh];
    for (int j = 0; j < 8; ++j) bcol[8 * kh + j] = bf16_to_float(x.b[j]);
  }
  V16 d;
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r / 4) + 4 * (l / 32) + r % 4;
    double s = c[r];
    for (int kh = 0; kh < 2; ++kh) {
      const In x = all[row + 32 * kh];
      for (int j = 0; j < 8; ++j) s += (double)bf16_to_float(x.a[j]) * (double)bcol[8 * kh + j];
    }
    d[r] = (float)s;
  }
  return d;
}
// MFMA 16x16x32 bf16: A lane l = row l % 16, k 8 (l / 16) ..; B lane l = column
// l % 16; D lane l, r = row 4 (l / 16) + r, column l % 16
template <class V8, class V4>
__forceinline__ V4 mfma16x16x32(V8 a, V8 b, V4 c) {
  struct In {
    uint16_t a[8], b[8];
  } in;
  __builtin_memcpy(in.a, &a, 16);
  __builtin_memcpy(in.b, &b, 16);
  const auto all = gather(in);
  const int l = lane();
  const int col = l % 16;
  float bcol[32];
  for (int kq = 0; kq < 4; ++kq) {
    const In x = all[col + 16 * kq];
    for (int j = 0; j < 8; ++j) bcol[8 * kq + j] = bf16_to_float(x.b[j]);
  }
  V4 d;
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * (l / 16) + r;
    double s = c[r];
    for (int kq = 0; kq < 4; ++kq) {
      const In x = all[row + 16 * kq];
      for (int j = 0; j < 8; ++j) s += (double)bf16_to_float(x.a[j]) * (double)bcol[8 * kq + j];
    }
    d[r] = (float)s;
  }
  return d;
}

// buffer resources built by __builtin_amdgcn_make_buffer_rsrc
struct rsrc_t {
  uint32_t w[4];
};
__forceinline__ rsrc_t make_rsrc(const void* p, short stride, int num, int flags) {
  const uint64_t b = (uint64_t)p;
  rsrc_t r;
  r.w[0] = (uint32_t)b;
  r.w[1] = ((uint32_t)(b >> 32) & 0xffffu) | ((uint32_t)(uint16_t)stride << 16);
  r.w[2] = (uint32_t)num;
  r.w[3] = (uint32_t)flags;
  return r;
}
template <class T>
__forceinline__ void raw_buffer_store(T v, rsrc_t r, int voffset, int soffset) {
  buffer_store(r.w, voffset + soffset, &v, sizeof(T));
}

}  // namespace emu

// ---- the builtins, mapped onto the emulation -----------------------------------
#define __builtin_amdgcn_readfirstlane(x) emu::readfirstlane(x)
#define __builtin_amdgcn_readlane(x, l) emu::readlane((x), (l))
#define __builtin_amdgcn_update_dpp(o, s, c, rm, bm, bc) emu::update_dpp((o), (s), (c), (rm), (bm), (bc))
#define __builtin_amdgcn_permlane32_swap(a, b, f, c) emu::permlane32_swap((a), (b), (f), (c))
#define __builtin_amdgcn_ds_read_tr16_b64_v4i16(p) emu::ds_read_tr16_b64((const void*)(p))
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, x, y, z) emu::mfma32x32x16((a), (b), (c))
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, x, y, z) emu::mfma16x16x32((a), (b), (c))
#define __builtin_amdgcn_exp2f(x) exp2f(x)
#define __builtin_amdgcn_logf(x) log2f(x)
#define __builtin_amdgcn_s_waitcnt(x) emu::waitcnt((unsigned)(x))
#define __builtin_amdgcn_sched_barrier(x) ((void)0)
#define __builtin_amdgcn_sched_group_barrier(a, b, c) ((void)0)
#define __builtin_amdgcn_wave_barrier() emu::wave_sync()
#define __builtin_amdgcn_fence(...) std::atomic_thread_fence(std::memory_order_seq_cst)
#define __builtin_amdgcn_global_load_lds(g, l, size, off, aux) \
  emu::global_load_lds((const void*)(g), (const void*)(l), (size), (off))
#define __builtin_amdgcn_make_buffer_rsrc(p, stride, num, flags) emu::make_rsrc((p), (stride), (num), (flags))
#define __builtin_amdgcn_raw_buffer_store_b128(v, r, vo, so, aux) emu::raw_buffer_store((v), (r), (vo), (so))
#define __builtin_amdgcn_raw_buffer_store_b32(v, r, vo, so, aux) emu::raw_buffer_store((v), (r), (vo), (so))
typedef emu::rsrc_t __amdgpu_buffer_rsrc_t;

#include <atomic>

#define __ballot(p) emu::ballot(p)
#define __shfl(v, s, ...) emu::shfl((v), (s), ##__VA_ARGS__)
#define __shfl_xor(v, m, ...) emu::shfl_xor((v), (m), ##__VA_ARGS__)
#define __shfl_up(v, d, ...) emu::shfl_up((v), (d), ##__VA_ARGS__)
inline void __syncthreads() { emu::block_barrier(); }
inline int __syncthreads_or(int p) { return emu::block_or(p); }

inline float __uint_as_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
inline uint32_t __float_as_uint(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
inline float __int_as_float(int u) { float f; memcpy(&f, &u, 4); return f; }
inline int __float_as_int(float f) { int u; memcpy(&u, &f, 4); return u; }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int __ffsll(long long v) { return __builtin_ffsll(v); }

template <class T, class U>
inline T atomicAdd(T* p, U v) { return __atomic_fetch_add(p, (T)v, __ATOMIC_SEQ_CST); }
template <class T, class U>
inline T atomicMin(T* p, U v) {
  T cur = __atomic_load_n(p, __ATOMIC_SEQ_CST);
  while ((T)v < cur && !__atomic_compare_exchange_n(p, &cur, (T)v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST)) {
  }
  return cur;
}
template <class T, class U>
inline T atomicOr(T* p, U v) { return __atomic_fetch_or(p, (T)v, __ATOMIC_SEQ_CST); }
#define __HIP_MEMORY_SCOPE_AGENT 0
#define __hip_atomic_load(p, order, scope) __atomic_load_n((p), __ATOMIC_SEQ_CST)

template <class A, class B>
inline typename std::common_type<A, B>::type min(A a, B b) { return a < b ? a : b; }
template <class A, class B>
inline typename std::common_type<A, B>::type max(A a, B b) { return a > b ? a : b; }

// ---- the runtime calls the library makes ----------------------------------------
namespace emu {
using kernel_body = void (*)(void*);
void run_grid(dim3 grid, dim3 block, size_t lds, void (*body)(void*), void* ctx, const void* fn);
template <class... P, class... A>
void launch(void (*k)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t, A&&... args) {
  struct Ctx {
    void (*k)(P...);
    std::tuple<typename std::decay<P>::type...> params;
  } ctx{k, std::tuple<typename std::decay<P>::type...>(std::forward<A>(args)...)};
  run_grid(grid, block, lds, [](void* c) {
    Ctx* x = static_cast<Ctx*>(c);
    std::apply(x->k, x->params);
  }, &ctx, (const void*)k);
}
}  // namespace emu

#define hipLaunchKernelGGL(...) emu::launch(__VA_ARGS__)
inline hipError_t hipFuncSetAttribute(const void*, hipFuncAttribute, int) { return hipSuccess; }
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) { *v = 4; return hipSuccess; }
inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, const void*, int, size_t) { *n = 1; return hipSuccess; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) {
  memcpy(d, s, n);
  return hipSuccess;
}
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) { *p = const_cast<void*>(sym); return hipSuccess; }
template <class T>
inline hipError_t hipMalloc(T** p, size_t n) { *p = static_cast<T*>(malloc(n)); return *p ? hipSuccess : 2; }
inline hipError_t hipFree(void* p) { free(p); return hipSuccess; }
inline hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) { memcpy(d, s, n); return hipSuccess; }
inline hipError_t hipMemset(void* d, int v, size_t n) { memset(d, v, n); return hipSuccess; }
inline hipError_t hipDeviceSynchronize() { return hipSuccess; }
