// S5 KV-outer sparse prefill attention and S6 log-sum-exp combine for gfx950.
//
// Reference behaviour (pfnet-research/semantic-block-sparse-attention):
//   kv_outer.py:482-816        kv_outer_attention: one FA3 varlen call per
//                              (cluster, KV head) over its visible rows, whose
//                              query rows are the queries that selected it
//                              (Q heads folded into rows), plus an exactly
//                              causal FA3 call over the chunk's own window
//   fused_prefill.py:155-189   dense causal attention for the early chunks
//   kv_outer.py:370-428        _combine_grouped_kernel (query-major LSE fold)
//
// Design (MI355X): one persistent kernel walks a work list of items.  An item
// is (KV head, cluster or the local window, a tile of 128/G queries); its
// 128 (query, head) rows run against the cluster's contiguous packed run (or
// the prompt-order window, causally masked) in 32-key tiles.  Both GEMMs are
// on bf16 MFMA 32x32x16 in the transposed form S^T = K Q^T, O^T = V^T P^T,
// so the softmax probabilities come out of the first MFMA already in the
// B-operand layout of the second and never pass through LDS.
#include "sbsa_common.h"

#include <type_traits>

namespace {

struct AttnArgs {
  const bf16_t* q;          // [Qc, Hq, D] chunk queries
  int64_t q_sq, q_sh;
  int64_t q_bytes;          // extent of q in bytes (buffer range of the staged Q loads)
  const bf16_t* packed;     // [2, Lp, Hkv, D] cluster-ordered K/V
  int64_t packed_len;
  const bf16_t* korig;      // prompt-order keys from position wstart: k[pos - wstart, h, :]
  const bf16_t* vorig;      // prompt-order values, same rows
  int64_t o_st, o_sh;       // their token / head strides (elements)
  const int32_t* indptr;    // [Hkv, C+1] packed run starts
  const int32_t* nvis;      // [Hkv, C] visible rows per cluster
  const int32_t* rev_indptr;// [Hkv*C + 1]
  const int32_t* qvals;     // [nnz] query slots per (head, cluster)
  const PrefillItem* items;
  int32_t* queue;           // n[8], offset[8], counter[8]: one work queue per XCD
  bf16_t* part_o;           // [nnz, G, D]
  float* part_lse;          // [nnz, G]
  bf16_t* local_o;          // [Qc, Hq, D] strided
  int64_t lo_sq, lo_sh;
  float* local_lse;         // [Qc, Hq] or null
  int Hkv, C, Hq;
  int Qc;                   // queries of the chunk (query indices are clamped below it)
  int64_t chunk_start, wstart;
  float scale_log2;         // sm_scale * log2(e)
};

constexpr int KT = 32;                  // keys per tile
constexpr int ATTN_NB = 4;              // K (and V) tile buffers: loads run NB - 1 tiles ahead
constexpr int PREFILL_ROWS = 256;       // (query, head) rows per work item: 64 per wave
// Probabilities are taken against a reference maximum per row and may reach
// 2^RESCALE_LOG2 (well inside fp32 and bf16 range) before the row's reference
// is raised and its accumulators rescaled.
constexpr float RESCALE_LOG2 = 64.0f;
// queue layout: per-XCD item counts [0, 8), offsets [8, 16) and claim
// counters [16, 24); the overflow list's count, its claim counter, and from
// QUEUE_OVF_LIST the listed items
constexpr int QUEUE_OVF_N = 24;
constexpr int QUEUE_OVF_CLAIM = 25;
constexpr int QUEUE_OVF_LIST = 32;
constexpr int BUFFER_CONFIG = 0x00020000;   // raw buffer resource, 32-bit data format

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

__device__ __forceinline__ const bf16_t* uniform_ptr(const bf16_t* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const bf16_t*)(((uint64_t)hi << 32) | lo);
}

// One 16-byte-per-lane buffer load straight into LDS (lane l writes bytes
// 16 l .. 16 l + 15 past lds_addr).  Issued from inline assembly so that the
// compiler does not track it: it would otherwise make every later LDS read
// wait for the load (it cannot tell that the read is from another buffer).
// The kernel waits for these loads itself (s_waitcnt vmcnt) before the
// barrier that publishes a tile.  M0 holds the LDS base, as the instruction
// requires; nothing else in the kernel uses M0.
__device__ __forceinline__ void lds_dma16(u32x4_t rsrc, uint32_t lds_addr, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// The same for one dword per lane (lane l writes bytes 4 l .. 4 l + 3).
__device__ __forceinline__ void lds_dma4(u32x4_t rsrc, uint32_t lds_addr, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// v + (or max with) the same value of lane l ^ 32, in every lane: one swap of
// the lane halves instead of an LDS permute
__device__ __forceinline__ float halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float halves_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// LDS tile layout: K and V rows of D bf16, row-major, 16-byte chunks of row r
// permuted by an XOR so that the operand reads of one LDS cycle (256 bytes,
// the 64 banks) hit distinct banks:
//   K: chunk ^ (r % 16)     16 lanes read 16 bytes of 16 different rows
//   V: chunk ^ 4 (r % 4)    32 lanes read 8 bytes of 4 rows, 64 bytes each
// Tiles are filled straight from global memory by buffer loads into LDS
// (lane l writes slot l of a 1 KB run; rows past the item's last key are
// outside the buffer's range and read as zero).
template <int D>
struct AttnTileShape {
  static constexpr int CH = D / 8;                    // 16-byte chunks per row
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int TILE_BYTES = KT * ROW_BYTES;   // one of K or V
  static constexpr size_t lds_bytes() { return 2 * ATTN_NB * (size_t)TILE_BYTES; }   // NB K, NB V
  static constexpr int ROWS_PER_INST = 64 / CH;       // rows one wave instruction covers
  static constexpr int INSTS = KT / ROWS_PER_INST;    // instructions per K (or V) tile
  static constexpr int PER_WAVE = INSTS / 4;
};

// S^T's MFMAs as written instructions with vector-register accumulators.
// The compiler does not know these are MFMAs, so the wait states the
// hardware needs before the VALU reads an MFMA result are written out in
// s_mfma_results_to_valu (20 wait states, more than the 19 a 16-pass XDL
// result needs), which also orders every later use of the two tiles after
// it.  The inputs need no wait states: K fragments come from LDS reads (the
// compiler waits for them, as for any asm operand) and Q from global loads;
// the first step takes a zero accumulator, so no VALU write precedes any.
__device__ __forceinline__ void s_mfma_first(f32x16_t& d, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void s_mfma_acc(f32x16_t& d, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void s_mfma_results_to_valu(f32x16_t& x, f32x16_t& y) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(x), "+v"(y));
}

// Each wave owns 64 of an item's 256 (query, head) rows, as two groups of 32
// (x = 0, 1).  Both GEMMs run on bf16 MFMA 32x32x16 in the transposed form:
// S^T = K Q^T (32 keys x 32 rows per group and tile) and O^T += V^T P^T
// (32 dims x 32 rows).  Each K or V operand fragment read from LDS feeds the
// MFMAs of both groups, so a tile costs half the LDS reads per FLOP that a
// 32-row wave pays.  Lane l holds row l % 32 of each group; in S^T it holds
// keys 8 (i / 4) + 4 (l / 32) + i % 4, i < 16, which are exactly the B
// operand P^T of the two 16-key steps of O^T (keys {0-3, 8-11 | 4-7, 12-15}
// and {16-19, 24-27 | 20-23, 28-31}), so the probabilities never leave the
// lane.  The O accumulators (2 x D/32 x 16 fp32 per lane, 256 at D = 256)
// live in the accumulation registers; Q (2 x D/16 x 16 bytes) in the vector
// registers.
//
// Step t runs S(t) on the MFMA units, then O += V(t-1) P(t-1) while the VALU
// turns S(t) into P(t): one tile's softmax hides under the previous tile's
// second GEMM.  K(t+1) and V(t) stream into LDS during step t, one barrier
// per step.  At an item's last tile its next item's first K tile loads into
// the free K buffer, and once S(last) is done the next item's Q rows load
// into the Q registers, so an item starts with its operands in flight.
//
// Each row's probabilities are taken against a reference maximum fixed from
// the item's first tile, so no accumulator is rescaled in the loop.  A row
// whose probabilities pass 2^RESCALE_LOG2 (its sums per tile are checked,
// which any such probability would push past the bound) puts its item on an
// overflow list instead of storing it, and the REDO form of the kernel,
// launched after the main one, recomputes the listed items: a sweep over the
// tiles finds the rows' true maxima, and a second pass takes them as
// reference.  Probabilities up to the bound are safe in fp32 and bf16.
template <int D, int G, bool REDO>
__global__ __launch_bounds__(256, 1) void attn_items_kernel(AttnArgs a) {
  using S = AttnTileShape<D>;
  constexpr int KS = D / 16;        // 16-dim steps of S^T
  constexpr int DT = D / 32;        // 32-dim tiles of O^T
  constexpr int QPI = PREFILL_ROWS / G;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_attn[];
  __shared__ int s_items[2];
  __shared__ int s_queue[16];
  __shared__ int s_qslots[2][QPI < 64 ? 64 : QPI];   // a whole wave's lanes per row (the fetch writes 64)

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const float NEG_INF = -INFINITY;
  const int home = blockIdx.x & 7;
  int probe = 0;

  // --- per-lane address bases (fixed for the kernel) ---------------------
  const int r0 = wave * S::ROWS_PER_INST + lane / S::CH;
  const int cpos = lane % S::CH;
  uint32_t kslot[2], vslot;
  kslot[0] = (uint32_t)((cpos ^ (r0 & 15)) * 16);
  kslot[1] = (uint32_t)((cpos ^ ((r0 + 4 * S::ROWS_PER_INST) & 15)) * 16);
  vslot = (uint32_t)((cpos ^ ((r0 & 3) << 2)) * 16);
  int kbase[8];
#pragma unroll
  for (int s8 = 0; s8 < 8; ++s8) kbase[s8] = l32 * S::ROW_BYTES + 16 * ((2 * s8 + g) ^ (l32 & 15));
  const int i16 = lane & 15, hh = (lane >> 4) & 1;
  int vbase[4];
#pragma unroll
  for (int d4 = 0; d4 < 4; ++d4)
    vbase[d4] = (4 * g + (i16 >> 2)) * S::ROW_BYTES + 16 * (4 * (d4 ^ (i16 >> 2)) + 2 * hh + ((i16 & 3) >> 1)) +
                8 * (i16 & 1);
  // the per-lane LDS and load offsets are made opaque at every step, so the
  // compiler recomputes the addresses derived from them there instead of
  // holding (or spilling) them across the loop
  auto opaque_bases = [&]() {
#pragma unroll
    for (int k = 0; k < 8; ++k) asm volatile("" : "+v"(kbase[k]));
#pragma unroll
    for (int k = 0; k < 4; ++k) asm volatile("" : "+v"(vbase[k]));
    asm volatile("" : "+v"(kslot[0]), "+v"(kslot[1]), "+v"(vslot));
  };
  auto kbuf_at = [&](int i) { return smem_attn + (i % ATTN_NB) * S::TILE_BYTES; };
  auto vbuf_at = [&](int i) { return smem_attn + (ATTN_NB + i % ATTN_NB) * S::TILE_BYTES; };

  // --- work claims: per-XCD queues with stealing, two items ahead ---------
  // (REDO: the overflow list, one shared counter)
  if (!REDO && threadIdx.x < 16) s_queue[threadIdx.x] = a.queue[threadIdx.x];
  int pend = 0;
  if (!REDO && threadIdx.x == 0) pend = atomicAdd(&a.queue[16 + home], 1);
  __syncthreads();
  auto claim = [&]() -> int {
    if (REDO) {
      const int i = atomicAdd(&a.queue[QUEUE_OVF_CLAIM], 1);
      return i < a.queue[QUEUE_OVF_N] ? a.queue[QUEUE_OVF_LIST + i] : -1;
    }
    int claimed = -1;
    for (;;) {
      const int x = (home + probe) & 7;
      if (pend < s_queue[x]) {
        claimed = s_queue[8 + x] + pend;
        break;
      }
      if (++probe == 8) break;
      pend = atomicAdd(&a.queue[16 + ((home + probe) & 7)], 1);
    }
    if (claimed >= 0) pend = atomicAdd(&a.queue[16 + ((home + probe) & 7)], 1);
    return claimed;
  };
  int parity = 0;
  auto next_index = [&]() -> int {
    const int v = __builtin_amdgcn_readfirstlane(s_items[parity ^ 1]);
    if (threadIdx.x == 0) s_items[parity] = v >= 0 ? claim() : -1;
    parity ^= 1;
    return v;
  };

  // this lane's rows: group x is R = 64 wave + 32 x + l32 -> (query slot R / G, head R % G)
  int row_i[2], row_j[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    row_i[x] = (wave * 64 + x * 32 + l32) / G;
    row_j[x] = (wave * 64 + x * 32 + l32) % G;
  }

  // a cluster item's query slots into s_qslots[buf] (wave 0, buffer loads to LDS)
  auto fetch_slots = [&](const PrefillItem& r, int buf) {
    const int c = __builtin_amdgcn_readfirstlane(r.c);
    if (wave != 0 || c < 0) return;
    const int qn = __builtin_amdgcn_readfirstlane(r.qn);
    const uint64_t b = (uint64_t)(a.qvals + __builtin_amdgcn_readfirstlane(r.entry0));
    u32x4_t rsrc;
    rsrc.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
    rsrc.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
    rsrc.z = (uint32_t)qn * 4u;
    rsrc.w = (uint32_t)BUFFER_CONFIG;
    const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)s_qslots[buf]);
#pragma unroll
    for (int k = 0; k < QPI; k += 64) lds_dma4(rsrc, dst + 4 * k, (uint32_t)(lane + k) * 4u);
  };
  // a tile's loads as a plan (uniform: the buffer resource and the LDS slice)
  // and its PER_WAVE instructions, which the steady steps spread between MFMAs
  struct DmaPlan {
    u32x4_t rsrc;
    uint32_t dst, kvoff;
  };
  auto plan_tile = [&](const bf16_t* base, uint32_t rs_bytes, int nkeys, int t, unsigned char* dst_tile) -> DmaPlan {
    const int t0 = t * KT;
    const int rows = t < 0 ? 0 : max(nkeys - t0, 0);
    const int valid = __builtin_amdgcn_readfirstlane((int)((uint32_t)rows * rs_bytes));
    const uint64_t b = (uint64_t)((const unsigned char*)base + (uint64_t)max(t0, 0) * rs_bytes);
    DmaPlan pl;
    pl.rsrc.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
    pl.rsrc.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
    pl.rsrc.z = (uint32_t)valid;
    pl.rsrc.w = (uint32_t)BUFFER_CONFIG;
    pl.dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)(dst_tile + wave * 1024));
    pl.kvoff = (uint32_t)r0 * rs_bytes;
    return pl;
  };
  auto dma_one = [&](const DmaPlan& pl, uint32_t rs_bytes, int m, bool is_k) {
    const uint32_t roff = pl.kvoff + (uint32_t)(m * 4 * S::ROWS_PER_INST) * rs_bytes;
    const uint32_t slot = is_k ? kslot[m & 1] : vslot;
    lds_dma16(pl.rsrc, pl.dst + m * 4096, roff + slot);
  };
  auto issue = [&](const bf16_t* base, uint32_t rs_bytes, int nkeys, int t, unsigned char* dst_tile, bool is_k) {
    const int t0 = t * KT;
    // rows of the tile inside the item (none for a tile before or past it: the
    // buffer range is then empty and the loads only write zeros to LDS)
    const int rows = t < 0 ? 0 : max(nkeys - t0, 0);
    const int valid = __builtin_amdgcn_readfirstlane((int)((uint32_t)rows * rs_bytes));
    const uint64_t b = (uint64_t)((const unsigned char*)base + (uint64_t)max(t0, 0) * rs_bytes);
    u32x4_t rsrc;
    rsrc.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
    rsrc.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
    rsrc.z = (uint32_t)valid;
    rsrc.w = (uint32_t)BUFFER_CONFIG;
    const uint32_t dst = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(lds_void_t*)(dst_tile + wave * 1024));
    const uint32_t kvoff = (uint32_t)r0 * rs_bytes;
#pragma unroll
    for (int m = 0; m < S::PER_WAVE; ++m) {
      const uint32_t roff = kvoff + (uint32_t)(m * 4 * S::ROWS_PER_INST) * rs_bytes;
      const uint32_t slot = is_k ? kslot[m & 1] : vslot;
      lds_dma16(rsrc, dst + m * 4096, roff + slot);
    }
  };

  // --- one item's fields (uniform) ------------------------------------------
  struct Item {
    int h, c, qb, qn, nkeys;
    int64_t entry0;
    const bf16_t* kp;
    const bf16_t* vp;
    uint32_t rsb;
  };
  auto resolve = [&](const PrefillItem& r) -> Item {
    Item it;
    it.h = __builtin_amdgcn_readfirstlane(r.h);
    it.c = __builtin_amdgcn_readfirstlane(r.c);
    it.qb = __builtin_amdgcn_readfirstlane(r.qb);
    it.qn = __builtin_amdgcn_readfirstlane(r.qn);
    it.entry0 = __builtin_amdgcn_readfirstlane(r.entry0);
    const bool local = it.c < 0;
    const int64_t row0 = __builtin_amdgcn_readfirstlane(r.row0);
    const int nk = local ? (int)(a.chunk_start + it.qb + it.qn - a.wstart) : __builtin_amdgcn_readfirstlane(r.nkeys);
    it.nkeys = max(__builtin_amdgcn_readfirstlane(nk), 0);
    const bf16_t* kp;
    const bf16_t* vp;
    int64_t rs;
    if (local) {
      kp = a.korig + (int64_t)it.h * a.o_sh;
      vp = a.vorig + (int64_t)it.h * a.o_sh;
      rs = a.o_st;
    } else {
      kp = a.packed + row0 * a.Hkv * D + (int64_t)it.h * D;
      vp = kp + a.packed_len * a.Hkv * D;
      rs = (int64_t)a.Hkv * D;
    }
    it.kp = uniform_ptr(kp);
    it.vp = uniform_ptr(vp);
    it.rsb = (uint32_t)__builtin_amdgcn_readfirstlane((int)(rs * 2));
    return it;
  };
  // this lane's query of group x in item `it` (-1 past the item's queries)
  auto query_of = [&](const Item& it, int x, int sbuf) -> int {
    if (row_i[x] >= it.qn) return -1;
    return it.c < 0 ? it.qb + row_i[x] : s_qslots[sbuf][row_i[x]];
  };
  // Q^T rows (B of S^T) into registers: lane holds row (query, head) dims
  // 16 s + 8 g .. +8.  Rows past the item's queries take query 0's values.
  u32x4_t qr[2][KS];
  auto load_q = [&](const Item& it, const int (&qi)[2]) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const bf16_t* src = a.q + (int64_t)max(qi[x], 0) * a.q_sq + (int64_t)(it.h * G + row_j[x]) * a.q_sh + g * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) qr[x][s] = *reinterpret_cast<const u32x4_t*>(src + s * 16);
    }
  };

  // the same rows touched once per 128-byte line, into L2 only: one dword per
  // line loaded straight into a scratch word of LDS that is never read (the
  // loads complete at the next s_waitcnt; no register receives them)
  __shared__ int s_sink[64];
  auto warm_q = [&](const Item& it, const int (&qi)[2]) {
    const uint64_t b = (uint64_t)a.q;
    u32x4_t rsrc;
    rsrc.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
    rsrc.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
    rsrc.z = (uint32_t)min(a.q_bytes, (int64_t)0x7fffffff);
    rsrc.w = (uint32_t)BUFFER_CONFIG;
    const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)s_sink);
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int64_t row = ((int64_t)max(qi[x], 0) * a.q_sq + (int64_t)(it.h * G + row_j[x]) * a.q_sh) * 2;
#pragma unroll
      for (int k = g; k < D / 64; k += 2) {
        const int64_t off = row + 128 * k;
        lds_dma4(rsrc, dst, off < 0x7fffffff ? (uint32_t)off : 0x80000000u);
      }
    }
  };

  // --- the GEMMs and the softmax pieces ---------------------------------------
  constexpr int KA_AHEAD = 3;
  auto kread = [&](const unsigned char* sK, int s) -> u32x4_t {
    return *reinterpret_cast<const u32x4_t*>(sK + kbase[s & 7] + 256 * (s >> 3));
  };
  // S^T of both groups for one tile: each K fragment feeds two MFMAs.  These
  // MFMAs are written out (s_mfma_*) so that S^T stays in the vector
  // registers, where the softmax reads it, while the compiler keeps the O
  // accumulators in the accumulation registers.
  auto gemm_s = [&](f32x16_t (&sacc)[2], const unsigned char* sK) {
    u32x4_t ka[KA_AHEAD];
#pragma unroll
    for (int f = 0; f < KA_AHEAD; ++f) ka[f] = kread(sK, f);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4_t cur = ka[s % KA_AHEAD];
      if (s + KA_AHEAD < KS) ka[s % KA_AHEAD] = kread(sK, s + KA_AHEAD);
      if (s == 0) {
        s_mfma_first(sacc[0], cur, qr[0][s]);
        s_mfma_first(sacc[1], cur, qr[1][s]);
      } else {
        s_mfma_acc(sacc[0], cur, qr[0][s]);
        s_mfma_acc(sacc[1], cur, qr[1][s]);
      }
    }
    s_mfma_results_to_valu(sacc[0], sacc[1]);
  };
  auto vread = [&](const unsigned char* sV, int f) -> u32x4_t {
    const int m = f / DT, dt = f % DT;
    const unsigned char* p = sV + vbase[dt & 3] + 256 * (dt >> 2) + 16 * m * S::ROW_BYTES;
    s16x4_t part[2];
    part[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
    part[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + 8 * S::ROW_BYTES));
    u32x4_t r;
    __builtin_memcpy(&r, part, 16);
    return r;
  };

  // ===========================================================================
  if (threadIdx.x == 0) {
    s_items[0] = claim();
    s_items[1] = s_items[0] >= 0 ? claim() : -1;
  }
  __syncthreads();
  int idx = __builtin_amdgcn_readfirstlane(s_items[0]);
  if (idx < 0) return;
  int sbuf = 0;                        // s_qslots buffer of the current item
  Item cur;
  int qidx[2];
  {
    const PrefillItem rec = a.items[idx];
    fetch_slots(rec, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    cur = resolve(rec);
    qidx[0] = query_of(cur, 0, 0);
    qidx[1] = query_of(cur, 1, 0);
  }
  f32x16_t o[2][DT];
  const float lim = __builtin_exp2f(RESCALE_LOG2);

  for (;;) {
    load_q(cur, qidx);                 // Q is loaded at the item's start: its registers are
                                       // not live across items
    const int idx_n = next_index();
    PrefillItem rec_n{};
    if (idx_n >= 0) rec_n = a.items[idx_n];
    const bool local = cur.c < 0;
    const int nkeys = cur.nkeys;
    const int ntiles = max(1, (nkeys + KT - 1) / KT);
    // causal limits (local window items): key index limit per row, and the
    // wave's largest / smallest limit over its valid rows
    int qlim[2];
    int wave_lim = 0x7fffffff, wave_min = 0x7fffffff;
#pragma unroll
    for (int x = 0; x < 2; ++x) qlim[x] = local ? (int)(a.chunk_start + qidx[x] - a.wstart) : 0x7fffffff;
    if (local) {
      wave_lim = max(qlim[0], qlim[1]);
      wave_min = min(qidx[0] >= 0 ? qlim[0] : 0x7fffffff, qidx[1] >= 0 ? qlim[1] : 0x7fffffff);
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        wave_lim = max(wave_lim, __shfl_xor(wave_lim, off, 64));
        wave_min = min(wave_min, __shfl_xor(wave_min, off, 64));
      }
      wave_lim = __builtin_amdgcn_readfirstlane(wave_lim);
      wave_min = __builtin_amdgcn_readfirstlane(wave_min);
    }
    const int t_last_act = min(ntiles - 1, wave_lim / KT);   // last tile some row of the wave sees

    auto mask = [&](f32x16_t (&sacc)[2], int t) {
      const int t0 = t * KT;
      if (t0 + KT > nkeys || t0 + KT - 1 > wave_min) {
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = t0 + 8 * (e >> 2) + 4 * g + (e & 3);
            if (!(key < nkeys && key <= qlim[x])) sacc[x][e] = NEG_INF;
          }
      }
    };
    float m_ref[2] = {0.f, 0.f}, l_part[2] = {0.f, 0.f};
    auto row_max = [&](const f32x16_t (&sacc)[2], float (&mx)[2]) {
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        float v = NEG_INF;
#pragma unroll
        for (int e = 0; e < 16; e += 4)
          v = fmaxf(v, fmaxf(fmaxf(sacc[x][e], sacc[x][e + 1]), fmaxf(sacc[x][e + 2], sacc[x][e + 3])));
        mx[x] = halves_max(v);
      }
    };
    // probabilities exp2(s - m) of both groups as the B operands of O^T, and
    // this lane's sums of them
    auto exp_pack = [&](f32x16_t (&sacc)[2], u32x4_t (&pb)[2][2], float (&sum)[2]) {
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          sacc[x][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[x][e], a.scale_log2, -m_ref[x]));
          acc += sacc[x][e];
        }
        sum[x] = acc;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          pb[x][m].x = pack2bf(sacc[x][8 * m + 0], sacc[x][8 * m + 1]);
          pb[x][m].y = pack2bf(sacc[x][8 * m + 2], sacc[x][8 * m + 3]);
          pb[x][m].z = pack2bf(sacc[x][8 * m + 4], sacc[x][8 * m + 5]);
          pb[x][m].w = pack2bf(sacc[x][8 * m + 6], sacc[x][8 * m + 7]);
        }
      }
    };
    // O^T += V^T P^T for both groups: each V^T fragment feeds two MFMAs
    auto gemm_pv = [&](const u32x4_t (&pb)[2][2], const unsigned char* sV) {
      constexpr int NF = DT * 2;
      constexpr int VA_AHEAD = 3;
      u32x4_t va[VA_AHEAD];
#pragma unroll
      for (int f = 0; f < VA_AHEAD; ++f) va[f] = vread(sV, f);
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const u32x4_t cv = va[f % VA_AHEAD];
        if (f + VA_AHEAD < NF) va[f % VA_AHEAD] = vread(sV, f + VA_AHEAD);
        const int m = f / DT, dt = f % DT;
        o[0][dt] = mfma32x32x16(as_bf16x8(cv), as_bf16x8(pb[0][m]), o[0][dt]);
        o[1][dt] = mfma32x32x16(as_bf16x8(cv), as_bf16x8(pb[1][m]), o[1][dt]);
      }
    };

    // REDO: a sweep over the tiles for the rows' true maxima first (S only)
    if (REDO) {
      float lmax[2] = {NEG_INF, NEG_INF};
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      issue(cur.kp, cur.rsb, nkeys, 0, kbuf_at(0), true);
      for (int t = 0; t < ntiles; ++t) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (t + 1 < ntiles) issue(cur.kp, cur.rsb, nkeys, t + 1, kbuf_at(t + 1), true);
        if (t == 0 && idx_n >= 0) fetch_slots(rec_n, sbuf ^ 1);
        if (t <= t_last_act) {
          f32x16_t sc[2];
          gemm_s(sc, kbuf_at(t));
          mask(sc, t);
          float mx[2];
          row_max(sc, mx);
          lmax[0] = fmaxf(lmax[0], mx[0]);
          lmax[1] = fmaxf(lmax[1], mx[1]);
        }
      }
#pragma unroll
      for (int x = 0; x < 2; ++x) m_ref[x] = (lmax[x] == NEG_INF) ? 0.f : lmax[x] * a.scale_log2;
    }

#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[x][dt][e] = 0.f;
    bool over = false, next_issued = false;
    u32x4_t pb_prev[2][2];
    // loads of step t: K(t + NB - 1) and V(t + NB - 2) (zero-range loads past
    // the item's end, so every step issues the same number)
    auto issue_step = [&](int t) {
      issue(cur.kp, cur.rsb, nkeys, t + ATTN_NB - 1, kbuf_at(t + ATTN_NB - 1), true);
      issue(cur.vp, cur.rsb, nkeys, t + ATTN_NB - 2, vbuf_at(t + ATTN_NB - 2 + ATTN_NB), false);
    };
    // K(t) and V(t-1) were issued NB - 1 steps back: the loads of the NB - 2
    // steps since may stay in flight.  Every wave is done with K(t-1) and
    // V(t-2), whose buffers the step's loads refill.
    constexpr int VM_KEEP = (ATTN_NB - 2) * 2 * S::PER_WAVE;
    auto sync_step = [&]() {
      __builtin_amdgcn_s_waitcnt((VM_KEEP & 15) | ((VM_KEEP >> 4) << 14) | (7 << 4));
      __syncthreads();
      opaque_bases();
    };
    // the item's first NB - 1 steps' loads (virtual steps 1 - NB .. -1)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#pragma unroll
    for (int v = 1 - ATTN_NB; v < 0; ++v) issue_step(v);
    // the steps' three parts, as straight-line code for the steady state
    auto part_s = [&](int t, u32x4_t (&pb)[2][2], bool masked) {
      f32x16_t sc[2];
      gemm_s(sc, kbuf_at(t));
      if (masked) mask(sc, t);
      if (!REDO && t == 0) {
        // reference maximum: the row's maximum over the first tile (key 0 of
        // an item is visible to every row, so it is finite)
        float mx[2];
        row_max(sc, mx);
#pragma unroll
        for (int x = 0; x < 2; ++x) m_ref[x] = (mx[x] == NEG_INF) ? 0.f : mx[x] * a.scale_log2;
      }
      float sum[2];
      exp_pack(sc, pb, sum);
      over |= !(sum[0] <= lim) || !(sum[1] <= lim);
      l_part[0] += sum[0];
      l_part[1] += sum[1];
    };

    // step 0: S(0) and P(0)
    sync_step();
    issue_step(0);
    if (!REDO && idx_n >= 0) fetch_slots(rec_n, sbuf ^ 1);
    part_s(0, pb_prev, true);
    // steady steps: tiles seen whole by every row of the wave, not the last
    // one, the next tile's loads issued at the top
    const int t_steady = min(min(ntiles - 1, t_last_act + 1),
                             wave_min == 0x7fffffff ? 0x7fffffff : (wave_min + 1) / KT);
    int t = 1;
    for (; t < t_steady; ++t) {
      sync_step();
      // this step's loads, one instruction after every other fragment of the
      // second GEMM below (their issue hides under the MFMAs)
      const DmaPlan dk = plan_tile(cur.kp, cur.rsb, nkeys, t + ATTN_NB - 1, kbuf_at(t + ATTN_NB - 1));
      const DmaPlan dv = plan_tile(cur.vp, cur.rsb, nkeys, t + ATTN_NB - 2, vbuf_at(t + ATTN_NB - 2 + ATTN_NB));
      u32x4_t pb_cur[2][2];
      {
        f32x16_t sc[2];
        gemm_s(sc, kbuf_at(t));
        // O += V(t-1) P(t-1) with the softmax of S(t) woven between its MFMAs,
        // fragment by fragment (scheduling barriers keep the order): per
        // V^T fragment two MFMAs, two probabilities and one packed pair
        const unsigned char* sV = vbuf_at(t - 1);
        constexpr int NF = DT * 2;
        constexpr int VA_AHEAD = 3;
        u32x4_t va[VA_AHEAD];
#pragma unroll
        for (int f = 0; f < VA_AHEAD; ++f) va[f] = vread(sV, f);
        float sum[2] = {0.f, 0.f};
        uint32_t pk[2][8];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const u32x4_t cv = va[f % VA_AHEAD];
          if (f + VA_AHEAD < NF) va[f % VA_AHEAD] = vread(sV, f + VA_AHEAD);
          const int m = f / DT, dt = f % DT;
          o[0][dt] = mfma32x32x16(as_bf16x8(cv), as_bf16x8(pb_prev[0][m]), o[0][dt]);
          o[1][dt] = mfma32x32x16(as_bf16x8(cv), as_bf16x8(pb_prev[1][m]), o[1][dt]);
#pragma unroll
          for (int k = 0; k < 32 / NF; k += 2) {
            const int q = f * (32 / NF) + k;          // element pair (q, q + 1) of S(t)
            const int x = q / 16, e = q % 16;
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[x][e], a.scale_log2, -m_ref[x]));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[x][e + 1], a.scale_log2, -m_ref[x]));
            sum[x] += p0 + p1;
            pk[x][e / 2] = pack2bf(p0, p1);
          }
          static_assert(NF >= 4 * S::PER_WAVE, "one load instruction per two fragments");
          if (f % 2 == 0 && f / 2 < 2 * S::PER_WAVE) {
            const int m = f / 2;
            if (m < S::PER_WAVE) dma_one(dk, cur.rsb, m, true);
            else dma_one(dv, cur.rsb, m - S::PER_WAVE, false);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int mm = 0; mm < 2; ++mm) {
            pb_cur[x][mm].x = pk[x][4 * mm + 0];
            pb_cur[x][mm].y = pk[x][4 * mm + 1];
            pb_cur[x][mm].z = pk[x][4 * mm + 2];
            pb_cur[x][mm].w = pk[x][4 * mm + 3];
          }
        over |= !(sum[0] <= lim) || !(sum[1] <= lim);
        l_part[0] += sum[0];
        l_part[1] += sum[1];
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int m = 0; m < 2; ++m) pb_prev[x][m] = pb_cur[x][m];
    }
    // the general steps: masked tiles, tiles past some of the wave's rows,
    // and the last one; then the last tile's second GEMM
    for (; t <= ntiles; ++t) {
      sync_step();
      issue_step(t);
      const bool do_s = t < ntiles && t <= t_last_act;
      const bool do_pv = t - 1 <= t_last_act;
      u32x4_t pb_cur[2][2];
      if (do_s) part_s(t, pb_cur, true);
      if (do_pv) gemm_pv(pb_prev, vbuf_at(t - 1));
      if (do_s) {
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int m = 0; m < 2; ++m) pb_prev[x][m] = pb_cur[x][m];
      }
    }
    // an item with a row past the bound goes to the overflow list (thread 0
    // appends it); its rows are not stored here
    const bool redo = !REDO && __syncthreads_or(over ? 1 : 0);
    if (redo && threadIdx.x == 0) {
      const int k = atomicAdd(&a.queue[QUEUE_OVF_N], 1);
      a.queue[QUEUE_OVF_LIST + k] = idx;
    }

    // epilogue: normalise and store this lane's rows straight from the
    // accumulators.  A swap of the lane halves (lanes l and l + 32) gives
    // lane g = 0 all 8 dims of chunk 4 dt + 2 p and lane g = 1 those of chunk
    // 4 dt + 2 p + 1, so each lane writes whole 16-byte chunks.
    if (!redo) {
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const float l = halves_sum(l_part[x]);
        const float inv = (l > 0.f) ? 1.0f / l : 0.f;
        const int qi = qidx[x];
        const int i = row_i[x], j = row_j[x];
        if (qi >= 0 && g == 0) {
          const float lse = (l > 0.f) ? (m_ref[x] + log2f(l)) * 0.69314718055994531f : NEG_INF;
          float* ldst = local ? (a.local_lse ? a.local_lse + (int64_t)qi * a.Hq + cur.h * G + j : nullptr)
                              : a.part_lse + (cur.entry0 + i) * G + j;
          if (ldst) *ldst = lse;
        }
        bf16_t* dst = local ? a.local_o + (int64_t)(cur.qb + i) * a.lo_sq + (int64_t)(cur.h * G + j) * a.lo_sh
                            : a.part_o + ((cur.entry0 + i) * G + j) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const int qa = 2 * p, qb2 = 2 * p + 1;
            const uint32_t a0 = pack2bf(o[x][dt][4 * qa + 0] * inv, o[x][dt][4 * qa + 1] * inv);
            const uint32_t a1 = pack2bf(o[x][dt][4 * qa + 2] * inv, o[x][dt][4 * qa + 3] * inv);
            const uint32_t b0 = pack2bf(o[x][dt][4 * qb2 + 0] * inv, o[x][dt][4 * qb2 + 1] * inv);
            const uint32_t b1 = pack2bf(o[x][dt][4 * qb2 + 2] * inv, o[x][dt][4 * qb2 + 3] * inv);
            const auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
            u32x4_t w;
            w.x = s0[0];
            w.y = s1[0];
            w.z = s0[1];
            w.w = s1[1];
            if (qi >= 0) __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(dst + 8 * (4 * dt + 2 * p + g)));
          }
      }
    }

    if (idx_n < 0) break;
    idx = idx_n;
    cur = resolve(rec_n);
    sbuf ^= 1;
    qidx[0] = query_of(cur, 0, sbuf);
    qidx[1] = query_of(cur, 1, sbuf);
  }
}


// A work item's record through the scalar unit: the records are read-only
// while the attention kernels run (written by the item builder before them),
// so they are read as constant memory, and the read waits only for itself
// instead of for every outstanding vector load.
typedef __attribute__((address_space(4))) const PrefillItem const_item_t;
__device__ __forceinline__ PrefillItem load_item(const PrefillItem* items, int idx) {
  const_item_t& src = ((const_item_t*)(uintptr_t)items)[idx];
  PrefillItem r;
  r.h = src.h;
  r.c = src.c;
  r.qb = src.qb;
  r.qn = src.qn;
  r.nkeys = src.nkeys;
  r.entry0 = src.entry0;
  r.row0 = src.row0;
  r.pad = 0;
  return r;
}

// An accumulation register read into a vector register as a written
// instruction, and the accumulator tiles zeroed by written MFMAs: the O
// accumulators are then only ever used as accumulation registers, whole
// tiles at a time, and the register allocator keeps them there.
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}
// A 16-register accumulator tile set to zero by one MFMA of zero operands
// (4 wait states first: the zero operand was just written by the VALU, and
// the tile may just have been read by v_accvgpr_read).  A later MFMA that
// accumulates into the tile needs no wait states after it.
__device__ __forceinline__ void acc_zero_tile(f32x16_t& d) {
  const u32x4_t z = {0u, 0u, 0u, 0u};
  asm volatile("s_nop 3\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(d) : "v"(z));
}

// The main pass as one stream of tiles per block.  A block's items follow each
// other through one pipeline: the tiles of its items, in claim order, form
// the block's tile stream, and global step s runs S^T of stream tile s and
// O += V P of stream tile s - 1 while the K tile of step s + NB - 1 and the V
// tile of stream tile s + NB - 2 load.  The pipeline never drains at an item
// boundary: the next item's tiles are already in flight when an item ends.
// An item's rows are stored in the step that runs its last tile's second
// GEMM; the next item's Q rows load as soon as the item's last S^T is done.
// Claims run two items ahead of the load cursor through a ring of item slots
// in LDS, and a cluster item's query slots are fetched into LDS one item
// ahead of the load cursor.
//
// Wait accounting (per wave, vmcnt counts every vector memory instruction in
// issue order): each step issues exactly 2 PER_WAVE tile loads, so at the top
// of step s the loads of steps s - 1 and s - 2 may stay in flight
// (VM_KEEP).  A step that stored an item's rows issued exactly EPI_STORES
// stores after its loads (rows past the item's queries are stored out of the
// buffer range, where the store is dropped, so the count does not depend on
// the rows), and the next step's wait allows for them.  A step whose S^T
// starts an item waits for everything: its Q rows were the last loads.
template <int D, int G>
__global__ __launch_bounds__(256, 1) void attn_stream_kernel(AttnArgs a) {
  using S = AttnTileShape<D>;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int QPI = PREFILL_ROWS / G;
  constexpr int RING = 8;           // claim position p lives in slot p % RING
  static_assert(QPI % 64 == 0 || QPI < 64, "query slot fetch");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_attn[];
  __shared__ int s_ring[RING];
  __shared__ int s_over[4];
  __shared__ int s_queue[16];
  __shared__ __attribute__((aligned(16))) int s_qslots[RING][QPI < 64 ? 64 : QPI];   // the fetch writes 64 lanes

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const float NEG_INF = -INFINITY;
  const int home = blockIdx.x & 7;
  int probe = 0;

  // --- per-lane address bases ----------------------------------------------------
  // Recomputed from a fresh copy of the thread index (opaque to the compiler)
  // at every step and wherever the rows are needed, so that none of them is
  // held in a register across the loop.
  auto fresh_lane = [&]() -> int {
    int v = threadIdx.x & 63;
    asm volatile("" : "+v"(v));
    return v;
  };
  uint32_t kslot[2], vslot;
  int kbase[8], vbase[4];
  auto refresh_bases = [&]() {
    const int ln = fresh_lane();
    const int lr = ln & 31, lg = ln >> 5;
    const int r0 = wave * S::ROWS_PER_INST + ln / S::CH;
    const int cpos = ln % S::CH;
    kslot[0] = (uint32_t)((cpos ^ (r0 & 15)) * 16);
    kslot[1] = (uint32_t)((cpos ^ ((r0 + 4 * S::ROWS_PER_INST) & 15)) * 16);
    vslot = (uint32_t)((cpos ^ ((r0 & 3) << 2)) * 16);
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) kbase[s8] = lr * S::ROW_BYTES + 16 * ((2 * s8 + lg) ^ (lr & 15));
    const int i16 = ln & 15, hh = (ln >> 4) & 1;
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4)
      vbase[d4] = (4 * lg + (i16 >> 2)) * S::ROW_BYTES + 16 * (4 * (d4 ^ (i16 >> 2)) + 2 * hh + ((i16 & 3) >> 1)) +
                  8 * (i16 & 1);
  };
  // this lane's rows: group x is R = 64 wave + 32 x + (lane % 32) -> (query slot R / G, head R % G)
  auto row_i = [&](int x) { return (wave * 64 + x * 32 + (fresh_lane() & 31)) / G; };
  auto row_j = [&](int x) { return (wave * 64 + x * 32 + (fresh_lane() & 31)) % G; };
  // stream tile s: its K tile in K buffer s % NB, its V tile in V buffer (s + 1) % NB
  auto kbuf_at = [&](int i) { return smem_attn + (i & (ATTN_NB - 1)) * S::TILE_BYTES; };
  auto vbuf_at = [&](int i) { return smem_attn + (ATTN_NB + (i & (ATTN_NB - 1))) * S::TILE_BYTES; };
  static_assert((ATTN_NB & (ATTN_NB - 1)) == 0, "buffer count is a power of two");

  // --- claims (thread 0): per-XCD queues with stealing ---------------------------
  if (threadIdx.x < 16) s_queue[threadIdx.x] = a.queue[threadIdx.x];
  int pend = 0;
  if (threadIdx.x == 0) pend = atomicAdd(&a.queue[16 + home], 1);
  __syncthreads();
  auto claim = [&]() -> int {
    int claimed = -1;
    for (;;) {
      const int x = (home + probe) & 7;
      if (pend < s_queue[x]) {
        claimed = s_queue[8 + x] + pend;
        break;
      }
      if (++probe == 8) break;
      pend = atomicAdd(&a.queue[16 + ((home + probe) & 7)], 1);
    }
    if (claimed >= 0) pend = atomicAdd(&a.queue[16 + ((home + probe) & 7)], 1);
    return claimed;
  };
  int last_claim = 0;               // thread 0: once a claim fails, every later one is -1
  auto claim_into = [&](int pos) {
    if (threadIdx.x == 0) {
      last_claim = last_claim >= 0 ? claim() : -1;
      s_ring[pos & (RING - 1)] = last_claim;
    }
  };
  auto ring_index = [&](int pos) -> int { return __builtin_amdgcn_readfirstlane(s_ring[pos & (RING - 1)]); };

  // --- items (uniform fields) ------------------------------------------------------
  struct Item {
    int idx, h, c, qb, qn, nkeys, ntiles;
    int64_t entry0;
    const bf16_t* kp;
    const bf16_t* vp;
    uint32_t rsb;
  };
  auto resolve = [&](int idx) -> Item {
    Item it;
    it.idx = idx;
    if (idx < 0) {
      it.h = it.c = it.qb = it.qn = it.nkeys = it.ntiles = 0;
      it.entry0 = 0;
      it.kp = it.vp = uniform_ptr(a.q);
      it.rsb = 0;
      return it;
    }
    const PrefillItem r = load_item(a.items, idx);
    it.h = __builtin_amdgcn_readfirstlane(r.h);
    it.c = __builtin_amdgcn_readfirstlane(r.c);
    it.qb = __builtin_amdgcn_readfirstlane(r.qb);
    it.qn = __builtin_amdgcn_readfirstlane(r.qn);
    it.entry0 = __builtin_amdgcn_readfirstlane(r.entry0);
    const bool local = it.c < 0;
    const int64_t row0 = __builtin_amdgcn_readfirstlane(r.row0);
    const int nk = local ? (int)(a.chunk_start + it.qb + it.qn - a.wstart) : __builtin_amdgcn_readfirstlane(r.nkeys);
    it.nkeys = max(__builtin_amdgcn_readfirstlane(nk), 0);
    it.ntiles = max(1, (it.nkeys + KT - 1) / KT);
    const bf16_t* kp;
    const bf16_t* vp;
    int64_t rs;
    if (local) {
      kp = a.korig + (int64_t)it.h * a.o_sh;
      vp = a.vorig + (int64_t)it.h * a.o_sh;
      rs = a.o_st;
    } else {
      kp = a.packed + row0 * a.Hkv * D + (int64_t)it.h * D;
      vp = kp + a.packed_len * a.Hkv * D;
      rs = (int64_t)a.Hkv * D;
    }
    it.kp = uniform_ptr(kp);
    it.vp = uniform_ptr(vp);
    it.rsb = (uint32_t)__builtin_amdgcn_readfirstlane((int)(rs * 2));
    return it;
  };
  // a cluster item's query slots into s_qslots[pos % RING] (wave 0, loads into LDS)
  auto fetch_slots = [&](int pos) {
    if (wave != 0) return;
    const int idx = ring_index(pos);
    if (idx < 0) return;
    const PrefillItem r = load_item(a.items, idx);
    const int c = __builtin_amdgcn_readfirstlane(r.c);
    if (c < 0) return;
    const int qn = __builtin_amdgcn_readfirstlane(r.qn);
    const uint64_t b = (uint64_t)(a.qvals + __builtin_amdgcn_readfirstlane(r.entry0));
    u32x4_t rsrc;
    rsrc.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
    rsrc.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
    rsrc.z = (uint32_t)qn * 4u;
    rsrc.w = (uint32_t)BUFFER_CONFIG;
    const uint32_t dst =
        __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)s_qslots[pos & (RING - 1)]);
#pragma unroll
    for (int k = 0; k < QPI; k += 64) lds_dma4(rsrc, dst + 4 * k, (uint32_t)(lane + k) * 4u);
  };
  // this lane's query of group x (-1 past the item's queries)
  auto query_of = [&](const Item& it, int x, int pos) -> int {
    if (row_i(x) >= it.qn) return -1;
    const int q = it.c < 0 ? it.qb + row_i(x) : s_qslots[pos & (RING - 1)][row_i(x)];
    return min(max(q, 0), a.Qc - 1);
  };
  u32x4_t qr[2][KS];
  auto load_q = [&](const Item& it, const int (&qi)[2]) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const bf16_t* src = a.q + (int64_t)max(qi[x], 0) * a.q_sq + (int64_t)(it.h * G + row_j(x)) * a.q_sh + g * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) qr[x][s] = *reinterpret_cast<const u32x4_t*>(src + s * 16);
    }
  };

  // --- tile loads --------------------------------------------------------------------
  struct DmaPlan {
    u32x4_t rsrc;
    uint32_t dst, kvoff, rsb;
  };
  // tile t of an item (an empty range for no item or t < 0: the loads then
  // only write zeros, so every step issues the same number)
  auto plan_tile = [&](const Item& it, bool is_k, int t, unsigned char* dst_tile) -> DmaPlan {
    const int t0 = t * KT;
    const int rows = (it.idx < 0 || t < 0) ? 0 : max(it.nkeys - t0, 0);
    const int valid = __builtin_amdgcn_readfirstlane((int)((uint32_t)rows * it.rsb));
    const bf16_t* base = is_k ? it.kp : it.vp;
    const uint64_t b = (uint64_t)((const unsigned char*)base + (uint64_t)max(t0, 0) * it.rsb);
    DmaPlan pl;
    pl.rsrc.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
    pl.rsrc.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
    pl.rsrc.z = (uint32_t)valid;
    pl.rsrc.w = (uint32_t)BUFFER_CONFIG;
    pl.dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)(dst_tile + wave * 1024));
    pl.kvoff = (uint32_t)(wave * S::ROWS_PER_INST + fresh_lane() / S::CH) * it.rsb;
    pl.rsb = it.rsb;
    return pl;
  };
  auto dma_one = [&](const DmaPlan& pl, int m, bool is_k) {
    const uint32_t roff = pl.kvoff + (uint32_t)(m * 4 * S::ROWS_PER_INST) * pl.rsb;
    const uint32_t slot = is_k ? kslot[m & 1] : vslot;
    lds_dma16(pl.rsrc, pl.dst + m * 4096, roff + slot);
  };

  // --- GEMMs ---------------------------------------------------------------------------
  constexpr int KA_AHEAD = 3;
  auto kread = [&](const unsigned char* sK, int s) -> u32x4_t {
    return *reinterpret_cast<const u32x4_t*>(sK + kbase[s & 7] + 256 * (s >> 3));
  };
  auto gemm_s = [&](f32x16_t (&sacc)[2], const unsigned char* sK) {
    u32x4_t ka[KA_AHEAD];
#pragma unroll
    for (int f = 0; f < KA_AHEAD; ++f) ka[f] = kread(sK, f);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4_t cur = ka[s % KA_AHEAD];
      if (s + KA_AHEAD < KS) ka[s % KA_AHEAD] = kread(sK, s + KA_AHEAD);
      if (s == 0) {
        s_mfma_first(sacc[0], cur, qr[0][s]);
        s_mfma_first(sacc[1], cur, qr[1][s]);
      } else {
        s_mfma_acc(sacc[0], cur, qr[0][s]);
        s_mfma_acc(sacc[1], cur, qr[1][s]);
      }
    }
    s_mfma_results_to_valu(sacc[0], sacc[1]);
  };
  auto vread = [&](const unsigned char* sV, int f) -> u32x4_t {
    const int m = f / DT, dt = f % DT;
    const unsigned char* p = sV + vbase[dt & 3] + 256 * (dt >> 2) + 16 * m * S::ROW_BYTES;
    s16x4_t part[2];
    part[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
    part[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + 8 * S::ROW_BYTES));
    u32x4_t r;
    __builtin_memcpy(&r, part, 16);
    return r;
  };
  f32x16_t o[2][DT];
  auto zero_o = [&]() {
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        acc_zero_tile(o[x][dt]);
  };
  // --- the softmax pieces and the rows' state ---------------------------------------
  struct RowState {
    int qidx[2];
    float m_ref[2], l[2];
  };
  const float lim = __builtin_exp2f(RESCALE_LOG2);
  auto row_max = [&](const f32x16_t (&sacc)[2], float (&mx)[2]) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      float v = NEG_INF;
#pragma unroll
      for (int e = 0; e < 16; e += 4)
        v = fmaxf(v, fmaxf(fmaxf(sacc[x][e], sacc[x][e + 1]), fmaxf(sacc[x][e + 2], sacc[x][e + 3])));
      mx[x] = halves_max(v);
    }
  };
  auto exp_pack = [&](f32x16_t (&sacc)[2], const float (&m)[2], u32x4_t (&pb)[2][2], float (&sum)[2]) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sacc[x][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[x][e], a.scale_log2, -m[x]));
        acc += sacc[x][e];
      }
      sum[x] = acc;
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        pb[x][mm].x = pack2bf(sacc[x][8 * mm + 0], sacc[x][8 * mm + 1]);
        pb[x][mm].y = pack2bf(sacc[x][8 * mm + 2], sacc[x][8 * mm + 3]);
        pb[x][mm].z = pack2bf(sacc[x][8 * mm + 4], sacc[x][8 * mm + 5]);
        pb[x][mm].w = pack2bf(sacc[x][8 * mm + 6], sacc[x][8 * mm + 7]);
      }
    }
  };
  // An item's rows: normalise and store straight from the accumulators (a
  // swap of the lane halves gives each lane whole 16-byte chunks).  Every lane
  // issues EPI_STORES buffer stores; a row past the item's queries (and the
  // LSE store of lanes g = 1) is given an offset past the buffer's range.  An
  // item with a row past the probability bound is listed for the recomputing
  // pass instead, and stores nothing (the return value says whether the
  // stores were issued).
  constexpr int EPI_STORES = 2 * (2 * DT + 1);
  // an offset past every range used here (ranges stay below 2^31 bytes), so
  // that adding the access size cannot wrap
  constexpr int OUT_OF_RANGE = (int)0x80000000u;
  auto epilogue = [&](const Item& it, const RowState& rs, bool over) -> bool {
    // any row of the block past the bound: one word per wave, one barrier
    // (the words are rewritten only at the next item's end, several
    // barriers later)
    const bool wave_over = __ballot(over) != 0;
    if ((threadIdx.x & 63) == 0) s_over[wave] = wave_over ? 1 : 0;
    __syncthreads();
    const bool redo = (s_over[0] | s_over[1] | s_over[2] | s_over[3]) != 0;
    if (redo) {
      if (threadIdx.x == 0) {
        const int k = atomicAdd(&a.queue[QUEUE_OVF_N], 1);
        a.queue[QUEUE_OVF_LIST + k] = it.idx;
      }
      return false;
    }
    // the accumulators' last MFMAs are done (20 wait states before the
    // written reads, more than a 16-pass result needs)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::: "memory");
    const bool local = it.c < 0;
    // uniform bases and ranges: the item's output rows and its LSE values
    const bf16_t* obase;
    int64_t obytes;
    const float* lbase;
    int64_t lbytes;
    if (local) {
      obase = a.local_o + (int64_t)it.qb * a.lo_sq + (int64_t)(it.h * G) * a.lo_sh;
      obytes = ((int64_t)(it.qn - 1) * a.lo_sq + (int64_t)(G - 1) * a.lo_sh + D) * 2;
      lbase = a.local_lse ? a.local_lse : (const float*)a.q;
      lbytes = a.local_lse ? (int64_t)a.Qc * a.Hq * 4 : 0;
    } else {
      obase = a.part_o + it.entry0 * G * D;
      obytes = (int64_t)it.qn * G * D * 2;
      lbase = a.part_lse + it.entry0 * G;
      lbytes = (int64_t)it.qn * G * 4;
    }
    const __amdgpu_buffer_rsrc_t orsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)uniform_ptr(obase), 0, (int)obytes, BUFFER_CONFIG);
    // (each half through a uint32_t: readfirstlane returns int, which would
    // sign-extend into the high dword)
    const uint64_t lb = (uint64_t)lbase;
    const uint32_t lb_lo = __builtin_amdgcn_readfirstlane((uint32_t)lb);
    const uint32_t lb_hi = __builtin_amdgcn_readfirstlane((uint32_t)(lb >> 32));
    const float* lbase_u = (const float*)(((uint64_t)lb_hi << 32) | (uint64_t)lb_lo);
    const __amdgpu_buffer_rsrc_t lrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)lbase_u, 0, (int)lbytes, BUFFER_CONFIG);
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const float l = halves_sum(rs.l[x]);
      const float inv = (l > 0.f) ? 1.0f / l : 0.f;
      const int qi = rs.qidx[x];
      const int i = row_i(x), j = row_j(x);
      const bool valid = qi >= 0;
      {
        const float lse = (l > 0.f) ? (rs.m_ref[x] + log2f(l)) * 0.69314718055994531f : NEG_INF;
        const int64_t loff = local ? ((int64_t)qi * a.Hq + it.h * G + j) * 4 : (int64_t)(i * G + j) * 4;
        const int off = (valid && g == 0) ? (int)loff : OUT_OF_RANGE;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lse), lrsrc, off, 0, 0);
      }
      const int64_t roff = local ? ((int64_t)i * a.lo_sq + (int64_t)j * a.lo_sh) * 2 : (int64_t)(i * G + j) * D * 2;
      const int rbase = valid ? (int)roff : OUT_OF_RANGE;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int qa = 2 * p, qb2 = 2 * p + 1;
          float v[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = acc_read(o[x][dt][4 * qa + e]);
            v[4 + e] = acc_read(o[x][dt][4 * qb2 + e]);
          }
          const uint32_t a0 = pack2bf(v[0] * inv, v[1] * inv);
          const uint32_t a1 = pack2bf(v[2] * inv, v[3] * inv);
          const uint32_t b0 = pack2bf(v[4] * inv, v[5] * inv);
          const uint32_t b1 = pack2bf(v[6] * inv, v[7] * inv);
          const auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
          u32x4_t w;
          w.x = s0[0];
          w.y = s1[0];
          w.z = s0[1];
          w.w = s1[1];
          const int off = valid ? rbase + 16 * (4 * dt + 2 * p + g) : OUT_OF_RANGE;
          __builtin_amdgcn_raw_buffer_store_b128(w, orsrc, off, 0, 2);
        }
    }
    return true;
  };

  // ====================================================================================
  // prologue: claims of positions 0 and 1 and their query slots, then the
  // loads of virtual steps 1 - NB .. -1
  // Claims: positions 0 .. AHEAD - 1 here, position p + AHEAD at the top of
  // the step whose S^T starts position p.  After a step's loads the load
  // cursor points at the tile NB steps past that step's S^T, which can be NB
  // positions ahead of it (items of one tile), and it then fetches the query
  // slots of the position after that one: AHEAD = NB + 1 keeps every ring
  // entry the cursor reads claimed, and claimed at least one barrier earlier
  // where waves other than the claiming one read it.  The ring holds
  // positions p .. p + AHEAD.  (Entries start at -1, no item.)
  constexpr int AHEAD = ATTN_NB + 1;
  static_assert(AHEAD + 1 <= RING, "claim ring");
  if (threadIdx.x < RING) s_ring[threadIdx.x] = -1;
  __syncthreads();
  for (int p = 0; p < AHEAD; ++p) claim_into(p);
  __syncthreads();
  if (ring_index(0) < 0) return;
  fetch_slots(0);
  fetch_slots(1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // load cursor: claim position ip, tile it_tile of the next K tile to load;
  // (vq_item, vq_tile): the K tile loaded last step, whose V tile loads next
  int ip = 0, it_tile = 0;
  Item iss = resolve(ring_index(0));
  Item vq_item = iss;
  int vq_tile = -1;
  // step s's loads: K of stream tile s + NB - 1 and V of stream tile s + NB - 2.
  // Entering a new position (at most one per step) fetches the query slots of
  // the position after it.
  auto plan_step = [&](int s, DmaPlan& pk, DmaPlan& pv) {
    pk = plan_tile(iss, true, it_tile, kbuf_at(s + ATTN_NB - 1));
    pv = plan_tile(vq_item, false, vq_tile, vbuf_at(s + ATTN_NB - 1));
    vq_item = iss;
    vq_tile = iss.idx < 0 ? -1 : it_tile;
    if (iss.idx >= 0 && ++it_tile == iss.ntiles) {
      ++ip;
      it_tile = 0;
      iss = resolve(ring_index(ip));
      if (iss.idx >= 0) fetch_slots(ip + 1);
    }
  };
  for (int v = 1 - ATTN_NB; v < 0; ++v) {
    refresh_bases();
    DmaPlan pk, pv;
    plan_step(v, pk, pv);
#pragma unroll
    for (int m = 0; m < S::PER_WAVE; ++m) dma_one(pk, m, true);
#pragma unroll
    for (int m = 0; m < S::PER_WAVE; ++m) dma_one(pv, m, false);
    __syncthreads();
  }

  // consume cursor: claim position cp, tile ct of the tile whose S^T runs next
  int cp = 0, ct = 0;
  Item cur = resolve(ring_index(0));
  Item prev = cur;
  RowState rs_cur, rs_prev;
  rs_cur.qidx[0] = query_of(cur, 0, 0);
  rs_cur.qidx[1] = query_of(cur, 1, 0);
  rs_cur.l[0] = rs_cur.l[1] = 0.f;
  rs_cur.m_ref[0] = rs_cur.m_ref[1] = 0.f;
  rs_prev = rs_cur;
  load_q(cur, rs_cur.qidx);
  bool over_cur = false, over_prev = false;
  // causal limits of the current item (local window items): the key limit per
  // row and the wave's smallest limit over its valid rows (tiles wholly below
  // it need no mask)
  int qlim[2], wave_min = 0x7fffffff;
  auto setup_limits = [&]() {
    const bool local = cur.c < 0;
    wave_min = 0x7fffffff;
#pragma unroll
    for (int x = 0; x < 2; ++x)
      qlim[x] = local ? (int)(a.chunk_start + rs_cur.qidx[x] - a.wstart) : 0x7fffffff;
    if (local) {
      wave_min = min(rs_cur.qidx[0] >= 0 ? qlim[0] : 0x7fffffff, rs_cur.qidx[1] >= 0 ? qlim[1] : 0x7fffffff);
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) wave_min = min(wave_min, __shfl_xor(wave_min, off, 64));
      wave_min = __builtin_amdgcn_readfirstlane(wave_min);
    }
  };
  setup_limits();
  zero_o();
  u32x4_t pb_prev[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) pb_prev[x][mm] = u32x4_t{0u, 0u, 0u, 0u};
  bool pv_pending = false;          // an item's last tile waits for its second GEMM
  bool stored = false;              // the last step stored an item's rows

  constexpr int VM_KEEP = (ATTN_NB - 2) * 2 * S::PER_WAVE;
  static_assert(VM_KEEP + EPI_STORES <= 63, "vmcnt range");
  // after a step: the tile S^T ran on waits for its second GEMM; move to the
  // next tile, or the next item (its Q rows load now: this item's last S^T is
  // done)
  // One step: S^T of stream tile s (tile ct of cur) and O += V P of stream
  // tile s - 1, with the loads of step s between the second GEMM's MFMAs.
  // FIRST: the tile starts cur (the rows' reference maxima come from it) and
  // tile s - 1, if any, was prev's last.  A step that starts an item waits for
  // every load (its Q rows were the last); the others keep VM_KEEP loads in
  // flight, plus the stores of an item's rows the step before issued.
  int s = 0;
  auto step = [&](auto first_tag) {
    constexpr bool FIRST = decltype(first_tag)::value;
    if (FIRST) {
      __builtin_amdgcn_s_waitcnt(0);
      if (cur.idx >= 0) claim_into(cp + AHEAD);
    } else if (stored) {
      constexpr int keep = VM_KEEP + EPI_STORES;
      __builtin_amdgcn_s_waitcnt((keep & 15) | ((keep >> 4) << 14) | (7 << 4));
    } else {
      __builtin_amdgcn_s_waitcnt((VM_KEEP & 15) | ((VM_KEEP >> 4) << 14) | (7 << 4));
    }
    stored = false;
    __syncthreads();
    refresh_bases();
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) asm volatile("" : "+a"(o[x][dt]));
    DmaPlan pk, pv;
    plan_step(s, pk, pv);
    // A tile that no row of the wave sees (past its causal limits, or no
    // tile at all) is masked whole: its probabilities are zero, and its
    // second GEMM adds nothing.  The V tile of no tile is zeros (an empty
    // load range).
    const int t0 = ct * KT;
    f32x16_t sc[2];
    gemm_s(sc, kbuf_at(s));
    if (t0 + KT > cur.nkeys || t0 + KT - 1 > wave_min) {
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = t0 + 8 * (e >> 2) + 4 * g + (e & 3);
          if (!(key < cur.nkeys && key <= qlim[x])) sc[x][e] = NEG_INF;
        }
    }
    if (FIRST) {
      // reference maximum: the rows' maxima over the item's first tile (key
      // 0 of an item is visible to every row, so it is finite)
      float mx[2];
      row_max(sc, mx);
#pragma unroll
      for (int x = 0; x < 2; ++x) rs_cur.m_ref[x] = (mx[x] == NEG_INF) ? 0.f : mx[x] * a.scale_log2;
    }
    // O += V(s-1) P(s-1) with the softmax of S(s) woven between its MFMAs,
    // fragment by fragment, and one tile load after every other fragment
    // (scheduling barriers keep the order)
    const unsigned char* sV = vbuf_at(s);
    constexpr int NF = DT * 2;
    constexpr int VA_AHEAD = 3;
    u32x4_t va[VA_AHEAD];
#pragma unroll
    for (int f = 0; f < VA_AHEAD; ++f) va[f] = vread(sV, f);
    float sum[2] = {0.f, 0.f};
    uint32_t pkd[2][8];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const u32x4_t cv = va[f % VA_AHEAD];
      if (f + VA_AHEAD < NF) va[f % VA_AHEAD] = vread(sV, f + VA_AHEAD);
      const int m = f / DT, dt = f % DT;
      o[0][dt] = mfma32x32x16(as_bf16x8(cv), as_bf16x8(pb_prev[0][m]), o[0][dt]);
      o[1][dt] = mfma32x32x16(as_bf16x8(cv), as_bf16x8(pb_prev[1][m]), o[1][dt]);
#pragma unroll
      for (int k = 0; k < 32 / NF; k += 2) {
        const int q = f * (32 / NF) + k;
        const int x = q / 16, e = q % 16;
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[x][e], a.scale_log2, -rs_cur.m_ref[x]));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[x][e + 1], a.scale_log2, -rs_cur.m_ref[x]));
        sum[x] += p0 + p1;
        pkd[x][e / 2] = pack2bf(p0, p1);
      }
      static_assert(NF >= 4 * S::PER_WAVE, "one load instruction per two fragments");
      if (f % 2 == 0 && f / 2 < 2 * S::PER_WAVE) {
        const int mi = f / 2;
        if (mi < S::PER_WAVE) dma_one(pk, mi, true);
        else dma_one(pv, mi - S::PER_WAVE, false);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        pb_prev[x][mm].x = pkd[x][4 * mm + 0];
        pb_prev[x][mm].y = pkd[x][4 * mm + 1];
        pb_prev[x][mm].z = pkd[x][4 * mm + 2];
        pb_prev[x][mm].w = pkd[x][4 * mm + 3];
      }
    over_cur |= !(sum[0] <= lim) || !(sum[1] <= lim);
    rs_cur.l[0] += sum[0];
    rs_cur.l[1] += sum[1];
    ++s;
  };

  for (;;) {
    // cur's first tile (none past the last item) and prev's last second GEMM,
    // then prev's rows
    step(std::true_type{});
    if (pv_pending) stored = epilogue(prev, rs_prev, over_prev);
    if (cur.idx < 0) break;
    zero_o();
    for (ct = 1; ct < cur.ntiles; ++ct) step(std::false_type{});
    // cur's last S^T is done: the next item, whose Q rows load now
    pv_pending = true;
    prev = cur;
    rs_prev = rs_cur;
    over_prev = over_cur;
    ++cp;
    ct = 0;
    cur = resolve(ring_index(cp));
    over_cur = false;
    rs_cur.l[0] = rs_cur.l[1] = 0.f;
    if (cur.idx >= 0) {
      rs_cur.qidx[0] = query_of(cur, 0, cp);
      rs_cur.qidx[1] = query_of(cur, 1, cp);
      load_q(cur, rs_cur.qidx);
      setup_limits();
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
}


// S6: per (query, KV head), one wave.  The reference folds the query's
// partials into the window's result one cluster at a time (online
// log-sum-exp, cluster order).  Here the wave first lists the query's entries
// (lanes test 64 clusters at once), takes the maximum of all the LSEs, and then
// sums exp(lse - max)-weighted partials with four entries' loads in flight, so
// no load waits on the previous fold.  The result is the same merge, rounded
// once instead of per step.  Each lane owns E = G*D/64 consecutive values of
// one head.
constexpr int COMBINE_MAX_LIST = 1024;   // entries per (query, head): at most C

template <int E>
__device__ __forceinline__ void load_bf16_row(const bf16_t* src, float (&v)[E]) {
  if constexpr (E % 8 == 0) {
#pragma unroll
    for (int k = 0; k < E / 8; ++k) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(src + 8 * k);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v[8 * k + 2 * t] = __uint_as_float(ww[t] << 16);
        v[8 * k + 2 * t + 1] = __uint_as_float(ww[t] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = bf2f(src[e]);
  }
}

template <int D, int G>
__global__ __launch_bounds__(256) void combine_kernel(
    const int32_t* __restrict__ qmask, const int32_t* __restrict__ nvis,
    const int32_t* __restrict__ rev_indptr, const int32_t* __restrict__ qrank,
    const bf16_t* __restrict__ part_o, const float* __restrict__ part_lse,
    const bf16_t* __restrict__ local_o, int64_t lo_sq, int64_t lo_sh,
    const float* __restrict__ local_lse, bf16_t* __restrict__ out, int64_t out_sq, int64_t out_sh,
    float* __restrict__ out_lse, int Qc, int Hkv, int C) {
  constexpr int E = G * D / 64;
  static_assert(E >= 1 && D % E == 0, "lane share");
  __shared__ int s_list[4][COMBINE_MAX_LIST];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t gw = (int64_t)blockIdx.x * 4 + wave;
  if (gw >= (int64_t)Qc * Hkv) return;
  const int qi = (int)(gw / Hkv), h = (int)(gw % Hkv);
  const int j = (lane * E) / D, d0 = (lane * E) % D;
  const int Hq = Hkv * G;
  int* list = s_list[wave];

  // the query's entries, in cluster order
  const int32_t* qm = qmask + ((int64_t)qi * Hkv + h) * (C / 32);
  const int32_t* qr = qrank + ((int64_t)qi * Hkv + h) * C;
  const uint64_t below = (1ull << lane) - 1;
  int n = 0;
  for (int c0 = 0; c0 < C; c0 += 64) {
    const int c = c0 + lane;
    bool sel = false;
    int entry = 0;
    if (c < C && (((uint32_t)qm[c >> 5] >> (c & 31)) & 1u) && nvis[h * C + c] > 0) {
      sel = true;
      entry = rev_indptr[h * C + c] + qr[c];
    }
    const uint64_t m = __ballot(sel);
    if (sel) list[n + __popcll(m & below)] = entry;
    n += __popcll(m);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // the largest LSE: the window's and every partial's
  const float lse_w = local_lse[(int64_t)qi * Hq + h * G + j];
  float mx = lse_w;
  for (int k = 0; k < n; k += 4) {
    float l4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) l4[u] = k + u < n ? part_lse[(int64_t)list[k + u] * G + j] : -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u) mx = fmaxf(mx, l4[u]);
  }

  float acc[E];
  float den;
  {
    float v[E];
    load_bf16_row<E>(local_o + (int64_t)qi * lo_sq + (int64_t)(h * G + j) * lo_sh + d0, v);
    den = expf(lse_w - mx);
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = v[e] * den;
  }
  for (int k = 0; k < n; k += 4) {
    float v[4][E], wt[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool ok = k + u < n;
      const int64_t entry = ok ? list[k + u] : 0;
      wt[u] = ok ? part_lse[entry * G + j] : -INFINITY;
      if (ok) load_bf16_row<E>(part_o + (entry * G + j) * D + d0, v[u]);
      else
#pragma unroll
        for (int e = 0; e < E; ++e) v[u][e] = 0.f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float w = expf(wt[u] - mx);
      den += w;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = fmaf(v[u][e], w, acc[e]);
    }
  }
  const float inv = 1.0f / fmaxf(den, 1e-30f);
  bf16_t* dst = out + (int64_t)qi * out_sq + (int64_t)(h * G + j) * out_sh + d0;
  if constexpr (E % 8 == 0) {
#pragma unroll
    for (int k = 0; k < E / 8; ++k) {
      u32x4_t w;
      w.x = pack2bf(acc[8 * k + 0] * inv, acc[8 * k + 1] * inv);
      w.y = pack2bf(acc[8 * k + 2] * inv, acc[8 * k + 3] * inv);
      w.z = pack2bf(acc[8 * k + 4] * inv, acc[8 * k + 5] * inv);
      w.w = pack2bf(acc[8 * k + 6] * inv, acc[8 * k + 7] * inv);
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(dst + 8 * k));
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) dst[e] = f2bf(acc[e] * inv);
  }
  if (out_lse && (lane * E) % D == 0) out_lse[(int64_t)qi * Hq + h * G + j] = mx + logf(den);
}

// one kernel's launch over a persistent grid (one block per CU at its LDS size)
template <typename K>
int launch_persistent(K kernel, size_t lds, const AttnArgs& a, int grid, int& auto_grid, bool& configured,
                      hipStream_t stream) {
  if (!configured) {
    if (hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
        hipSuccess)
      return SBSA_ERR_UNSUPPORTED;
    configured = true;
  }
  if (grid <= 0) {
    if (!auto_grid) {
      int dev = 0, cus = 0, occ = 0;
      (void)hipGetDevice(&dev);
      (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)kernel, 256, lds);
      auto_grid = (cus > 0 ? cus : 256) * (occ > 0 ? occ : 1);
    }
    grid = auto_grid;
  }
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), lds, stream, a);
  return SBSA_OK;
}

// the main pass, then the recomputation of the items it listed as past the
// probability bound (an empty list ends that launch at once)
template <int D, int G>
int launch_attn(const AttnArgs& a, int grid, hipStream_t stream) {
  const size_t lds = AttnTileShape<D>::lds_bytes();
  static bool conf_main = false, conf_redo = false;
  static int grid_main = 0, grid_redo = 0;
  int rc = launch_persistent(attn_stream_kernel<D, G>, lds, a, grid, grid_main, conf_main, stream);
  if (rc) return rc;
  return launch_persistent(attn_items_kernel<D, G, true>, lds, a, grid, grid_redo, conf_redo, stream);
}

template <int D, int G>
int launch_combine(const int32_t* qmask, const int32_t* nvis, const int32_t* rev_indptr,
                   const int32_t* qrank, const bf16_t* part_o, const float* part_lse,
                   const bf16_t* local_o, int64_t lo_sq, int64_t lo_sh, const float* local_lse,
                   bf16_t* out, int64_t out_sq, int64_t out_sh, float* out_lse, int Qc, int Hkv,
                   int C, hipStream_t stream) {
  int64_t waves = (int64_t)Qc * Hkv;
  hipLaunchKernelGGL((combine_kernel<D, G>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     stream, qmask, nvis, rev_indptr, qrank, part_o, part_lse, local_o, lo_sq,
                     lo_sh, local_lse, out, out_sq, out_sh, out_lse, Qc, Hkv, C);
  return SBSA_OK;
}

#define SBSA_DISPATCH_DG(D_, G_, FN, ...)                            \
  do {                                                               \
    if (D_ == 128 && G_ == 1) return FN<128, 1>(__VA_ARGS__);        \
    if (D_ == 128 && G_ == 2) return FN<128, 2>(__VA_ARGS__);        \
    if (D_ == 128 && G_ == 4) return FN<128, 4>(__VA_ARGS__);        \
    if (D_ == 128 && G_ == 8) return FN<128, 8>(__VA_ARGS__);        \
    if (D_ == 256 && G_ == 1) return FN<256, 1>(__VA_ARGS__);        \
    if (D_ == 256 && G_ == 2) return FN<256, 2>(__VA_ARGS__);        \
    if (D_ == 256 && G_ == 4) return FN<256, 4>(__VA_ARGS__);        \
    if (D_ == 256 && G_ == 8) return FN<256, 8>(__VA_ARGS__);        \
    return SBSA_ERR_UNSUPPORTED;                                     \
  } while (0)

int attn_dispatch(int D, int G, const AttnArgs& a, int grid, hipStream_t stream) {
  SBSA_DISPATCH_DG(D, G, launch_attn, a, grid, stream);
}

int combine_dispatch(int D, int G, const int32_t* qmask, const int32_t* nvis,
                     const int32_t* rev_indptr, const int32_t* qrank, const bf16_t* part_o,
                     const float* part_lse, const bf16_t* local_o, int64_t lo_sq, int64_t lo_sh,
                     const float* local_lse, bf16_t* out, int64_t out_sq, int64_t out_sh,
                     float* out_lse, int Qc, int Hkv, int C, hipStream_t stream) {
  SBSA_DISPATCH_DG(D, G, launch_combine, qmask, nvis, rev_indptr, qrank, part_o, part_lse, local_o,
                   lo_sq, lo_sh, local_lse, out, out_sq, out_sh, out_lse, Qc, Hkv, C, stream);
}

}  // namespace

extern "C" {

int sbsa_prefill_item_rows(void) { return PREFILL_ROWS; }

int sbsa_prefill_attend(const void* q, int64_t q_sq, int64_t q_sh, int num_queries,
                        int num_q_heads, int num_kv_heads, int dim, const void* packed,
                        int64_t packed_len, const void* k_orig, const void* v_orig, int64_t o_st,
                        int64_t o_sh, const int32_t* indptr, const int32_t* nvis, int num_clusters,
                        const int32_t* rev_indptr, const int32_t* qvals, const void* items,
                        int32_t* queue, void* part_o, float* part_lse,
                        void* local_o, int64_t lo_sq, int64_t lo_sh, float* local_lse,
                        int64_t chunk_start, int64_t wstart, float sm_scale, int grid,
                        hipStream_t stream) {
  if (!q || !k_orig || !v_orig || !items || !queue || !local_o) return SBSA_ERR_ARG;
  if (num_kv_heads < 1 || num_q_heads % num_kv_heads) return SBSA_ERR_ARG;
  if (q_sq % 8 || q_sh % 8 || o_st % 8 || o_sh % 8 || lo_sq % 8 || lo_sh % 8) return SBSA_ERR_ARG;
  if (chunk_start < wstart || wstart < 0) return SBSA_ERR_ARG;
  // The tile loads address K/V through raw buffer resources whose range (the rows
  // left from a tile's first row, in bytes) is 32-bit: the longest row range a work
  // item can read, the window from wstart to the chunk's last query or a whole packed
  // run, must stay below 4 GiB.
  const int64_t window_bytes = (chunk_start + num_queries - wstart) * o_st * 2;
  const int64_t packed_bytes = packed ? packed_len * num_kv_heads * (int64_t)dim * 2 : 0;
  if (window_bytes >= (int64_t(1) << 32) || packed_bytes >= (int64_t(1) << 32))
    return SBSA_ERR_UNSUPPORTED;
  AttnArgs a;
  a.q = (const bf16_t*)q;
  a.q_sq = q_sq;
  a.q_sh = q_sh;
  a.q_bytes = ((int64_t)(num_queries - 1) * q_sq + (int64_t)(num_q_heads - 1) * q_sh + dim) * 2;
  a.packed = (const bf16_t*)packed;
  a.packed_len = packed_len;
  a.korig = (const bf16_t*)k_orig;
  a.vorig = (const bf16_t*)v_orig;
  a.o_st = o_st;
  a.o_sh = o_sh;
  a.indptr = indptr;
  a.nvis = nvis;
  a.rev_indptr = rev_indptr;
  a.qvals = qvals;
  a.items = (const PrefillItem*)items;
  a.queue = queue;
  a.part_o = (bf16_t*)part_o;
  a.part_lse = part_lse;
  a.local_o = (bf16_t*)local_o;
  a.lo_sq = lo_sq;
  a.lo_sh = lo_sh;
  a.local_lse = local_lse;
  a.Hkv = num_kv_heads;
  a.C = num_clusters;
  a.Hq = num_q_heads;
  a.Qc = num_queries;
  a.chunk_start = chunk_start;
  a.wstart = wstart;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  int rc = attn_dispatch(dim, num_q_heads / num_kv_heads, a, grid, stream);
  if (rc) return rc;
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_prefill_combine(const int32_t* qmask, const int32_t* nvis, const int32_t* rev_indptr,
                         const int32_t* qrank, const void* part_o, const float* part_lse,
                         const void* local_o, int64_t lo_sq, int64_t lo_sh, const float* local_lse,
                         void* out, int64_t out_sq, int64_t out_sh, float* out_lse,
                         int num_queries, int num_q_heads, int num_kv_heads, int dim,
                         int num_clusters, hipStream_t stream) {
  if (!qmask || !nvis || !rev_indptr || !qrank || !local_o || !local_lse || !out) return SBSA_ERR_ARG;
  if (num_kv_heads < 1 || num_q_heads % num_kv_heads || num_clusters % 32) return SBSA_ERR_ARG;
  if (num_clusters > COMBINE_MAX_LIST) return SBSA_ERR_UNSUPPORTED;
  // rows are read and written in 16-byte pieces when a lane's share of a head is a
  // multiple of 8 values: every row start must then be 16-byte aligned
  if ((num_q_heads / num_kv_heads) * dim % 512 == 0 &&
      (out_sq % 8 || out_sh % 8 || lo_sq % 8 || lo_sh % 8 || ((uintptr_t)out & 15) ||
       ((uintptr_t)local_o & 15)))
    return SBSA_ERR_ARG;
  if (num_queries == 0) return SBSA_OK;
  int rc = combine_dispatch(dim, num_q_heads / num_kv_heads, qmask, nvis, rev_indptr, qrank,
                            (const bf16_t*)part_o, part_lse, (const bf16_t*)local_o, lo_sq, lo_sh,
                            local_lse, (bf16_t*)out, out_sq, out_sh, out_lse, num_queries,
                            num_kv_heads, num_clusters, stream);
  if (rc) return rc;
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

}  // extern "C"
