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
  int Qc;                   // queries of the chunk
  int64_t chunk_start, wstart;
  float scale_log2;         // sm_scale * log2(e)
#ifdef SBSA_ATTN_PROBE
  int probe_slot;
#endif
};

#ifdef SBSA_ATTN_PROBE
// timing probe (a build flag, not in the product): per launch slot and block,
// the wall clock at each item start, tagged with the item
struct ProbeRec { uint64_t t; int idx, ntiles, qn, c; };
constexpr int PROBE_SLOTS = 32, PROBE_BLOCKS = 256, PROBE_RECS = 640;
__device__ ProbeRec g_attn_probe[PROBE_SLOTS][PROBE_BLOCKS][PROBE_RECS];
__device__ __forceinline__ void probe_mark(const AttnArgs& a, int& k, int idx, int nt, int qn, int c) {
  if (threadIdx.x == 0 && a.probe_slot < PROBE_SLOTS && blockIdx.x < PROBE_BLOCKS && k < PROBE_RECS) {
    ProbeRec r;
    r.t = __builtin_amdgcn_s_memrealtime();
    r.idx = idx; r.ntiles = nt; r.qn = qn; r.c = c;
    g_attn_probe[a.probe_slot][blockIdx.x][k] = r;
  }
  ++k;
}
#define PROBE(...) probe_mark(a, probe_k, __VA_ARGS__)
#else
#define PROBE(...) ((void)0)
#endif

constexpr int KT = 32;                  // keys per tile
constexpr int PREFILL_ROWS = 128;       // (query, head) rows per work item: 32 per wave
// Probabilities are taken against a reference maximum per row and may reach
// 2^OVERFLOW_LOG2 (well inside fp32 and bf16 range) before an item is redone.
constexpr float OVERFLOW_LOG2 = 64.0f;
constexpr int BUFFER_CONFIG = 0x00020000;   // raw buffer resource, 32-bit data format
// an offset past every range a store uses here (ranges stay below 2^31 bytes,
// so adding the access size cannot wrap): such a store is dropped
constexpr int OUT_OF_RANGE = (int)0x80000000u;

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
  // K, K, V, V tiles; the pipelined kernel adds a staging area for its
  // epilogue (one 32-row slice per wave), the other stages in the tile buffers
  static constexpr size_t stage_offset(bool pipe) { return pipe ? 4 * (size_t)TILE_BYTES : 0; }
  static constexpr size_t lds_bytes(bool pipe) {
    return 4 * (size_t)TILE_BYTES + (pipe ? (size_t)PREFILL_ROWS * ROW_BYTES : 0);
  }
  static constexpr int ROWS_PER_INST = 64 / CH;       // rows one wave instruction covers
  static constexpr int INSTS = KT / ROWS_PER_INST;    // instructions per K (or V) tile
  static constexpr int PER_WAVE = INSTS / 4;
};

// Both GEMMs on bf16 MFMA 32x32x16 in the transposed form: S^T = K Q^T
// (32 keys x 32 rows per tile) and O^T += V^T P^T (32 dims x 32 rows).  Lane
// l holds row l % 32 of the wave's 32 (query, head) rows; in S^T it holds keys
// 8 (i / 4) + 4 (l / 32) + i % 4, i < 16, which are exactly the B operand
// P^T of the two 16-key steps of O^T (keys {0-3, 8-11 | 4-7, 12-15} and
// {16-19, 24-27 | 20-23, 28-31}), so the probabilities never leave the lane.
// PIPE: the next item's Q and first tiles are loaded while this item's
// epilogue runs, which needs a staging area of its own (128 KB of LDS in all
// at D = 256).  The kernel of the dense chunks, which run beside the index
// build, stays at 64 KB of LDS and under 384 registers per lane so that the
// build's kernels fit on the same compute units.
template <int D, int G, bool PIPE>
__global__ __launch_bounds__(256, 1) void attn_items_kernel(AttnArgs a) {
  using S = AttnTileShape<D>;
  constexpr int KS = D / 16;        // 16-dim steps of S^T
  constexpr int DT = D / 32;        // 32-dim tiles of O^T
  // vector memory instructions of an item's epilogue: its rows (32 per wave,
  // ROWS_PER_INST per store) and one LSE store
  constexpr int EPI_STORES = 32 / S::ROWS_PER_INST + 1;
  static_assert(EPI_STORES <= 63, "vmcnt range");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_attn[];
  __shared__ int s_items[2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar LDS bases
  const int l32 = lane & 31, g = lane >> 5;
  const float NEG_INF = -INFINITY;
  // blocks are dispatched round-robin over the 8 XCDs: take work from this
  // XCD's queue, then steal from the others
  const int home = blockIdx.x & 7;
  int probe = 0;

  // --- per-lane address bases (fixed for the kernel) ---------------------
  // loads: instruction m of this wave covers rows r0 + 4 m RPI; their row % 4
  // is r0 % 4, their row % 16 alternates with m when 4 RPI == 8
  const int r0 = wave * S::ROWS_PER_INST + lane / S::CH;
  const int cpos = lane % S::CH;
  uint32_t kslot[2], vslot;
  kslot[0] = (uint32_t)((cpos ^ (r0 & 15)) * 16);
  kslot[1] = (uint32_t)((cpos ^ ((r0 + 4 * S::ROWS_PER_INST) & 15)) * 16);
  vslot = (uint32_t)((cpos ^ ((r0 & 3) << 2)) * 16);
  // K operand (A of S^T): row l32, chunk (2 s + g) ^ (l32 % 16); for s < 8 the
  // chunk stays below 16, past it the XOR keeps the +16 (256 bytes)
  int kbase[8];
#pragma unroll
  for (int s8 = 0; s8 < 8; ++s8) kbase[s8] = l32 * S::ROW_BYTES + 16 * ((2 * s8 + g) ^ (l32 & 15));
  // V^T operand (A of O^T, transposing reads): the 16-lane group (g, hh)
  // covers dims dt*32 + hh*16 .. +16 of rows K0..K0+3 with K0 = 16 m + 4 g
  // (+8 for the second read); lane i of the group reads row K0 + i/4, dims
  // 4 (i % 4).., chunk (4 dt + 2 hh + (i % 4)/2) ^ 4 (i / 4)
  const int i16 = lane & 15, hh = (lane >> 4) & 1;
  int vbase[4];
#pragma unroll
  for (int d4 = 0; d4 < 4; ++d4)
    vbase[d4] = (4 * g + (i16 >> 2)) * S::ROW_BYTES + 16 * (4 * (d4 ^ (i16 >> 2)) + 2 * hh + ((i16 & 3) >> 1)) +
                8 * (i16 & 1);

  // LDS: K tiles in buffers 0/1, V tiles in buffers 2/3
  auto kbuf_at = [&](int i) { return smem_attn + i * S::TILE_BYTES; };
  auto vbuf_at = [&](int i) { return smem_attn + (2 + i) * S::TILE_BYTES; };

  // Thread 0 claims work one item ahead: the atomic for the following claim
  // is issued when a claim resolves, so its latency hides behind an item's
  // work.  Items are used one further ahead: when an item starts, the next
  // one is claimed and its record is loaded, and once the item's first tiles
  // are in, wave 0 loads the next item's query slots straight into LDS.  An
  // item then starts with all of its addresses known, and its Q loads and
  // first tile loads share one round trip.
  // the queues' sizes and offsets are read once, into LDS
  __shared__ int s_queue[16];
  if (threadIdx.x < 16) s_queue[threadIdx.x] = a.queue[threadIdx.x];
  int pend = 0;
  if (threadIdx.x == 0) pend = atomicAdd(&a.queue[16 + home], 1);
  __syncthreads();
  // The first 2 B positions of each segment (B = blocks per segment) are
  // paired statically: the block of rank i in its segment takes positions i
  // and 2 B - 1 - i.  Segments start with their longest items, so a pair
  // (long, short) evens out the blocks' first shares, which would otherwise
  // go by the order of the first atomic claims.  The later positions are
  // claimed through the segment's counter.
  const int nstat = (gridDim.x % 8 == 0) ? 2 * (int)(gridDim.x / 8) : 0;
  const int srank = (int)(blockIdx.x >> 3);
  int nclaims = 0;
  // thread 0 only: the next item of this block's queue (stealing from the
  // other XCDs' queues once it is empty), -1 when every queue is
  auto claim = [&]() -> int {
    while (nclaims < 2 && nstat > 0) {
      const int pos = nclaims++ == 0 ? srank : nstat - 1 - srank;
      if (pos < s_queue[home]) return s_queue[8 + home] + pos;
    }
    int claimed = -1;
    for (;;) {
      const int x = (home + probe) & 7;
      if (nstat + pend < s_queue[x]) {
        claimed = s_queue[8 + x] + nstat + pend;
        break;
      }
      if (++probe == 8) break;
      pend = atomicAdd(&a.queue[16 + ((home + probe) & 7)], 1);
    }
    if (claimed >= 0) pend = atomicAdd(&a.queue[16 + ((home + probe) & 7)], 1);
    return claimed;
  };
  // Claims run two items ahead through two LDS slots, so reading one needs no
  // barrier: when an item starts, the next item's index (slot of parity i + 1)
  // was written when the previous item started, and every item's steps end
  // with barriers; thread 0 then writes the index after next into the slot
  // the current item's index came from, which every thread read one item ago.
  int parity = 0;
  auto next_index = [&]() -> int {
    const int v = __builtin_amdgcn_readfirstlane(s_items[parity ^ 1]);   // uniform: scalar loads below
    if (threadIdx.x == 0) s_items[parity] = v >= 0 ? claim() : -1;
    parity ^= 1;
    return v;
  };
  // this lane's Q row R = wave*32 + l32 is (query slot R / G, head R % G)
  const int row_i = (wave * 32 + l32) / G, row_j = (wave * 32 + l32) % G;
  // a cluster item's query slots, qvals[entry0 ..][0 .. qn), into s_qslots
  // (wave 0; slots past qn read as 0 and are not used)
  __shared__ int s_qslots[PREFILL_ROWS];
  auto fetch_slots = [&](const PrefillItem& r) {
    const int c = __builtin_amdgcn_readfirstlane(r.c);
    if (wave != 0 || c < 0) return;
    const int qn = __builtin_amdgcn_readfirstlane(r.qn);
    const uint64_t b = (uint64_t)(a.qvals + __builtin_amdgcn_readfirstlane(r.entry0));
    u32x4_t rsrc;
    rsrc.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
    rsrc.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
    rsrc.z = (uint32_t)qn * 4u;
    rsrc.w = (uint32_t)BUFFER_CONFIG;
    const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)s_qslots);
#pragma unroll
    for (int k = 0; k < PREFILL_ROWS / G; k += 64) lds_dma4(rsrc, dst + 4 * k, (uint32_t)(lane + k) * 4u);
  };
  // direct loads of the K (or V) rows of tile t into an LDS buffer; rows
  // past the item's last key are outside the buffer range and read as 0
  auto issue = [&](const bf16_t* base, uint32_t rs_bytes, int nkeys, int t, unsigned char* dst_tile, bool is_k) {
    const int t0 = t * KT;
    const int valid = __builtin_amdgcn_readfirstlane((int)((uint32_t)(nkeys - t0) * rs_bytes));
    const uint64_t b = (uint64_t)((const unsigned char*)base + (uint64_t)t0 * rs_bytes);
    u32x4_t rsrc;     // raw buffer resource: base, stride 0, valid bytes, config
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

  // The item being started: its fields (uniform), this lane's query (-1 past
  // the item's queries; a cluster item's slots were loaded into LDS during the
  // previous item), its Q rows in registers and its first tiles in flight.
  // An item is started as soon as the previous one no longer needs its Q
  // registers and tile buffers, so these loads run under that item's
  // epilogue.  Q^T (B of S^T): lane holds row R -> (slot row_i, head row_j),
  // dims 16 s + 8 g .. +8.  Rows past the item's queries take query slot 0's
  // values: they are computed like any row and never stored.
  int b_h = 0, b_c = 0, b_qb = 0, b_qn = 0, b_nkeys = 0, b_qidx = -1;
  int64_t b_entry0 = 0;
  const bf16_t* b_kp = nullptr;
  const bf16_t* b_vp = nullptr;
  uint32_t b_rsb = 0;
  u32x4_t qr[KS];
  bool q_staged = false;      // PIPE: the next item's Q rows are in the staging area
  auto begin = [&](const PrefillItem& r) {
    b_h = __builtin_amdgcn_readfirstlane(r.h);
    b_c = __builtin_amdgcn_readfirstlane(r.c);
    b_qb = __builtin_amdgcn_readfirstlane(r.qb);
    b_qn = __builtin_amdgcn_readfirstlane(r.qn);
    b_entry0 = __builtin_amdgcn_readfirstlane(r.entry0);
    const bool local = b_c < 0;
    const int64_t row0 = __builtin_amdgcn_readfirstlane(r.row0);
    int nkeys = local ? (int)(a.chunk_start + b_qb + b_qn - a.wstart) : __builtin_amdgcn_readfirstlane(r.nkeys);
    // an item without keys runs one fully masked tile: its output is 0 and its
    // LSE -inf, and its step publishes the next item's slots like any other
    b_nkeys = max(__builtin_amdgcn_readfirstlane(nkeys), 0);
    const bf16_t* kp;
    const bf16_t* vp;
    int64_t rs;
    if (local) {
      kp = a.korig + (int64_t)b_h * a.o_sh;   // row 0 is position wstart
      vp = a.vorig + (int64_t)b_h * a.o_sh;
      rs = a.o_st;
    } else {
      kp = a.packed + row0 * a.Hkv * D + (int64_t)b_h * D;
      vp = kp + a.packed_len * a.Hkv * D;
      rs = (int64_t)a.Hkv * D;
    }
    // uniform values (scalar registers): the buffer resources built from them
    // need no per-lane loop
    b_kp = uniform_ptr(kp);
    b_vp = uniform_ptr(vp);
    b_rsb = (uint32_t)__builtin_amdgcn_readfirstlane((int)(rs * 2));
    b_qidx = row_i >= b_qn ? -1 : (local ? b_qb + row_i : s_qslots[row_i]);
    if (PIPE && q_staged) {
      // the wave's rows were loaded into its staging slice during the
      // previous item (K-tile layout): wait for its own loads, then read
      __builtin_amdgcn_s_waitcnt(0);
      const unsigned char* sq = smem_attn + S::stage_offset(true) + wave * 32 * S::ROW_BYTES;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        qr[s] = *reinterpret_cast<const u32x4_t*>(sq + kbase[s & 7] + 256 * (s >> 3));
    } else {
      const bf16_t* src = a.q + (int64_t)max(b_qidx, 0) * a.q_sq + (int64_t)(b_h * G + row_j) * a.q_sh + g * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) qr[s] = *reinterpret_cast<const u32x4_t*>(src + s * 16);
    }
    q_staged = false;
    issue(b_kp, b_rsb, b_nkeys, 0, kbuf_at(0), true);
    issue(b_vp, b_rsb, b_nkeys, 0, vbuf_at(0), false);
    if (b_nkeys > KT) issue(b_kp, b_rsb, b_nkeys, 1, kbuf_at(1), true);
  };

  PrefillItem rec{};
  if (threadIdx.x == 0) {
    s_items[0] = claim();
    s_items[1] = s_items[0] >= 0 ? claim() : -1;
  }
  __syncthreads();
  int idx = __builtin_amdgcn_readfirstlane(s_items[0]);
  if (idx >= 0) {
    rec = a.items[idx];
    fetch_slots(rec);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    begin(rec);
  }
  int idx_n = -1;
  bool begun_under_epilogue = false;   // PIPE: this item's first loads precede the last item's stores
  int idx_after = -1;                  // PIPE: the item after the next one, claimed before those stores
#ifdef SBSA_ATTN_PROBE
  int probe_k = 0;
#endif
  PROBE(-2, 0, 0, 0);
  for (; idx >= 0; idx = idx_n) {
    // this item, as begin() left it
    const int h = __builtin_amdgcn_readfirstlane(b_h), c = __builtin_amdgcn_readfirstlane(b_c);
    const int qb = __builtin_amdgcn_readfirstlane(b_qb), qn = __builtin_amdgcn_readfirstlane(b_qn);
    const int64_t entry0 = b_entry0;
    const int nkeys = __builtin_amdgcn_readfirstlane(b_nkeys);
    const bf16_t* const kp = b_kp;
    const bf16_t* const vp = b_vp;
    const uint32_t rs_bytes = b_rsb;
    const int qidx_r = b_qidx;
    const bool local = c < 0;
    const int ntiles = max(1, (nkeys + KT - 1) / KT);
    PROBE(idx, ntiles, qn, c);
    if (!begun_under_epilogue) {
      idx_n = next_index();
      if (idx_n >= 0) rec = a.items[idx_n];
    } else {
      idx_n = idx_after;      // claimed, and its record loaded, before the last epilogue's stores
    }
    // once, after this item's first tiles are in (every wave has read its
    // slot by then); the next item's first step publishes it
    bool prefetched = false;
    auto prefetch_queries = [&]() {
      if (idx_n >= 0 && !prefetched) fetch_slots(rec);
      prefetched = true;
    };
    const int qlim = local ? (int)(a.chunk_start + qidx_r - a.wstart) : 0x7fffffff;
    // the last key any row of this wave may see, and the last key every row
    // sees (no limit inside a cluster item)
    int wave_lim = 0x7fffffff, wave_min = 0x7fffffff;
    if (local) {
      wave_lim = qlim;
      wave_min = qidx_r >= 0 ? qlim : 0x7fffffff;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        wave_lim = max(wave_lim, __shfl_xor(wave_lim, o, 64));
        wave_min = min(wave_min, __shfl_xor(wave_min, o, 64));
      }
      wave_lim = __builtin_amdgcn_readfirstlane(wave_lim);
      wave_min = __builtin_amdgcn_readfirstlane(wave_min);
    }

    // S^T = K Q^T for one tile; K fragments are read KA_AHEAD ahead
    constexpr int KA_AHEAD = 3;
    auto kread = [&](const unsigned char* sK, int s) -> u32x4_t {
      return *reinterpret_cast<const u32x4_t*>(sK + kbase[s & 7] + 256 * (s >> 3));
    };
    auto gemm_s_body = [&](f32x16_t& sacc, const unsigned char* sK) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[e] = 0.f;
      u32x4_t ka[KA_AHEAD];
#pragma unroll
      for (int f = 0; f < KA_AHEAD; ++f) ka[f] = kread(sK, f);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4_t cur = ka[s % KA_AHEAD];
        if (s + KA_AHEAD < KS) ka[s % KA_AHEAD] = kread(sK, s + KA_AHEAD);
        sacc = mfma32x32x16(as_bf16x8(cur), as_bf16x8(qr[s]), sacc);
      }
    };
    auto gemm_s = [&](f32x16_t& sacc, const unsigned char* sK) {
      gemm_s_body(sacc, sK);
      __builtin_amdgcn_sched_group_barrier(0x100, KA_AHEAD, 0);
#pragma unroll
      for (int f = 0; f < KS - KA_AHEAD; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, KA_AHEAD, 0);
    };

    // masking of tile t (only tiles that cross the item's end or a row's
    // causal limit) and this lane's running maximum of the raw scores
    float lmax_all = NEG_INF;
    auto mask_track = [&](f32x16_t& sacc, int t) {
      const int t0 = t * KT;
      if (t0 + KT > nkeys || t0 + KT - 1 > wave_min) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = t0 + 8 * (e >> 2) + 4 * g + (e & 3);
          if (!(key < nkeys && key <= qlim)) sacc[e] = NEG_INF;
        }
      }
#pragma unroll
      for (int e = 0; e < 16; e += 4)
        lmax_all = fmaxf(lmax_all, fmaxf(fmaxf(sacc[e], sacc[e + 1]), fmaxf(sacc[e + 2], sacc[e + 3])));
    };

    // the masking alone, for the passes that do not track the maximum
    auto mask_only = [&](f32x16_t& sacc, int t) {
      const int t0 = t * KT;
      if (t0 + KT > nkeys || t0 + KT - 1 > wave_min) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = t0 + 8 * (e >> 2) + 4 * g + (e & 3);
          if (!(key < nkeys && key <= qlim)) sacc[e] = NEG_INF;
        }
      }
    };

    // probabilities exp2(s - m) of a tile against the row's reference maximum
    // as the B operands of the two 16-key steps of O^T
    float m_ref = 0.f, l_part = 0.f;
    auto exp_pack = [&](f32x16_t& sacc, u32x4_t (&pb)[2]) {
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[e], a.scale_log2, -m_ref));
        sacc[e] = p;
        sum += p;
      }
      l_part += sum;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        pb[m].x = pack2bf(sacc[8 * m + 0], sacc[8 * m + 1]);
        pb[m].y = pack2bf(sacc[8 * m + 2], sacc[8 * m + 3]);
        pb[m].z = pack2bf(sacc[8 * m + 4], sacc[8 * m + 5]);
        pb[m].w = pack2bf(sacc[8 * m + 6], sacc[8 * m + 7]);
      }
    };

    // O^T += V^T P^T: two transposing reads per 32-dim x 16-key fragment,
    // VA_AHEAD fragments ahead of the MFMAs
    f32x16_t o[DT];
    auto gemm_pv = [&](const u32x4_t (&pb)[2], const unsigned char* sV) {
      constexpr int NF = DT * 2;          // fragments (m, dt), m-major
      constexpr int VA_AHEAD = 4;
      u32x4_t va[VA_AHEAD];
      auto vread = [&](int f) -> u32x4_t {
        const int m = f / DT, dt = f % DT;
        const unsigned char* p = sV + vbase[dt & 3] + 256 * (dt >> 2) + 16 * m * S::ROW_BYTES;
        s16x4_t part[2];
        part[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
        part[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + 8 * S::ROW_BYTES));
        u32x4_t r;
        __builtin_memcpy(&r, part, 16);
        return r;
      };
#pragma unroll
      for (int f = 0; f < VA_AHEAD; ++f) va[f] = vread(f);
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const u32x4_t cur = va[f % VA_AHEAD];
        if (f + VA_AHEAD < NF) va[f % VA_AHEAD] = vread(f + VA_AHEAD);
        const int m = f / DT, dt = f % DT;
        o[dt] = mfma32x32x16(as_bf16x8(cur), as_bf16x8(pb[m]), o[dt]);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * VA_AHEAD, 0);
#pragma unroll
      for (int f = 0; f < NF - VA_AHEAD; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, VA_AHEAD, 0);
    };

    // One step: S(t+1) on the MFMA units while the VALU turns S(t) into
    // probabilities, then O += V(t) P(t).  K(t+2) and V(t+1) stream into the
    // buffers that K(t) and V(t-1) left.  Two forms: the steady one, for
    // tiles whose successor some row of the wave still sees, is straight-line
    // code the scheduler can interleave; the general one handles the wave's
    // last active tile and the tiles past every row of the wave, whose loads
    // the wave still issues for the others.
    // PIPE: the next item's Q rows into this wave's staging slice, in the
    // K-tile layout (row r, 16-byte chunk c at slot (c % 16 ^ r % 16) + 16 (c / 16));
    // issued in step 1, once the next item's query slots are published, after
    // that step's tile loads, so the step's wait can leave them in flight
    constexpr int QN = 32 / S::ROWS_PER_INST;      // loads per wave
    auto stage_q = [&]() {
      const int nh = __builtin_amdgcn_readfirstlane(rec.h), nc = __builtin_amdgcn_readfirstlane(rec.c);
      const int nqb = __builtin_amdgcn_readfirstlane(rec.qb), nqn = __builtin_amdgcn_readfirstlane(rec.qn);
      const uint64_t b = (uint64_t)a.q;
      u32x4_t rsrc;
      rsrc.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
      rsrc.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
      rsrc.z = (uint32_t)a.q_bytes;
      rsrc.w = (uint32_t)BUFFER_CONFIG;
      const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)(
          smem_attn + S::stage_offset(true) + wave * 32 * S::ROW_BYTES));
      const int p = lane % S::CH;
#pragma unroll
      for (int m = 0; m < QN; ++m) {
        const int r = m * S::ROWS_PER_INST + lane / S::CH;
        const int R = wave * 32 + r, i = R / G, j = R % G;
        const int qi = i < nqn ? (nc < 0 ? nqb + i : s_qslots[i]) : -1;
        const int cg = ((p & 15) ^ (r & 15)) + 16 * (p >> 4);
        const uint32_t off = qi < 0 ? 0x80000000u
                                    : (uint32_t)(((int64_t)qi * a.q_sq + (int64_t)(nh * G + j) * a.q_sh) * 2 + 16 * cg);
        lds_dma16(rsrc, dst + m * S::ROWS_PER_INST * S::ROW_BYTES, off);
      }
    };
    // returns whether this step staged the next item's Q
    auto issue_next = [&](int t) -> bool {
      if (t + 2 < ntiles) issue(kp, rs_bytes, nkeys, t + 2, kbuf_at(t & 1), true);
      if (t + 1 < ntiles) issue(vp, rs_bytes, nkeys, t + 1, vbuf_at((t + 1) & 1), false);
      if (PIPE && t == 1 && idx_n >= 0 && !q_staged) {
        stage_q();
        q_staged = true;
        return true;
      }
      return false;
    };
    auto finish_step = [&](bool staged) {
      if (staged) {
        // every load but this step's QN staging loads (vmcnt QN, lgkmcnt 0)
        __builtin_amdgcn_s_waitcnt((QN & 15) | ((QN >> 4) << 14) | (7 << 4));
      } else {
        __builtin_amdgcn_s_waitcnt(0);
      }
      __syncthreads();
    };
    auto step_full = [&](int t, f32x16_t& cur, f32x16_t& nxt) {
      const bool staged = issue_next(t);
      mask_only(cur, t);
      u32x4_t pb[2];
      gemm_s_body(nxt, kbuf_at((t + 1) & 1));
      exp_pack(cur, pb);
      // the VALU work of exp_pack between the MFMAs of S(t+1)
      __builtin_amdgcn_sched_group_barrier(0x100, KA_AHEAD, 0);
#pragma unroll
      for (int f = 0; f < KS - KA_AHEAD; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
#pragma unroll
      for (int f = 0; f < KA_AHEAD; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
      gemm_pv(pb, vbuf_at(t & 1));
      finish_step(staged);
    };
    // the general form, for the tiles around a wave's last active one; with
    // sweep set it only tracks the rows' maxima (no probabilities, no O)
    auto step = [&](int t, f32x16_t& cur, f32x16_t& nxt, bool sweep) {
      const bool staged = issue_next(t);
      const bool act = t * KT <= wave_lim;
      const bool act_n = t + 1 < ntiles && (t + 1) * KT <= wave_lim;
      u32x4_t pb[2];
      if (act) {
        if (sweep) mask_track(cur, t);
        else mask_only(cur, t);
      }
      if (act_n) gemm_s(nxt, kbuf_at((t + 1) & 1));
      if (act && !sweep) {
        exp_pack(cur, pb);
        gemm_pv(pb, vbuf_at(t & 1));
      }
      finish_step(staged);
    };

    // Each row's probabilities are taken against a reference maximum fixed
    // from the first tile; no accumulator is rescaled in the loop.  If a row's
    // sum of probabilities passes 2^OVERFLOW_LOG2 (which any probability past
    // that bound would cause; a probability up to it is safe in fp32 and
    // bf16), the item is redone: a sweep over the tiles finds the rows' true
    // maxima, and the last pass takes them as reference.
    for (int pass = 0; pass < 3; ++pass) {
      const bool sweep = pass == 1;
      if (pass > 0) {           // pass 0's first tiles were issued by begin()
        issue(kp, rs_bytes, nkeys, 0, kbuf_at(0), true);
        issue(vp, rs_bytes, nkeys, 0, vbuf_at(0), false);
        if (ntiles > 1) issue(kp, rs_bytes, nkeys, 1, kbuf_at(1), true);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
      l_part = 0.f;
      lmax_all = NEG_INF;
      if (PIPE && pass == 0 && begun_under_epilogue) {
        // the first tiles were issued before the previous item's EPI_STORES
        // stores: wait for every load but leave those stores in flight
        __builtin_amdgcn_s_waitcnt((EPI_STORES & 15) | ((EPI_STORES >> 4) << 14) | (7 << 4));
      } else {
        __builtin_amdgcn_s_waitcnt(0);
      }
      __syncthreads();
      prefetch_queries();
      f32x16_t sA, sB;
      gemm_s(sA, kbuf_at(0));
      mask_track(sA, 0);
      if (pass == 0) {
        // reference maximum: the row's maximum over the first tile (key 0 of
        // an item is visible to every row, so it is finite)
        const float mx = halves_max(lmax_all);
        m_ref = (mx == NEG_INF) ? 0.f : mx * a.scale_log2;
      }
      int t = 0;
      if (!sweep) {
        // tiles 0..t_last hold keys some row of this wave may see; the steady
        // loop runs while the next tile is active too
        const int t_last = min(ntiles - 1, wave_lim / KT);
        for (; t + 2 <= t_last; t += 2) {
          step_full(t, sA, sB);
          step_full(t + 1, sB, sA);
        }
      }
      for (; t < ntiles; t += 2) {
        step(t, sA, sB, sweep);
        if (t + 1 < ntiles) step(t + 1, sB, sA, sweep);
      }
      if (pass == 0) {
        const float l = halves_sum(l_part);
        const bool over = !(l <= __builtin_exp2f(OVERFLOW_LOG2));
        if (!__syncthreads_or(over ? 1 : 0)) break;
      } else if (sweep) {
        const float mx = halves_max(lmax_all);
        m_ref = (mx == NEG_INF) ? 0.f : mx * a.scale_log2;
      }
    }

    // PIPE: the next item's Q and first tiles load under this item's epilogue,
    // and the item after it is claimed and its record loaded before the
    // epilogue's stores, so that no wait of the next item waits for them
    begun_under_epilogue = PIPE && idx_n >= 0;
    if (PIPE && idx_n >= 0) {
      begin(rec);
      idx_after = next_index();
      if (idx_after >= 0) rec = a.items[idx_after];
    }

    // epilogue: normalise, then write the partial (or the local window) and
    // its LSE.  The rows go through this wave's own 32-row slice of a staging
    // area (PIPE: its own; otherwise the idle tile buffers), so that every
    // store is 16 bytes per lane and whole rows per instruction: the item's
    // rows are contiguous in part_o, and the G heads of a query are
    // contiguous in the window output.
    {
      const float l = halves_sum(l_part);
      const float inv = (l > 0.f) ? 1.0f / l : 0.f;
      // PIPE: every store of the epilogue is issued by every lane (EPI_STORES
      // per wave), through buffer resources over the item's rows: a lane
      // without a row stores at an offset past the range, where the store is
      // dropped.  The next item's first wait counts on that number.  The
      // compact form keeps plain stores under the rows' conditions: the
      // resources would take it past 384 registers per lane, and the index
      // build's kernels would no longer fit beside its blocks.
      if (!PIPE) {
        if (qidx_r >= 0 && g == 0) {
          const float lse = (l > 0.f) ? (m_ref + log2f(l)) * 0.69314718055994531f : NEG_INF;
          float* ldst = local ? (a.local_lse ? a.local_lse + (int64_t)qidx_r * a.Hq + h * G + row_j : nullptr)
                              : a.part_lse + (entry0 + row_i) * G + row_j;
          if (ldst) *ldst = lse;
        }
      } else {
        const float lse = (l > 0.f) ? (m_ref + log2f(l)) * 0.69314718055994531f : NEG_INF;
        const float* lbase;
        int64_t lbytes, loff;
        if (local) {
          lbase = a.local_lse ? a.local_lse : reinterpret_cast<const float*>(a.q);
          lbytes = a.local_lse ? (int64_t)a.Qc * a.Hq * 4 : 0;
          loff = ((int64_t)qidx_r * a.Hq + h * G + row_j) * 4;
        } else {
          lbase = a.part_lse + entry0 * G;
          lbytes = (int64_t)qn * G * 4;
          loff = (int64_t)(row_i * G + row_j) * 4;
        }
        const __amdgpu_buffer_rsrc_t lrsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform_ptr(reinterpret_cast<const bf16_t*>(lbase)), 0, (int)lbytes, BUFFER_CONFIG);
        const int off = (qidx_r >= 0 && g == 0) ? (int)loff : OUT_OF_RANGE;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lse), lrsrc, off, 0, 0);
      }
      // 16-byte chunk c of row r sits at chunk c ^ (r % 32) of the row.  Lane
      // (l32, g) holds dims 32 dt + 8 q4 + 4 g .. +3; a swap between the lane
      // halves (lanes l and l + 32) gives lane g = 0 all 8 dims of chunk
      // 4 dt + 2 p and lane g = 1 those of chunk 4 dt + 2 p + 1 (q4 = 2 p, 2 p + 1),
      // so each lane writes whole 16-byte chunks
      unsigned char* stage = smem_attn + S::stage_offset(PIPE) + wave * 32 * S::ROW_BYTES;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int qa = 2 * p, qb2 = 2 * p + 1;
          const uint32_t a0 = pack2bf(o[dt][4 * qa + 0] * inv, o[dt][4 * qa + 1] * inv);
          const uint32_t a1 = pack2bf(o[dt][4 * qa + 2] * inv, o[dt][4 * qa + 3] * inv);
          const uint32_t b0 = pack2bf(o[dt][4 * qb2 + 0] * inv, o[dt][4 * qb2 + 1] * inv);
          const uint32_t b1 = pack2bf(o[dt][4 * qb2 + 2] * inv, o[dt][4 * qb2 + 3] * inv);
          // lanes < 32 keep their q4 = 2p pair and take the upper lanes' one;
          // lanes >= 32 take the lower lanes' q4 = 2p + 1 pair and keep theirs
          const auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
          u32x4_t w;
          w.x = s0[0];
          w.y = s1[0];
          w.z = s0[1];
          w.w = s1[1];
          const int c = (4 * dt + 2 * p + g) ^ (l32 & (S::CH - 1));
          *reinterpret_cast<u32x4_t*>(stage + l32 * S::ROW_BYTES + 16 * c) = w;
        }
      // the wave's lanes hand their rows to each other through the staging
      // slice (in order on the GPU, where a wave's LDS operations run in issue
      // order; the barrier keeps the compiler from moving them)
      __builtin_amdgcn_wave_barrier();
      // read back whole rows (instruction m covers rows ROWS_PER_INST m ..),
      // reads first, then the stores, so no store waits on a single read
      constexpr int NR = 32 / S::ROWS_PER_INST;
      const int c16 = lane % S::CH;
      const bf16_t* obase = local ? a.local_o + (int64_t)qb * a.lo_sq + (int64_t)(h * G) * a.lo_sh
                                  : a.part_o + entry0 * G * D;
      const int64_t obytes = local ? ((int64_t)(qn - 1) * a.lo_sq + (int64_t)(G - 1) * a.lo_sh + D) * 2
                                   : (int64_t)qn * G * D * 2;
      __amdgpu_buffer_rsrc_t orsrc;
      if (PIPE) orsrc = __builtin_amdgcn_make_buffer_rsrc((void*)uniform_ptr(obase), 0, (int)obytes, BUFFER_CONFIG);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u32x4_t rows[NR / 2];
#pragma unroll
        for (int mm = 0; mm < NR / 2; ++mm) {
          const int m = half * (NR / 2) + mm;
          const int r = m * S::ROWS_PER_INST + lane / S::CH;
          rows[mm] = *reinterpret_cast<const u32x4_t*>(stage + r * S::ROW_BYTES + 16 * (c16 ^ (r & (S::CH - 1))));
        }
#pragma unroll
        for (int mm = 0; mm < NR / 2; ++mm) {
          const int m = half * (NR / 2) + mm;
          const int RR = wave * 32 + m * S::ROWS_PER_INST + lane / S::CH;
          const int i = RR / G, j = RR % G;
          // read once, later, by the combine: non-temporal, kept out of the way
          // of the K/V in L2
          if (PIPE) {
            const int64_t roff = local ? ((int64_t)i * a.lo_sq + (int64_t)j * a.lo_sh) * 2
                                       : (int64_t)(i * G + j) * D * 2;
            __builtin_amdgcn_raw_buffer_store_b128(rows[mm], orsrc, i < qn ? (int)roff + 16 * c16 : OUT_OF_RANGE,
                                                   0, 2);
          } else {
            bf16_t* dst = local ? a.local_o + (int64_t)(qb + i) * a.lo_sq + (int64_t)(h * G + j) * a.lo_sh
                                : a.part_o + ((entry0 + i) * G + j) * D;
            if (i < qn) __builtin_nontemporal_store(rows[mm], reinterpret_cast<u32x4_t*>(dst + 8 * c16));
          }
        }
      }
    }
    if (!PIPE && idx_n >= 0) {
      __syncthreads();          // every wave is done with its staging rows
      begin(rec);
    }
  }
  PROBE(-3, 0, 0, 0);
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
    float* __restrict__ out_lse, int Qc, int Hkv, int C, const int32_t* __restrict__ skip) {
  constexpr int E = G * D / 64;
  if (skip && *skip) return;   // the chunk's partials passed their buffer: it runs again
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

template <int D, int G, bool PIPE>
int launch_attn_kernel(const AttnArgs& a, int grid, hipStream_t stream) {
  const size_t lds = AttnTileShape<D>::lds_bytes(PIPE);
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)attn_items_kernel<D, G, PIPE>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return SBSA_ERR_UNSUPPORTED;
    configured = true;
  }
  static int auto_grid = 0;
  if (grid <= 0) {
    if (!auto_grid) {
      int dev = 0, cus = 0, occ = 0;
      (void)hipGetDevice(&dev);
      (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)attn_items_kernel<D, G, PIPE>,
                                                         256, lds);
      auto_grid = (cus > 0 ? cus : 256) * (occ > 0 ? occ : 1);
    }
    grid = auto_grid;
  }
  hipLaunchKernelGGL((attn_items_kernel<D, G, PIPE>), dim3(grid), dim3(256), lds, stream, a);
  return SBSA_OK;
}

// the pipelined kernel for chunks with cluster items (sparse chunks, which
// run after the index build), the compact one for dense chunks; the
// pipelined kernel's staged Q loads address q with 31-bit offsets
template <int D, int G>
int launch_attn(const AttnArgs& a, int grid, hipStream_t stream) {
  return a.packed && a.q_bytes < 0x7fffffff ? launch_attn_kernel<D, G, true>(a, grid, stream)
                                            : launch_attn_kernel<D, G, false>(a, grid, stream);
}

template <int D, int G>
int launch_combine(const int32_t* qmask, const int32_t* nvis, const int32_t* rev_indptr,
                   const int32_t* qrank, const bf16_t* part_o, const float* part_lse,
                   const bf16_t* local_o, int64_t lo_sq, int64_t lo_sh, const float* local_lse,
                   bf16_t* out, int64_t out_sq, int64_t out_sh, float* out_lse, int Qc, int Hkv,
                   int C, const int32_t* skip, hipStream_t stream) {
  int64_t waves = (int64_t)Qc * Hkv;
  hipLaunchKernelGGL((combine_kernel<D, G>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     stream, qmask, nvis, rev_indptr, qrank, part_o, part_lse, local_o, lo_sq,
                     lo_sh, local_lse, out, out_sq, out_sh, out_lse, Qc, Hkv, C, skip);
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
                     float* out_lse, int Qc, int Hkv, int C, const int32_t* skip,
                     hipStream_t stream) {
  SBSA_DISPATCH_DG(D, G, launch_combine, qmask, nvis, rev_indptr, qrank, part_o, part_lse, local_o,
                   lo_sq, lo_sh, local_lse, out, out_sq, out_sh, out_lse, Qc, Hkv, C, skip, stream);
}

}  // namespace

extern "C" {

#ifdef SBSA_ATTN_PROBE
int sbsa_probe_read(void* host, size_t bytes) {
  if (bytes > sizeof(g_attn_probe)) bytes = sizeof(g_attn_probe);
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_attn_probe), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 3;
}
#endif

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
  if (q_sq % 8 || q_sh % 8 || o_st % 8 || o_sh % 8 || lo_sq % 4 || lo_sh % 4) return SBSA_ERR_ARG;
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
#ifdef SBSA_ATTN_PROBE
  static int probe_next = 0;
  a.probe_slot = probe_next++;
#endif
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
                         int num_clusters, const int32_t* skip, hipStream_t stream) {
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
                            num_kv_heads, num_clusters, skip, stream);
  if (rc) return rc;
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

}  // extern "C"
