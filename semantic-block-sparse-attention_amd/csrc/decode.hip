// S7-S9: the graph-capturable sparse decode step for gfx950.
//
// Reference behaviour (pfnet-research/semantic-block-sparse-attention):
//   fused_decode.py:39-60     _suffix_write_kernel (the token's K/V into the store)
//   trivial_router.py:24-45   routing vector of the query
//   fused_decode.py:81-199    _decode_select_kernel (scores, bisection, CSR)
//   fused_decode.py:202-331   _decode_attend_kernel (prompt splits via the CSR,
//                             suffix splits via the block table)
//   fused_decode.py:334-358   _decode_merge_kernel
//
// Two launches, no host reads, no allocation: every size the kernels need
// (the position, the selected token count) is read on the device, so a HIP
// graph can capture the step and replay it at fixed addresses.
//   1. step: one block per (KV head, split).  Every block first selects for
//      its head (routing, scores on MFMA, per-component LSE, bisection under
//      the budget, the CSR of the selection into LDS); split 0 also writes
//      the CSR to the workspace and the token's K/V into the suffix store.
//      A head's keys are one list, the selected prompt rows in CSR order
//      followed by the live suffix rows (the current token's row read from
//      k_new/v_new); each split takes an even, 32-aligned range of it, in
//      rounds of RC rows.  Per round the block resolves the rows' addresses
//      into LDS; each wave loads the K rows of its 16-key groups straight into
//      registers and runs S^T = K Q^T on MFMA with the G query heads as
//      columns, while every wave copies a share of the V rows into LDS
//      (global loads to LDS).  P goes through LDS, and each wave accumulates
//      O^T = V^T P^T for its own D/4 dimensions over all the round's keys, so
//      the split's partial is written with no fold across waves.
//   2. merge: one block per (query head, 64 dimensions) folds the splits.
#include "sbsa_common.h"

#include <mutex>

namespace {

struct DecodeArgs {
  const bf16_t* q_post;     // [Hq, D] rows at q_sh
  int64_t q_sh;
  const bf16_t* q_pre;      // [Hq, D] router input rows at qp_sh
  int64_t qp_sh;
  int router_pass;          // 1: q_pre is pre-RoPE queries, 0: already routing vectors
  const bf16_t* k_new;      // [Hkv, D] rows at kn_sh, or null (no suffix write)
  const bf16_t* v_new;
  int64_t kn_sh;
  const int32_t* pos;       // [1] the query token's position
  const bf16_t* codebooks;  // [Hkv, 2, C, D/2]
  const int32_t* sizes;     // [Hkv, C] full bucket sizes
  const int32_t* indptr;    // [Hkv, C+1]
  const bf16_t* packed;     // [2, Lp, Hkv, D]
  int64_t packed_len;
  bf16_t* suffix_kv;        // [2, NBLK, BS, Hkv, D]
  int64_t suffix_nblk;
  int BS;
  const int32_t* table;     // logical block -> physical block
  int64_t prompt_len;
  const int32_t* plen_dev;  // [1] the prompt length on the device (overrides prompt_len), or null
  const bf16_t* kpre_new;   // [Hkv, D] pre-RoPE key rows at kn_sh, or null
  bf16_t* suffix_kpre;      // [NBLK, BS, Hkv, D], or null (no pre-RoPE suffix store)
  int32_t* rstart;          // [Hkv, C]
  int32_t* rlen;
  int32_t* rcum;
  int32_t* rcount;          // [Hkv]
  int32_t* rtokens;
  float* pacc;              // [Hq, S, D]
  float* pm;                // [Hq, S]
  float* pl;
  bf16_t* out;              // [Hq, D] rows at out_sh
  int64_t out_sh;
  float* out_lse;           // [Hq] natural-log LSE, or null
  int Hq, Hkv, C, G;
  int nsplit, ssplit, max_tiles, iters, sink;
  float inv_temp, beta, target, scale_log2;
};

#ifdef SBSA_DEC_PROBE
// timing probe (a build flag, not in the product): wall clock per block and
// phase of the last step, and per merge block its start and end
__device__ uint64_t g_dec_probe[1024][16];
__device__ uint64_t g_merge_probe[1024][2];
#define DPROBE(k) do { if (threadIdx.x == 0) g_dec_probe[blockIdx.x * gridDim.y + blockIdx.y][(k)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#define DPROBEW(k) do { if ((threadIdx.x & 63) == 0) g_dec_probe[blockIdx.x * gridDim.y + blockIdx.y][(k) + (threadIdx.x >> 6)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define DPROBE(k) ((void)0)
#define DPROBEW(k) ((void)0)
#endif

constexpr int MAX_C = 1024;
constexpr int MAX_SPLITS = 512;   // prompt + suffix splits of one step
constexpr int DT = 32;            // keys per wave tile
constexpr int MAX_TABLE = 256;    // suffix block-table entries staged in LDS

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const u32x4_t global_u32x4_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// LDS layout of the step's attention: RC rows of V in tiles of 32 rows, each
// row D bf16 with its 16-byte chunks permuted (chunk ^ 2 (row % 4)) so that the
// transposing reads spread over the banks, then P^T [16][RC + 8] bf16.  K
// rows go to registers: wave w holds NG groups of 16 keys.
template <int D>
struct DecodeStep {
  static constexpr int ROW_BYTES = 2 * D;
  static constexpr int CH = D / 8;               // 16-byte chunks per row
  static constexpr int RPI = 64 / CH;            // rows per wave load instruction
  static constexpr int INSTS = DT / RPI;         // load instructions per V tile
  static constexpr int TILE_BYTES = DT * ROW_BYTES;
  static constexpr int RC = D >= 256 ? 192 : 384;  // rows per round
  static constexpr int NG = RC / 64;             // 16-key groups per wave
  static constexpr int DBW = D / 64;             // 16-dim blocks of O per wave
  static constexpr size_t V_BYTES = (size_t)RC * ROW_BYTES;
  static constexpr size_t LDS_BYTES = V_BYTES + (size_t)16 * (RC + 8) * 2;
};

// Dynamic LDS of the step kernel: the attention's V tiles and P^T, or the
// selection's routing vectors [16][D+8] bf16 and component weights [G][C] f32.
template <int D>
size_t step_lds_bytes(int G, int C) {
  size_t sel = (size_t)16 * (D + 8) * 2 + (size_t)G * C * 4;
  return sel > DecodeStep<D>::LDS_BYTES ? sel : DecodeStep<D>::LDS_BYTES;
}

// ------------------------------------------------------------- selection ---
// All 256 threads.  NK = clusters per lane of wave 0 (C <= 64 NK).  Leaves
// the CSR of the head's selection in s_rstart / s_rcum (rcount entries) and
// s_cnt = {rcount, rtokens}.  `prefetch` issues the caller's loads behind the
// selection's first ones; `after_routing` runs in every wave once the routing
// rows are in LDS (pos_v and plen are read only after it); `idle_loads` runs
// in waves 1-3 while wave 0 bisects, and its copies into LDS have landed when
// the selection returns.  Every load before the routing is issued in
// straight-line code, so the routing waits for its own row only.
template <int D, int G, int NK, typename Prefetch, typename AfterRouting, typename IdleLoads>
__device__ __forceinline__ void select_phase(const DecodeArgs& a, int h, bool leader, const int& pos_v,
                                             const int64_t& plen, Prefetch prefetch,
                                             AfterRouting after_routing, IdleLoads idle_loads,
                                             unsigned char* smem, int* s_rstart, int* s_rcum, int* s_cnt) {
  constexpr int KS = D / 32;
  constexpr int LDQ = D + 8;
  bf16_t* svec = reinterpret_cast<bf16_t*>(smem);                   // [16][LDQ]
  float* ssc = reinterpret_cast<float*>(smem + 16 * LDQ * 2);        // [G][C]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int C = a.C;
  const int half = D / 2;
  const int nk = C / 64;
  constexpr int PER = D / 64;

  // loads in the order of use: the router input row of this wave's first
  // head (raw bits, converted at the routing), the sizes and run starts, the
  // codebook tiles, then the caller's.  No copy into LDS is in flight before
  // the routing: the compiler waits for every load while one is.
  uint32_t vq[PER];
  DPROBE(12);
  {
    // every wave loads a valid row (waves past G: the last head's, unused)
    const bf16_t* src = a.q_pre + (int64_t)(h * G + min(wave, G - 1)) * a.qp_sh;
#pragma unroll
    for (int i = 0; i < PER; ++i) vq[i] = src[lane + 64 * i];
  }
  // the clusters' sizes and run starts of this lane (read by wave 0 only; a
  // cluster past C reads the last one's)
  int sz[NK], ip[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int c = min(64 * k + lane, C - 1);
    sz[k] = a.sizes[h * C + c];
    ip[k] = a.indptr[h * (C + 1) + c];
  }
  const bf16_t* cb = a.codebooks + (int64_t)h * 2 * C * half;
  auto load_cb = [&](int cbk, u32x4_t* b) {
    const int cc = cbk * 16 + (lane & 15);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      int d = s * 32 + (lane >> 4) * 8;
      int part = d / half;
      b[s] = *reinterpret_cast<const u32x4_t*>(cb + ((int64_t)part * C + cc) * half + (d - part * half));
    }
  };
  // this wave's first PT codebook tiles (all of them up to C = 256), in flight
  // during the routing (loaded unconditionally, a tile past C clamped to the
  // last, so that the routing's wait counts only the loads before its row)
  constexpr int PT = NK < 2 ? 2 : (NK > 4 ? 4 : NK);
  u32x4_t bt[PT][KS];
#pragma unroll
  for (int i = 0; i < PT; ++i) load_cb(min(wave + 4 * i, C / 16 - 1), bt[i]);
  prefetch();
  // 1. routing vectors of the G query heads (rows >= G are zero)
  for (int e = threadIdx.x; e < 16 * (D / 8); e += 256) {
    int r = e / (D / 8), ch = e % (D / 8);
    if (r >= G) *reinterpret_cast<u32x4_t*>(&svec[r * LDQ + ch * 8]) = u32x4_t{0, 0, 0, 0};
  }
  // keeps the first row's conversion here, after the codebook loads were issued
#pragma unroll
  for (int i = 0; i < PER; ++i) asm volatile("" : "+v"(vq[i]));
  for (int t = wave; t < G; t += 4) {
    const bf16_t* src = a.q_pre + (int64_t)(h * G + t) * a.qp_sh;
    float v[PER];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      v[i] = bf2f((t == wave) ? (bf16_t)vq[i] : src[lane + 64 * i]);
      ss += v[i] * v[i];
    }
    if (a.router_pass) {
      float n1 = fmaxf(sqrtf(wave_sum_dpp(ss)), 1e-12f);
      float ss2 = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        v[i] = round_bf16(v[i] / n1);
        ss2 += v[i] * v[i];
      }
      float n2 = fmaxf(sqrtf(wave_sum_dpp(ss2)), 1e-12f);
#pragma unroll
      for (int i = 0; i < PER; ++i) v[i] = v[i] / n2;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) svec[t * LDQ + lane + 64 * i] = f2bf(v[i]);
    DPROBE(13);
  }
  __syncthreads();
  DPROBE(1);
  after_routing();
  // 2. scores s[t][c] = v_t . c / tau on MFMA (16 rows, G real)
  u32x4_t aop[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    aop[s] = *reinterpret_cast<const u32x4_t*>(&svec[(lane & 15) * LDQ + s * 32 + (lane >> 4) * 8]);
  auto score_tile = [&](int cbk, const u32x4_t* b) {
    const int cc = cbk * 16 + (lane & 15);
    f32x4_t acc = f32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma16x16x32(as_bf16x8(aop[s]), as_bf16x8(b[s]), acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int t = (lane >> 4) * 4 + i;
      if (t < G) ssc[t * C + cc] = acc[i] * a.inv_temp;
    }
  };
#pragma unroll
  for (int i = 0; i < PT; ++i)
    if (wave + 4 * i < C / 16) score_tile(wave + 4 * i, bt[i]);
  for (int cbk = wave + 4 * PT; cbk < C / 16; cbk += 4) {
    u32x4_t b[KS];
    load_cb(cbk, b);
    score_tile(cbk, b);
  }
  __syncthreads();
  DPROBE(2);
  if (wave != 0) {
    idle_loads();
    // the token's K/V into the suffix store, once per head (a position past
    // the reservation is not written: the table does not cover it)
    const int64_t q_pos = __builtin_amdgcn_readfirstlane(pos_v);
    if (leader && a.k_new && q_pos >= plen && q_pos - plen < (int64_t)a.max_tiles * 16) {
      const int64_t blk = q_pos / a.BS;
      const int64_t off = q_pos - blk * a.BS;
      const int64_t phys = a.table[blk];
      const int64_t plane = a.suffix_nblk * a.BS * a.Hkv * D;
      const int64_t at = ((phys * a.BS + off) * a.Hkv + h) * D;
      bf16_t* dst = a.suffix_kv + at;
      for (int d = threadIdx.x - 64; d < D; d += 192) {
        dst[d] = a.k_new[(int64_t)h * a.kn_sh + d];
        dst[plane + d] = a.v_new[(int64_t)h * a.kn_sh + d];
      }
      // the pre-RoPE key too, for a later move of the token into the clusters
      if (a.suffix_kpre && a.kpre_new)
        for (int d = threadIdx.x - 64; d < D; d += 192) a.suffix_kpre[at + d] = a.kpre_new[(int64_t)h * a.kn_sh + d];
    }
    __builtin_amdgcn_s_waitcnt(0);       // the caller's copies into LDS (idle_loads) have landed
  } else {
    // 4. bisection and the CSR; sizes are integers below 2^24, so
    //    the reference's fp32 sums are exact and equal these integer sums
#pragma unroll
    for (int k = 0; k < NK; ++k) sz[k] = (k < nk) ? sz[k] : 0;
    // 3. per component LSE over the clusters, then each cluster's weight
    //    p_c = sum_t exp(s_tc - lse_t): the same sums in the same order as a
    //    pass per component, with the G components' reductions interleaved
    constexpr float LOG2E = 1.4426950408889634f;
    float sv[G][NK], mt[G], lt[G];
#pragma unroll
    for (int t = 0; t < G; ++t) {
      mt[t] = -INFINITY;
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        sv[t][k] = (k < nk) ? ssc[t * C + lane + 64 * k] : 0.f;
        if (k < nk) mt[t] = fmaxf(mt[t], sv[t][k]);
      }
    }
#pragma unroll
    for (int t = 0; t < G; ++t) mt[t] = wave_max_dpp(mt[t]);
#pragma unroll
    for (int t = 0; t < G; ++t) {
      lt[t] = 0.f;
#pragma unroll
      for (int k = 0; k < NK; ++k)
        if (k < nk) lt[t] += __builtin_amdgcn_exp2f((sv[t][k] - mt[t]) * LOG2E);
    }
#pragma unroll
    for (int t = 0; t < G; ++t) lt[t] = wave_sum_dpp(lt[t]);
    float pw[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) pw[k] = 0.f;
#pragma unroll
    for (int t = 0; t < G; ++t) {
      const float lse2 = mt[t] * LOG2E + __builtin_amdgcn_logf(lt[t]);    // log2 of the normaliser
#pragma unroll
      for (int k = 0; k < NK; ++k) pw[k] += __builtin_amdgcn_exp2f(__builtin_fmaf(sv[t][k], LOG2E, -lse2));
    }
    const float NEG = -3.4e38f, POS = 3.4e38f;
    float score[NK];
    int size[NK];
    float hi = -INFINITY, lo = INFINITY;
    int live_total = 0;
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      score[k] = NEG;
      size[k] = 0;
      if (k < nk) {
        const int c = lane + 64 * k;
        const float p = pw[k];
        const int s = (a.sink > 0 && c == 0) ? 0 : sz[k];
        size[k] = s;
        const bool live = s > 0;
        float sc = logf(fmaxf(p, 1e-38f));
        if (a.beta != 0.f) sc = sc - a.beta * logf(1.0f + (float)s);
        sc = live ? sc : NEG;
        score[k] = sc;
        hi = fmaxf(hi, sc);
        lo = fminf(lo, live ? sc : POS);
        live_total += live ? s : 0;
      }
    }
    hi = wave_max_dpp(hi) + 1e-6f;
    lo = wave_min_dpp(lo) - 1e-6f;
    lo = fminf(lo, hi - 1e-5f);
    live_total = wave_sum_i32_dpp(live_total);
    const float budget = (a.sink > 0) ? fmaxf(a.target - (float)a.sink, 0.f) : a.target;
    const bool all_fit = (float)live_total < budget;
    const int bud_i = budget_count(budget);
    DPROBE(14);
    // two bisection steps per round: the first step's mid and both possible
    // second mids are counted together (the same fp32 mids as one step at a time)
    for (int it = 0; it < a.iters; it += 2) {
      const float m0 = (lo + hi) * 0.5f;
      const float m1 = (m0 + hi) * 0.5f;     // second mid if m0 reaches the budget
      const float m2 = (lo + m0) * 0.5f;     // second mid otherwise
      int c0 = 0, c1 = 0, c2 = 0;
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        c0 += score[k] >= m0 ? size[k] : 0;
        c1 += score[k] >= m1 ? size[k] : 0;
        c2 += score[k] >= m2 ? size[k] : 0;
      }
      wave_sum3_i32_swap(c0, c1, c2);
      if (c0 >= bud_i) {
        lo = m0;
        if (it + 1 < a.iters) {
          if (c1 >= bud_i) lo = m1;
          else hi = m1;
        }
      } else {
        hi = m0;
        if (it + 1 < a.iters) {
          if (c2 >= bud_i) lo = m2;
          else hi = m2;
        }
      }
    }
    DPROBE(15);
    const float theta = all_fit ? NEG : lo;
    int carry_n = 0, carry_tok = 0;
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      if (k < nk) {
        const int c = lane + 64 * k;
        const bool sel = (size[k] > 0 && score[k] >= theta) || (a.sink > 0 && c == 0 && sz[k] > 0);
        const int si = sel ? 1 : 0;
        const int sl = sel ? sz[k] : 0;
        const int pi = wave_incl_scan_dpp(si);
        const int pt = wave_incl_scan_dpp(sl);
        if (sel) {
          const int p = carry_n + pi - 1;
          const int cum = carry_tok + pt - sl;
          s_rstart[p] = ip[k];
          s_rcum[p] = cum;
          if (leader) {
            a.rstart[h * C + p] = ip[k];
            a.rlen[h * C + p] = sl;
            a.rcum[h * C + p] = cum;
          }
        }
        carry_n += __builtin_amdgcn_readlane(pi, 63);
        carry_tok += __builtin_amdgcn_readlane(pt, 63);
      }
    }
    if (lane == 0) {
      s_cnt[0] = carry_n;
      s_cnt[1] = carry_tok;
      if (leader) {
        a.rcount[h] = carry_n;
        a.rtokens[h] = carry_tok;
      }
    }
  }
  __syncthreads();
  DPROBE(4);
}

// ------------------------------------------------------------------ step ---
template <int D, int G, int NK>
__global__ __launch_bounds__(256) void decode_step_kernel(DecodeArgs a) {
  using T = DecodeStep<D>;
  constexpr int KS = D / 32;
  static_assert(G <= 16, "query heads per KV head");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_dec[];
  __shared__ int s_rcum[MAX_C];
  __shared__ int s_rstart[MAX_C];
  __shared__ int s_cnt[2];
  __shared__ int s_table[MAX_TABLE];
  __shared__ const bf16_t* s_kaddr[T::RC];
  __shared__ const bf16_t* s_vaddr[T::RC];
  __shared__ float s_m[4][16];
  __shared__ float s_l[4][16];
  const int h = blockIdx.x;
  const int split = blockIdx.y;
  const int S = gridDim.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  DPROBE(0);
  // Q^T as the B operand: column l16 is query head h*G + l16 (zero past G);
  // in flight during the selection
  u32x4_t qr[KS];
  // the position, and the prompt length on the device: tokens moved into the
  // clusters after the prefill raise it, so a captured step reads it there.
  // Both are vector loads issued behind the selection's first loads (a scalar
  // load would be waited on by the first LDS access).
  int pos_v = 0, plen_v = 0;
  auto early_loads = [&]() {
    pos_v = __hip_atomic_load(a.pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    plen_v = __hip_atomic_load(a.plen_dev ? a.plen_dev : a.pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool ok = l16 < G;
    const bf16_t* src = a.q_post + (int64_t)(h * G + (ok ? l16 : 0)) * a.q_sh + lg * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) qr[s] = *reinterpret_cast<const u32x4_t*>(src + s * 32);
  };
  // suffix block table entries the live suffix uses (at most MAX_TABLE),
  // copied straight into LDS by wave 1 while wave 0 bisects
  int64_t plen = a.prompt_len, tb0 = 0, tb_n = 0;
  bool table_in_lds = false;
  auto after_routing = [&]() {
    if (a.plen_dev) plen = (int64_t)__builtin_amdgcn_readfirstlane(plen_v);
    // the blocks of the live suffix, positions plen .. plen + nsuf - 1
    const int64_t qp = __builtin_amdgcn_readfirstlane(pos_v);
    int64_t nsuf = qp - plen + 1;
    nsuf = nsuf < 0 ? 0 : (nsuf > (int64_t)a.max_tiles * 16 ? (int64_t)a.max_tiles * 16 : nsuf);
    tb0 = plen / a.BS;
    tb_n = nsuf > 0 ? (plen + nsuf - 1) / a.BS - tb0 + 1 : 0;
    table_in_lds = tb_n <= MAX_TABLE;
  };
  auto table_loads = [&]() {
    if (table_in_lds && wave == 1) {
#pragma unroll
      for (int k = 0; k < MAX_TABLE / 64; ++k)
        if (k * 64 + lane < tb_n)
          __builtin_amdgcn_global_load_lds((const void*)(a.table + tb0 + k * 64 + lane),
                                           (lds_void_t*)(s_table + 64 * k), 4, 0, 0);
    }
  };

  select_phase<D, G, NK>(a, h, split == 0, pos_v, plen, early_loads, after_routing, table_loads, smem_dec,
                      s_rstart, s_rcum, s_cnt);
  if (l16 >= G) {
#pragma unroll
    for (int s = 0; s < KS; ++s) qr[s] = u32x4_t{0, 0, 0, 0};
  }
  const int64_t q_pos = __builtin_amdgcn_readfirstlane(pos_v);

  // this split's range of the head's key list (prompt rows, then suffix rows)
  const int rcount = s_cnt[0];
  const int count = s_cnt[1];
  int64_t nsuf64 = q_pos - plen + 1;
  nsuf64 = nsuf64 < 0 ? 0 : (nsuf64 > (int64_t)a.max_tiles * 16 ? (int64_t)a.max_tiles * 16 : nsuf64);
  const int total = count + (int)nsuf64;
  const int per = ((total + S - 1) / S + DT - 1) / DT * DT;
  const int r_lo = min(split * per, total);
  const int r_hi = min(r_lo + per, total);
  const int64_t pplane = a.packed_len * a.Hkv * D;
  const int64_t splane = a.suffix_nblk * a.BS * a.Hkv * D;

  // Rows are taken RC at a time (one round at the headline shape).  Wave w
  // holds the K rows of 16-key groups w, w + 4, ... in registers, straight
  // from memory, and computes S^T = K Q^T for them; every wave copies a share
  // of the V rows into LDS.  P (bf16) goes through LDS, and each wave then
  // accumulates O^T = V^T P^T for its own D/4 dims over all the round's keys,
  // so the split's partial needs no fold across waves.
  constexpr int RC = T::RC, NG = T::NG, DBW = T::DBW;
  unsigned char* sV = smem_dec;                                        // RC/32 tiles of 32 V rows
  bf16_t* sP = reinterpret_cast<bf16_t*>(smem_dec + T::V_BYTES);       // [16][RC + 8]
  constexpr int LDP = RC + 8;
  const int cpos = lane % T::CH;
  const int z = (l16 >> 2) & 3;
  int vbase[4];
#pragma unroll
  for (int dl = 0; dl < 4; ++dl)
    vbase[dl] = (lg * 4 + (l16 >> 2)) * T::ROW_BYTES + 32 * (dl ^ z) + 16 * ((l16 & 3) >> 1) + 8 * (l16 & 1);

  float m_run = -INFINITY;       // of query head l16, log2 units, the same in every wave
  float l_part = 0.f;            // this lane's share of the normaliser (its keys)
  f32x4_t o[DBW];
#pragma unroll
  for (int j = 0; j < DBW; ++j) o[j] = f32x4_t{0, 0, 0, 0};

  for (int c0 = r_lo; c0 < r_hi; c0 += RC) {
    const int cn = min(RC, r_hi - c0);
    for (int t = threadIdx.x; t < RC; t += 256) {
      // address of row c0 + t of the key list (rows past cn: a valid dummy row)
      const int oo = c0 + t;
      const bf16_t* kp = a.packed + (int64_t)h * D;
      const bf16_t* vp = kp + pplane;
      if (t < cn) {
        if (oo < count) {
          int lo = 0, hi = rcount;
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (s_rcum[mid] <= oo) lo = mid + 1;
            else hi = mid;
          }
          const int r = lo > 0 ? lo - 1 : 0;
          const int64_t row = (int64_t)s_rstart[r] + (oo - s_rcum[r]);
          kp = a.packed + (row * a.Hkv + h) * D;
          vp = kp + pplane;
        } else {
          const int64_t p = plen + (oo - count);
          if (a.k_new && p == q_pos) {
            kp = a.k_new + (int64_t)h * a.kn_sh;
            vp = a.v_new + (int64_t)h * a.kn_sh;
          } else {
            // p <= the query position (an int32), the block size is positive
            const int64_t blk = (int64_t)((uint32_t)p / (uint32_t)a.BS);
            const int64_t off = p - blk * a.BS;
            const int64_t phys = table_in_lds ? (int64_t)s_table[blk - tb0] : (int64_t)a.table[blk];
            kp = a.suffix_kv + ((phys * a.BS + off) * a.Hkv + h) * D;
            vp = kp + splane;
          }
        }
      }
      s_kaddr[t] = kp;
      s_vaddr[t] = vp;
    }
    __syncthreads();
    DPROBE(5);
    // this wave's K groups into registers: lane (l16, lg) holds key g*16 + l16,
    // dims s*32 + lg*8 .. +7, the A operand of S^T
    u32x4_t kr[NG][KS];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int g = wave + 4 * j;
      if (g * 16 < cn) {
        // global (not flat) loads: a flat load is also counted by the LDS
        // counter, which the V copies below wait on for their addresses
        const global_u32x4_t* row = (const global_u32x4_t*)(s_kaddr[g * 16 + l16] + lg * 8);
#pragma unroll
        for (int s = 0; s < KS; ++s) kr[j][s] = row[s * 4];
      }
    }
    // V tiles w, w + 4, ... into LDS (16-byte chunks permuted by chunk ^ 2 (row % 4))
    for (int t0 = wave * 32; t0 < cn; t0 += 128) {
      unsigned char* dst = sV + (t0 / 32) * T::TILE_BYTES;
#pragma unroll
      for (int m = 0; m < T::INSTS; ++m) {
        const int r = m * T::RPI + lane / T::CH;
        const bf16_t* vr = s_vaddr[t0 + r];
        __builtin_amdgcn_global_load_lds((const void*)(vr + 8 * (cpos ^ ((r & 3) << 1))),
                                         (lds_void_t*)(dst + m * 1024), 16, 0, 0);
      }
    }
    // S^T: lane holds keys g*16 + lg*4 + i of query head l16
    f32x4_t sc[NG];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int g = wave + 4 * j;
      sc[j] = f32x4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      if (g * 16 < cn) {
        f32x4_t acc = f32x4_t{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KS; ++s) acc = mfma16x16x32(as_bf16x8(kr[j][s]), as_bf16x8(qr[s]), acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = (g * 16 + lg * 4 + i < cn) ? acc[i] * a.scale_log2 : -INFINITY;
          sc[j][i] = v;
          mx = fmaxf(mx, v);
        }
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (lg == 0) s_m[wave][l16] = mx;
    __syncthreads();
    const float m_new = fmaxf(m_run, fmaxf(fmaxf(s_m[0][l16], s_m[1][l16]), fmaxf(s_m[2][l16], s_m[3][l16])));
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    m_run = m_new;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int g = wave + 4 * j;
      if (g * 16 < RC) {
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pv[i] = __builtin_amdgcn_exp2f(sc[j][i] - m_use);
          sum += pv[i];
        }
        u32x2_t pk;
        pk.x = pack2bf(pv[0], pv[1]);
        pk.y = pack2bf(pv[2], pv[3]);
        *reinterpret_cast<u32x2_t*>(&sP[l16 * LDP + g * 16 + lg * 4]) = pk;
      }
    }
    l_part = l_part * alpha + sum;
#pragma unroll
    for (int j = 0; j < DBW; ++j) o[j] = o[j] * alpha;
    __builtin_amdgcn_s_waitcnt(0);           // this wave's V copies have landed
    __syncthreads();
    // O^T += V^T P^T over the round's keys, 32 at a time, for dims
    // (wave * DBW + j) * 16 .. +15; P^T as the B operand: keys
    // {4 lg..4 lg+3, 16+4 lg..16+4 lg+3} of head l16 (V^T is read in that order)
    for (int t0 = 0; t0 < cn; t0 += 32) {
      const unsigned char* tile = sV + (t0 / 32) * T::TILE_BYTES;
      u32x4_t pb;
      const u32x2_t p0 = *reinterpret_cast<const u32x2_t*>(&sP[l16 * LDP + t0 + lg * 4]);
      const u32x2_t p1 = *reinterpret_cast<const u32x2_t*>(&sP[l16 * LDP + t0 + 16 + lg * 4]);
      pb.x = p0.x; pb.y = p0.y; pb.z = p1.x; pb.w = p1.y;
#pragma unroll
      for (int j = 0; j < DBW; ++j) {
        const int db = wave * DBW + j;
        s16x4_t part[2];
#pragma unroll
        for (int hlf = 0; hlf < 2; ++hlf) {
          const unsigned char* p = tile + vbase[db & 3] + hlf * 16 * T::ROW_BYTES + 128 * (db >> 2);
          part[hlf] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
        }
        u32x4_t va;
        __builtin_memcpy(&va, part, 16);
        o[j] = mfma16x16x32(as_bf16x8(va), as_bf16x8(pb), o[j]);
      }
    }
    if (c0 + RC < r_hi) __syncthreads();     // the next round reuses the V tiles, P and addresses
  }
  DPROBEW(8);

  // the split's partial: this wave's dims of O (relative to m_run), and the
  // normaliser summed over the lanes' and the waves' keys
  float lsum = l_part;
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (lg == 0) s_l[wave][l16] = lsum;
  if (l16 < G) {
    const int hq = h * G + l16;
    float* dst = a.pacc + ((int64_t)hq * S + split) * D + lg * 4;
#pragma unroll
    for (int j = 0; j < DBW; ++j)
      *reinterpret_cast<f32x4_t*>(dst + (wave * DBW + j) * 16) = o[j];
  }
  __syncthreads();
  DPROBE(6);
  if (threadIdx.x < G) {
    const int j = threadIdx.x;
    const int hq = h * G + j;
    a.pm[(int64_t)hq * S + split] = m_run;   // every lane of head j holds the same m_run
    a.pl[(int64_t)hq * S + split] = (s_l[0][j] + s_l[1][j]) + (s_l[2][j] + s_l[3][j]);
  }
  DPROBE(7);
}

// ----------------------------------------------------------------- merge ---
// Block (query head, 64 dimensions); wave w sums splits w, w+4, ... of its 64
// dims.  The partials are loaded first; every wave derives the splits' common
// maximum and scales itself (no block barrier before the sums).
template <int D, int PS>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a, int S) {
  constexpr int PRE = 16;                 // splits per wave loaded up front
  // PS: splits per lane of the maxima and sums (S <= 64 PS)
  __shared__ float s_sc[4][64 * PS];
  __shared__ float s_red[4][64];
  const int hq = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#ifdef SBSA_DEC_PROBE
  if (threadIdx.x == 0) g_merge_probe[blockIdx.x * gridDim.y + blockIdx.y][0] = __builtin_amdgcn_s_memrealtime();
#endif
  const int d = blockIdx.y * 64 + lane;
  const float* src = a.pacc + (int64_t)hq * S * D + d;
  float v[PRE];
#pragma unroll
  for (int i = 0; i < PRE; ++i) {
    const int s = wave + 4 * i;
    v[i] = s < S ? src[(int64_t)s * D] : 0.f;
  }
  const float* pm = a.pm + (int64_t)hq * S;
  const float* pl = a.pl + (int64_t)hq * S;
  float pmv[PS], plv[PS];
#pragma unroll
  for (int k = 0; k < PS; ++k) {
    const int s = lane + 64 * k;
    pmv[k] = s < S ? pm[s] : -INFINITY;
    plv[k] = s < S ? pl[s] : 0.f;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < PS; ++k) mx = fmaxf(mx, pmv[k]);
  mx = wave_max_dpp(mx);
  const float mu = (mx == -INFINITY) ? 0.f : mx;
  float den = 0.f;
#pragma unroll
  for (int k = 0; k < PS; ++k) {
    const int s = lane + 64 * k;
    const float sc = (pmv[k] == -INFINITY) ? 0.f : exp2f(pmv[k] - mu);
    if (s < S) s_sc[wave][s] = sc;
    den += plv[k] * sc;
  }
  den = wave_sum_dpp(den);
  __builtin_amdgcn_wave_barrier();
  float num = 0.f;
#pragma unroll
  for (int i = 0; i < PRE; ++i) {
    const int s = wave + 4 * i;
    if (s < S) num += v[i] * s_sc[wave][s];
  }
  for (int s = wave + 4 * PRE; s < S; s += 4) num += src[(int64_t)s * D] * s_sc[wave][s];
  s_red[wave][lane] = num;
  __syncthreads();
  if (wave == 0) {
    const float tot = (s_red[0][lane] + s_red[1][lane]) + (s_red[2][lane] + s_red[3][lane]);
    a.out[(int64_t)hq * a.out_sh + d] = f2bf(den == 0.f ? 0.f : tot / den);
    if (lane == 0 && blockIdx.y == 0 && a.out_lse)
      a.out_lse[hq] = (den > 0.f) ? (mu + log2f(den)) * 0.69314718055994531f : -INFINITY;
  }
#ifdef SBSA_DEC_PROBE
  if (threadIdx.x == 0) g_merge_probe[blockIdx.x * gridDim.y + blockIdx.y][1] = __builtin_amdgcn_s_memrealtime();
#endif
}

template <int D, int G, int NK>
int launch_step(const DecodeArgs& a, hipStream_t stream) {
  const size_t lds = step_lds_bytes<D>(G, a.C);
  static size_t configured = 0;
  if (lds > configured) {
    if (hipFuncSetAttribute((const void*)decode_step_kernel<D, G, NK>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return SBSA_ERR_UNSUPPORTED;
    configured = lds;
  }
  const int S = a.nsplit + a.ssplit;
  hipLaunchKernelGGL((decode_step_kernel<D, G, NK>), dim3(a.Hkv, S), dim3(256), lds, stream, a);
  if (S <= 64)
    hipLaunchKernelGGL((decode_merge_kernel<D, 1>), dim3(a.Hq, D / 64), dim3(256), 0, stream, a, S);
  else
    hipLaunchKernelGGL((decode_merge_kernel<D, MAX_SPLITS / 64>), dim3(a.Hq, D / 64), dim3(256), 0, stream, a, S);
  return SBSA_OK;
}

template <int D, int G>
int launch_step_nk(const DecodeArgs& a, hipStream_t stream) {
  if (a.C <= 64) return launch_step<D, G, 1>(a, stream);
  if (a.C <= 128) return launch_step<D, G, 2>(a, stream);
  if (a.C <= 256) return launch_step<D, G, 4>(a, stream);
  return launch_step<D, G, 16>(a, stream);
}

size_t workspace_ints(int num_kv_heads, int num_clusters) {
  size_t ints = (size_t)3 * num_kv_heads * num_clusters + 3 * (size_t)num_kv_heads;
  return (ints + 63) / 64 * 64;
}

}  // namespace

extern "C" {

size_t sbsa_decode_workspace_bytes(int num_q_heads, int num_kv_heads, int num_clusters, int dim,
                                   int num_splits, int suffix_splits) {
  size_t s = (size_t)num_splits + suffix_splits;
  return workspace_ints(num_kv_heads, num_clusters) * 4 + (size_t)num_q_heads * s * dim * 4 +
         2 * (size_t)num_q_heads * s * 4;
}

}  // extern "C"

namespace {

// The step's body, shared by sbsa_decode_step (workspace from the caller) and
// sbsa_decode_step_noalloc (the library's static scratch array).
int decode_step_impl(const void* q_post, int64_t q_sh, const void* q_pre, int64_t qp_sh,
                     int router_pass, const void* k_new, const void* v_new, int64_t kn_sh,
                     const int32_t* pos, const void* codebooks, const int32_t* sizes,
                     const int32_t* indptr, const void* packed, int64_t packed_len,
                     void* suffix_kv, int64_t suffix_nblk, int suffix_block, const int32_t* table,
                     int64_t prompt_len, int max_tiles, const int32_t* prompt_len_dev,
                     const void* kpre_new, void* suffix_kpre, int num_q_heads, int num_kv_heads,
                     int num_clusters, int dim, float inv_temperature, float beta,
                     float target_tokens, int iters, int sink_tokens, float sm_scale,
                     int num_splits, int suffix_splits, void* workspace, size_t workspace_bytes,
                     void* out, int64_t out_sh, float* out_lse, int32_t* csr_out,
                     hipStream_t stream) {
  if (!q_post || !q_pre || !pos || !codebooks || !sizes || !indptr || !packed || !suffix_kv ||
      !table || !workspace || !out)
    return SBSA_ERR_ARG;
  if ((k_new == nullptr) != (v_new == nullptr)) return SBSA_ERR_ARG;
  if (num_kv_heads < 1 || num_q_heads % num_kv_heads || num_splits < 1 || suffix_splits < 1)
    return SBSA_ERR_ARG;
  if (q_sh % 8 || qp_sh % 8 || kn_sh % 8 || max_tiles < 0) return SBSA_ERR_ARG;
  if (suffix_block < 1 || suffix_nblk < 1) return SBSA_ERR_ARG;
  const int G = num_q_heads / num_kv_heads;
  const int C = num_clusters;
  if (C % 64 || C > MAX_C) return SBSA_ERR_UNSUPPORTED;
  if (num_splits + suffix_splits > MAX_SPLITS) return SBSA_ERR_UNSUPPORTED;
  if ((packed_len + 1) * num_kv_heads * (int64_t)dim >= (1ll << 31) ||
      (suffix_nblk * suffix_block + 1) * num_kv_heads * (int64_t)dim >= (1ll << 31))
    return SBSA_ERR_UNSUPPORTED;
  if (workspace_bytes < sbsa_decode_workspace_bytes(num_q_heads, num_kv_heads, C, dim, num_splits,
                                                    suffix_splits))
    return SBSA_ERR_CAPACITY;
  DecodeArgs a;
  a.q_post = (const bf16_t*)q_post;
  a.q_sh = q_sh;
  a.q_pre = (const bf16_t*)q_pre;
  a.qp_sh = qp_sh;
  a.router_pass = router_pass;
  a.k_new = (const bf16_t*)k_new;
  a.v_new = (const bf16_t*)v_new;
  a.kn_sh = kn_sh;
  a.pos = pos;
  a.codebooks = (const bf16_t*)codebooks;
  a.sizes = sizes;
  a.indptr = indptr;
  a.packed = (const bf16_t*)packed;
  a.packed_len = packed_len;
  a.suffix_kv = (bf16_t*)suffix_kv;
  a.suffix_nblk = suffix_nblk;
  a.BS = suffix_block;
  a.table = table;
  a.prompt_len = prompt_len;
  a.plen_dev = prompt_len_dev;
  a.kpre_new = (const bf16_t*)kpre_new;
  a.suffix_kpre = (bf16_t*)suffix_kpre;
  int32_t* w = (int32_t*)workspace;
  a.rstart = w;
  a.rlen = w + num_kv_heads * C;
  a.rcum = w + 2 * num_kv_heads * C;
  a.rcount = w + 3 * num_kv_heads * C;
  a.rtokens = a.rcount + num_kv_heads;
  const int S = num_splits + suffix_splits;
  a.pacc = (float*)(w + workspace_ints(num_kv_heads, C));
  a.pm = a.pacc + (size_t)num_q_heads * S * dim;
  a.pl = a.pm + (size_t)num_q_heads * S;
  a.out = (bf16_t*)out;
  a.out_sh = out_sh;
  a.out_lse = out_lse;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.C = C;
  a.G = G;
  a.nsplit = num_splits;
  a.ssplit = suffix_splits;
  a.max_tiles = max_tiles;
  a.iters = iters;
  a.sink = sink_tokens;
  a.inv_temp = inv_temperature;
  a.beta = beta;
  a.target = target_tokens;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  int rc = SBSA_ERR_UNSUPPORTED;
#define SBSA_ATT(D_, G_) if (dim == D_ && G == G_) rc = launch_step_nk<D_, G_>(a, stream);
  SBSA_ATT(128, 1) SBSA_ATT(128, 2) SBSA_ATT(128, 4) SBSA_ATT(128, 8)
  SBSA_ATT(256, 1) SBSA_ATT(256, 2) SBSA_ATT(256, 4) SBSA_ATT(256, 8)
#undef SBSA_ATT
  if (rc) return rc;
  if (csr_out) {
    if (hipMemcpyAsync(csr_out, workspace, ((size_t)3 * num_kv_heads * C + 2 * num_kv_heads) * 4,
                       hipMemcpyDeviceToDevice, stream) != hipSuccess)
      return SBSA_ERR_LAUNCH;
  }
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

// Scratch of the entry point that allocates nothing: one array per GPU, held
// until the process ends.  Host code never passes `scratch` itself to a kernel
// (in host code the name is a stand-in, not a device address): each device's
// address is looked up once with hipGetSymbolAddress, with that device
// current, and kept in scratch_ptr.
constexpr size_t DECODE_SCRATCH_BYTES = (size_t)8 << 20;
__device__ __align__(256) unsigned char scratch[DECODE_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mutex;
void* scratch_ptr[MAX_DEVICES] = {};

// This device's scratch address, looked up on its first use (nullptr on failure).
void* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    scratch_ptr[dev] = p;
  }
  return scratch_ptr[dev];
}

}  // namespace

extern "C" {

int sbsa_decode_step(const void* q_post, int64_t q_sh, const void* q_pre, int64_t qp_sh,
                     int router_pass, const void* k_new, const void* v_new, int64_t kn_sh,
                     const int32_t* pos, const void* codebooks, const int32_t* sizes,
                     const int32_t* indptr, const void* packed, int64_t packed_len,
                     void* suffix_kv, int64_t suffix_nblk, int suffix_block, const int32_t* table,
                     int64_t prompt_len, int max_tiles, const int32_t* prompt_len_dev,
                     const void* kpre_new, void* suffix_kpre, int num_q_heads, int num_kv_heads,
                     int num_clusters, int dim, float inv_temperature, float beta,
                     float target_tokens, int iters, int sink_tokens, float sm_scale,
                     int num_splits, int suffix_splits, void* workspace, size_t workspace_bytes,
                     void* out, int64_t out_sh, float* out_lse, int32_t* csr_out,
                     hipStream_t stream) {
  return decode_step_impl(q_post, q_sh, q_pre, qp_sh, router_pass, k_new, v_new, kn_sh, pos,
                          codebooks, sizes, indptr, packed, packed_len, suffix_kv, suffix_nblk,
                          suffix_block, table, prompt_len, max_tiles, prompt_len_dev, kpre_new,
                          suffix_kpre, num_q_heads, num_kv_heads,
                          num_clusters, dim, inv_temperature, beta, target_tokens, iters,
                          sink_tokens, sm_scale, num_splits, suffix_splits, workspace,
                          workspace_bytes, out, out_sh, out_lse, csr_out, stream);
}

size_t sbsa_decode_scratch_bytes(void) { return DECODE_SCRATCH_BYTES; }

int sbsa_decode_step_noalloc(const void* q_post, int64_t q_sh, const void* q_pre, int64_t qp_sh,
                             int router_pass, const void* k_new, const void* v_new, int64_t kn_sh,
                             const int32_t* pos, const void* codebooks, const int32_t* sizes,
                             const int32_t* indptr, const void* packed, int64_t packed_len,
                             void* suffix_kv, int64_t suffix_nblk, int suffix_block,
                             const int32_t* table, int64_t prompt_len, int max_tiles,
                             const int32_t* prompt_len_dev, const void* kpre_new,
                             void* suffix_kpre, int num_q_heads, int num_kv_heads,
                             int num_clusters, int dim,
                             float inv_temperature, float beta, float target_tokens, int iters,
                             int sink_tokens, float sm_scale, int num_splits, int suffix_splits,
                             void* out, int64_t out_sh, float* out_lse, int32_t* csr_out,
                             hipStream_t stream) {
  if (num_splits < 1 || suffix_splits < 1 || num_q_heads < 1 || num_kv_heads < 1 || dim < 1 ||
      num_clusters < 1)
    return SBSA_ERR_ARG;
  const size_t need = sbsa_decode_workspace_bytes(num_q_heads, num_kv_heads, num_clusters, dim,
                                                  num_splits, suffix_splits);
  if (need > DECODE_SCRATCH_BYTES) return SBSA_ERR_CAPACITY;
  void* ws = device_scratch();
  if (!ws) return SBSA_ERR_LAUNCH;
  return decode_step_impl(q_post, q_sh, q_pre, qp_sh, router_pass, k_new, v_new, kn_sh, pos,
                          codebooks, sizes, indptr, packed, packed_len, suffix_kv, suffix_nblk,
                          suffix_block, table, prompt_len, max_tiles, prompt_len_dev, kpre_new,
                          suffix_kpre, num_q_heads, num_kv_heads,
                          num_clusters, dim, inv_temperature, beta, target_tokens, iters,
                          sink_tokens, sm_scale, num_splits, suffix_splits, ws, need, out,
                          out_sh, out_lse, csr_out, stream);
}

}  // extern "C"

#ifdef SBSA_DEC_PROBE
extern "C" int sbsa_dec_probe_read(void* host, size_t bytes, void* host_merge, size_t merge_bytes) {
  if (hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dec_probe), bytes) != hipSuccess) return 1;
  if (hipMemcpyFromSymbol(host_merge, HIP_SYMBOL(g_merge_probe), merge_bytes) != hipSuccess) return 1;
  return 0;
}
#endif
