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
//      k_new/v_new); each split takes an even, 32-aligned range of it.  The
//      block resolves its rows' addresses into LDS, each wave gathers 32-key
//      tiles straight into LDS (global loads to LDS) and runs S^T = K Q^T and
//      O^T = V^T P^T on MFMA with the G query heads as columns; the waves'
//      partials are folded in LDS into the split's partial.
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

constexpr int MAX_C = 1024;
constexpr int MAX_SPLITS = 512;   // prompt + suffix splits of one step
constexpr int DT = 32;            // keys per wave tile
constexpr int ROW_CHUNK = 256;    // rows whose addresses a block resolves at once
constexpr int MAX_TABLE = 256;    // suffix block-table entries staged in LDS

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// Per-wave LDS tile: DT rows of K then DT rows of V, each row D bf16 with
// its 16-byte chunks permuted (K: chunk ^ (row % 8), V: chunk ^ 2 (row % 4))
// so that the MFMA operand reads spread over the banks.
template <int D>
struct DecodeTile {
  static constexpr int ROW_BYTES = 2 * D;
  static constexpr int CH = D / 8;               // 16-byte chunks per row
  static constexpr int RPI = 64 / CH;            // rows per wave load instruction
  static constexpr int INSTS = DT / RPI;         // load instructions per K (or V) tile
  static constexpr int KV_BYTES = DT * ROW_BYTES;
  static constexpr int WAVE_BYTES = 2 * KV_BYTES;
  static constexpr size_t STAGE_BYTES = 4 * (size_t)WAVE_BYTES;
};

// Dynamic LDS of the step kernel: the tile staging, or the selection's
// routing vectors [16][D+8] bf16 and component weights [G][C] f32.
template <int D>
size_t step_lds_bytes(int G, int C) {
  size_t sel = (size_t)16 * (D + 8) * 2 + (size_t)G * C * 4;
  return sel > DecodeTile<D>::STAGE_BYTES ? sel : DecodeTile<D>::STAGE_BYTES;
}

// ------------------------------------------------------------- selection ---
// All 256 threads.  NK = clusters per lane of wave 0 (C <= 64 NK).  Leaves
// the CSR of the head's selection in s_rstart / s_rcum (rcount entries) and
// s_cnt = {rcount, rtokens}.
template <int D, int NK, typename Prefetch>
__device__ __forceinline__ void select_phase(const DecodeArgs& a, int h, bool leader, int pos_v, int64_t plen,
                                             Prefetch prefetch, unsigned char* smem, int* s_rstart,
                                             int* s_rcum, int* s_cnt) {
  constexpr int KS = D / 32;
  constexpr int LDQ = D + 8;
  bf16_t* svec = reinterpret_cast<bf16_t*>(smem);                   // [16][LDQ]
  float* ssc = reinterpret_cast<float*>(smem + 16 * LDQ * 2);        // [G][C]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int C = a.C, G = a.G;
  const int half = D / 2;
  const int nk = C / 64;
  constexpr int PER = D / 64;

  // loads in the order of use: the router input row of this wave's first
  // head (raw bits, converted at the routing), the codebook tiles, then the
  // caller's.  Wave 0 copies the sizes and run starts straight into LDS
  // (s_rcum / s_rstart, rewritten with the CSR later).
  uint32_t vq[PER];
  if (wave < G) {
    const bf16_t* src = a.q_pre + (int64_t)(h * G + wave) * a.qp_sh;
#pragma unroll
    for (int i = 0; i < PER; ++i) vq[i] = src[lane + 64 * i];
  }
  if (wave == 0) {
    for (int k = 0; k < nk; ++k) {
      __builtin_amdgcn_global_load_lds((const void*)(a.sizes + h * C + 64 * k + lane),
                                       (lds_void_t*)(s_rcum + 64 * k), 4, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(a.indptr + h * (C + 1) + 64 * k + lane),
                                       (lds_void_t*)(s_rstart + 64 * k), 4, 0, 0);
    }
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
  // the first two codebook tiles of this wave, in flight during the routing
  u32x4_t b0[KS], b1[KS];
  if (wave < C / 16) load_cb(wave, b0);
  if (wave + 4 < C / 16) load_cb(wave + 4, b1);
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
  }
  __syncthreads();
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
  if (wave < C / 16) score_tile(wave, b0);
  if (wave + 4 < C / 16) score_tile(wave + 4, b1);
  for (int cbk = wave + 8; cbk < C / 16; cbk += 4) {
    u32x4_t b[KS];
    load_cb(cbk, b);
    score_tile(cbk, b);
  }
  __syncthreads();
  // 3. per component LSE, then w = exp(s - lse) in place
  for (int t = wave; t < G; t += 4) {
    float* row = ssc + t * C;
    float m = -INFINITY;
    for (int c = lane; c < C; c += 64) m = fmaxf(m, row[c]);
    m = wave_max_dpp(m);
    float l = 0.f;
    constexpr float LOG2E = 1.4426950408889634f;
    for (int c = lane; c < C; c += 64) l += __builtin_amdgcn_exp2f((row[c] - m) * LOG2E);
    l = wave_sum_dpp(l);
    const float lse2 = m * LOG2E + __builtin_amdgcn_logf(l);    // log2 of the normaliser
    for (int c = lane; c < C; c += 64) row[c] = __builtin_amdgcn_exp2f(__builtin_fmaf(row[c], LOG2E, -lse2));
  }
  __syncthreads();
  if (wave != 0) {
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
  } else {
    // 4. bisection and the CSR (wave 0); sizes are integers below 2^24, so
    //    the reference's fp32 sums are exact and equal these integer sums
    __builtin_amdgcn_s_waitcnt(0);       // this wave's copies into LDS have landed
    int sz[NK], ip[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      sz[k] = (k < nk) ? s_rcum[lane + 64 * k] : 0;
      ip[k] = (k < nk) ? s_rstart[lane + 64 * k] : 0;
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
        float p = 0.f;
        for (int t = 0; t < G; ++t) p += ssc[t * C + c];
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
      wave_sum3_i32_dpp(c0, c1, c2);
      if ((float)c0 >= budget) {
        lo = m0;
        if (it + 1 < a.iters) {
          if ((float)c1 >= budget) lo = m1;
          else hi = m1;
        }
      } else {
        hi = m0;
        if (it + 1 < a.iters) {
          if ((float)c2 >= budget) lo = m2;
          else hi = m2;
        }
      }
    }
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
}

// ------------------------------------------------------------------ step ---
template <int D, int G, int NK>
__global__ __launch_bounds__(256) void decode_step_kernel(DecodeArgs a) {
  using T = DecodeTile<D>;
  constexpr int KS = D / 32;
  constexpr int DB = D / 16;
  static_assert(G <= 16, "query heads per KV head");
  static_assert(16 * G * D <= (int)T::STAGE_BYTES, "wave partials fit the tile space");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_dec[];
  __shared__ int s_rcum[MAX_C];
  __shared__ int s_rstart[MAX_C];
  __shared__ int s_cnt[2];
  __shared__ int s_table[MAX_TABLE];
  __shared__ const bf16_t* s_kaddr[ROW_CHUNK];
  __shared__ const bf16_t* s_vaddr[ROW_CHUNK];
  __shared__ float s_m[4][16];
  __shared__ float s_l[4][16];
  const int h = blockIdx.x;
  const int split = blockIdx.y;
  const int S = gridDim.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  // the position as a vector load (a scalar load would be waited on by the
  // first LDS access)
  const int pos_v = __hip_atomic_load(a.pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the prompt length: tokens moved into the clusters after the prefill raise
  // it on the device, so a captured step reads it there
  const int64_t plen = a.plen_dev
      ? (int64_t)__builtin_amdgcn_readfirstlane(
            __hip_atomic_load(a.plen_dev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      : a.prompt_len;
  // suffix block table entries the live suffix may use (at most MAX_TABLE)
  const int64_t tb0 = plen / a.BS;
  const int64_t tb_n = a.max_tiles > 0 ? (plen + (int64_t)a.max_tiles * 16 - 1) / a.BS - tb0 + 1 : 0;
  const bool table_in_lds = tb_n <= MAX_TABLE;
  if (table_in_lds && wave == 0)   // copied straight into LDS; waited on in the selection
    for (int k = 0; k * 64 < tb_n; ++k)
      if (k * 64 + lane < tb_n)
        __builtin_amdgcn_global_load_lds((const void*)(a.table + tb0 + k * 64 + lane),
                                         (lds_void_t*)(s_table + 64 * k), 4, 0, 0);

  // Q^T as the B operand: column l16 is query head h*G + l16 (zero past G);
  // in flight during the selection
  u32x4_t qr[KS];
  auto load_q = [&]() {
    const bool ok = l16 < G;
    const bf16_t* src = a.q_post + (int64_t)(h * G + (ok ? l16 : 0)) * a.q_sh + lg * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qr[s] = ok ? *reinterpret_cast<const u32x4_t*>(src + s * 32) : u32x4_t{0, 0, 0, 0};
  };

  select_phase<D, NK>(a, h, split == 0, pos_v, plen, load_q, smem_dec, s_rstart, s_rcum, s_cnt);
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

  // fixed per-lane LDS offsets
  const int cpos = lane % T::CH;
  const int xb = (l16 >> 2) & 1, xl = l16 & 3;
  const int kbase_even = l16 * T::ROW_BYTES + 64 * xb + 16 * (lg ^ xl);
  const int kbase_odd = l16 * T::ROW_BYTES - 64 * xb + 16 * (lg ^ xl);
  const int z = (l16 >> 2) & 3;
  int vbase[4];
#pragma unroll
  for (int dl = 0; dl < 4; ++dl)
    vbase[dl] = (lg * 4 + (l16 >> 2)) * T::ROW_BYTES + 32 * (dl ^ z) + 16 * ((l16 & 3) >> 1) + 8 * (l16 & 1);
  unsigned char* sK = smem_dec + wave * T::WAVE_BYTES;
  unsigned char* sV = sK + T::KV_BYTES;

  float m_run = -INFINITY, l_run = 0.f;          // of query head l16
  f32x4_t o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4_t{0, 0, 0, 0};

  for (int c0 = r_lo; c0 < r_hi; c0 += ROW_CHUNK) {
    const int cn = min(ROW_CHUNK, r_hi - c0);
    {
      // address of row c0 + tid of the key list (rows past cn: a valid dummy row)
      const int oo = c0 + (int)threadIdx.x;
      const bf16_t* kp = a.packed + (int64_t)h * D;
      const bf16_t* vp = kp + pplane;
      if ((int)threadIdx.x < cn) {
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
            const int64_t blk = p / a.BS;
            const int64_t off = p - blk * a.BS;
            const int64_t phys = table_in_lds ? (int64_t)s_table[blk - tb0] : (int64_t)a.table[blk];
            kp = a.suffix_kv + ((phys * a.BS + off) * a.Hkv + h) * D;
            vp = kp + splane;
          }
        }
      }
      s_kaddr[threadIdx.x] = kp;
      s_vaddr[threadIdx.x] = vp;
    }
    __syncthreads();
    for (int t0 = wave * DT; t0 < cn; t0 += 4 * DT) {
      // gather the tile's K and V rows into this wave's LDS tile
#pragma unroll
      for (int m = 0; m < T::INSTS; ++m) {
        const int r = m * T::RPI + lane / T::CH;
        const bf16_t* kr = s_kaddr[t0 + r];
        const bf16_t* vr = s_vaddr[t0 + r];
        __builtin_amdgcn_global_load_lds((const void*)(kr + 8 * (cpos ^ (r & 7))),
                                         (lds_void_t*)(sK + m * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(vr + 8 * (cpos ^ ((r & 3) << 1))),
                                         (lds_void_t*)(sV + m * 1024), 16, 0, 0);
      }
      __builtin_amdgcn_s_waitcnt(0);
      // S^T = K Q^T: lane holds keys kb*16 + lg*4 + i of query head l16
      f32x4_t sacc[2] = {f32x4_t{0, 0, 0, 0}, f32x4_t{0, 0, 0, 0}};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const unsigned char* kb0 = sK + ((s & 1) ? kbase_odd : kbase_even) + 64 * s;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          u32x4_t ka = *reinterpret_cast<const u32x4_t*>(kb0 + kb * 16 * T::ROW_BYTES);
          sacc[kb] = mfma16x16x32(as_bf16x8(ka), as_bf16x8(qr[s]), sacc[kb]);
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (t0 + kb * 16 + lg * 4 + i >= cn) sacc[kb][i] = -INFINITY;
          mx = fmaxf(mx, sacc[kb][i]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      mx *= a.scale_log2;
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m_run - m_use);
      float sum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][i], a.scale_log2, -m_use));
          sacc[kb][i] = p;
          sum += p;
        }
      sum += __shfl_xor(sum, 16, 64);
      sum += __shfl_xor(sum, 32, 64);
      l_run = l_run * alpha + sum;
      m_run = m_new;
      // P^T as the B operand: keys {4 lg..4 lg+3, 16+4 lg..16+4 lg+3} of head l16
      u32x4_t pb;
      pb.x = pack2bf(sacc[0][0], sacc[0][1]);
      pb.y = pack2bf(sacc[0][2], sacc[0][3]);
      pb.z = pack2bf(sacc[1][0], sacc[1][1]);
      pb.w = pack2bf(sacc[1][2], sacc[1][3]);
      // O^T = alpha O^T + V^T P^T (V^T by transposing LDS reads in the same key order)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        s16x4_t part[2];
#pragma unroll
        for (int hlf = 0; hlf < 2; ++hlf) {
          const unsigned char* p = sV + vbase[db & 3] + hlf * 16 * T::ROW_BYTES + 128 * (db >> 2);
          part[hlf] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
        }
        u32x4_t va;
        __builtin_memcpy(&va, part, 16);
        o[db] = mfma16x16x32(as_bf16x8(va), as_bf16x8(pb), o[db] * alpha);
      }
    }
    __syncthreads();
  }

  // fold the four waves into the split's partial (tile space reused)
  float* s_acc = reinterpret_cast<float*>(smem_dec);   // [4][G][D]
  if (l16 < G) {
    if (lg == 0) {
      s_m[wave][l16] = m_run;
      s_l[wave][l16] = l_run;
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_acc[(wave * G + l16) * D + db * 16 + lg * 4 + i] = o[db][i];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G * D; e += 256) {
    const int j = e / D, d = e % D;
    const float mx = fmaxf(fmaxf(s_m[0][j], s_m[1][j]), fmaxf(s_m[2][j], s_m[3][j]));
    const float mu = (mx == -INFINITY) ? 0.f : mx;
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = (s_m[w][j] == -INFINITY) ? 0.f : exp2f(s_m[w][j] - mu);
      num += s_acc[(w * G + j) * D + d] * sc;
      den += s_l[w][j] * sc;
    }
    const int hq = h * G + j;
    a.pacc[((int64_t)hq * S + split) * D + d] = num;
    if (d == 0) {
      a.pm[(int64_t)hq * S + split] = mx;
      a.pl[(int64_t)hq * S + split] = den;
    }
  }
}

// ----------------------------------------------------------------- merge ---
// Block (query head, 64 dimensions); wave w sums splits w, w+4, ... of its 64
// dims.  The partials are loaded first; every wave derives the splits' common
// maximum and scales itself (no block barrier before the sums).
template <int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a, int S) {
  constexpr int PRE = 16;                 // splits per wave loaded up front
  __shared__ float s_sc[4][MAX_SPLITS];
  __shared__ float s_red[4][64];
  const int hq = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
  constexpr int PS = MAX_SPLITS / 64;
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
  hipLaunchKernelGGL(decode_merge_kernel<D>, dim3(a.Hq, D / 64), dim3(256), 0, stream, a, S);
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
