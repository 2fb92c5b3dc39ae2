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
//   1. select: one block per KV head -- suffix write, routing, scores on MFMA,
//      per-component LSE, bisection under the budget, CSR of the selection.
//   2. attend: one 4-wave block per (KV head, split) over the CSR's token
//      range (or a range of suffix tiles); the waves' partials are combined
//      in LDS, and the last block of a head to finish merges every split of
//      the head into the output (a per-head counter, reset by that block).
#include "sbsa_common.h"

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
  int32_t* rstart;          // [Hkv, C]
  int32_t* rlen;
  int32_t* rcum;
  int32_t* rcount;          // [Hkv]
  int32_t* rtokens;
  int32_t* done;            // [Hkv] finished-split counters (zero between steps)
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

// ---------------------------------------------------------------- select ---
template <int D>
__global__ __launch_bounds__(256) void decode_select_kernel(DecodeArgs a) {
  constexpr int KS = D / 32;
  constexpr int LDQ = D + 8;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  bf16_t* svec = reinterpret_cast<bf16_t*>(smem);                   // [16][LDQ]
  float* ssc = reinterpret_cast<float*>(smem + 16 * LDQ * 2);        // [G][C]
  const int h = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int C = a.C, G = a.G;
  const int half = D / 2;
  const int nk = C / 64;

  // loads that depend on nothing, issued first
  int sz[16], ip[16];
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      sz[k] = (k < nk) ? a.sizes[h * C + lane + 64 * k] : 0;
      ip[k] = (k < nk) ? a.indptr[h * (C + 1) + lane + 64 * k] : 0;
    }
  }
  // 0. suffix write of this KV head (a position past the reservation is not
  //    written: the table does not cover it)
  if (a.k_new) {
    const int64_t p = *a.pos;
    if (p >= a.prompt_len && p - a.prompt_len < (int64_t)a.max_tiles * 16) {
      const int64_t blk = p / a.BS;
      const int64_t off = p - blk * a.BS;
      const int64_t phys = a.table[blk];
      const int64_t plane = a.suffix_nblk * a.BS * a.Hkv * D;
      bf16_t* dst = a.suffix_kv + ((phys * a.BS + off) * a.Hkv + h) * D;
      for (int d = threadIdx.x; d < D; d += 256) {
        dst[d] = a.k_new[(int64_t)h * a.kn_sh + d];
        dst[plane + d] = a.v_new[(int64_t)h * a.kn_sh + d];
      }
    }
  }
  // 1. routing vectors of the G query heads (rows >= G are zero)
  for (int e = threadIdx.x; e < 16 * (D / 8); e += 256) {
    int r = e / (D / 8), ch = e % (D / 8);
    if (r >= G) *reinterpret_cast<u32x4_t*>(&svec[r * LDQ + ch * 8]) = u32x4_t{0, 0, 0, 0};
  }
  for (int t = wave; t < G; t += 4) {
    const bf16_t* src = a.q_pre + (int64_t)(h * G + t) * a.qp_sh;
    constexpr int PER = (D + 63) / 64;
    float v[PER];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int d = lane + 64 * i;
      v[i] = d < D ? bf2f(src[d]) : 0.f;
      ss += v[i] * v[i];
    }
    if (a.router_pass) {
      float n1 = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
      float ss2 = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        v[i] = round_bf16(v[i] / n1);
        ss2 += v[i] * v[i];
      }
      float n2 = fmaxf(sqrtf(wave_sum(ss2)), 1e-12f);
#pragma unroll
      for (int i = 0; i < PER; ++i) v[i] = v[i] / n2;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int d = lane + 64 * i;
      if (d < D) svec[t * LDQ + d] = f2bf(v[i]);
    }
  }
  __syncthreads();
  // 2. scores s[t][c] = v_t . c / tau on MFMA (16 rows, G real)
  u32x4_t aop[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    aop[s] = *reinterpret_cast<const u32x4_t*>(&svec[(lane & 15) * LDQ + s * 32 + (lane >> 4) * 8]);
  const bf16_t* cb = a.codebooks + (int64_t)h * 2 * C * half;
  for (int cbk = wave; cbk < C / 16; cbk += 4) {
    const int cc = cbk * 16 + (lane & 15);
    u32x4_t b[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      int d = s * 32 + (lane >> 4) * 8;
      int part = d / half;
      b[s] = *reinterpret_cast<const u32x4_t*>(cb + ((int64_t)part * C + cc) * half + (d - part * half));
    }
    f32x4_t acc = f32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma16x16x32(as_bf16x8(aop[s]), as_bf16x8(b[s]), acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int t = (lane >> 4) * 4 + i;
      if (t < G) ssc[t * C + cc] = acc[i] * a.inv_temp;
    }
  }
  __syncthreads();
  // 3. per component LSE, then w = exp(s - lse) in place
  for (int t = wave; t < G; t += 4) {
    float* row = ssc + t * C;
    float m = -INFINITY;
    for (int c = lane; c < C; c += 64) m = fmaxf(m, row[c]);
    m = wave_max(m);
    float l = 0.f;
    for (int c = lane; c < C; c += 64) l += expf(row[c] - m);
    l = wave_sum(l);
    float lse = m + logf(l);
    for (int c = lane; c < C; c += 64) row[c] = expf(row[c] - lse);
  }
  __syncthreads();
  if (wave != 0) return;
  // 4. bisection and CSR emission (wave 0); sizes are integers below 2^24, so
  //    the reference's fp32 sums are exact and equal these integer sums
  const float NEG = -3.4e38f, POS = 3.4e38f;
  float score[16];
  int size[16];
  float hi = -INFINITY, lo = INFINITY;
  int live_total = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
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
  hi = wave_max(hi) + 1e-6f;
  lo = wave_min(lo) - 1e-6f;
  lo = fminf(lo, hi - 1e-5f);
  live_total = wave_sum_i32(live_total);
  const float budget = (a.sink > 0) ? fmaxf(a.target - (float)a.sink, 0.f) : a.target;
  const bool all_fit = (float)live_total < budget;
  for (int it = 0; it < a.iters; ++it) {
    const float mid = (lo + hi) * 0.5f;
    int above = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k)
      if (k < nk && score[k] >= mid) above += size[k];
    above = wave_sum_i32(above);
    const bool reach = (float)above >= budget;
    lo = reach ? mid : lo;
    hi = reach ? hi : mid;
  }
  const float theta = all_fit ? NEG : lo;
  int carry_n = 0, carry_tok = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    if (k < nk) {
      const int c = lane + 64 * k;
      const bool sel = (size[k] > 0 && score[k] >= theta) || (a.sink > 0 && c == 0 && sz[k] > 0);
      const int si = sel ? 1 : 0;
      const int sl = sel ? sz[k] : 0;
      const int pi = wave_incl_scan(si);
      const int pt = wave_incl_scan(sl);
      if (sel) {
        const int p = carry_n + pi - 1;
        a.rstart[h * C + p] = ip[k];
        a.rlen[h * C + p] = sl;
        a.rcum[h * C + p] = carry_tok + pt - sl;
      }
      carry_n += __shfl(pi, 63, 64);
      carry_tok += __shfl(pt, 63, 64);
    }
  }
  if (lane == 0) {
    a.rcount[h] = carry_n;
    a.rtokens[h] = carry_tok;
  }
}

// ------------------------------------------------------------ attend+merge --
// A 16-key tile: S = Q K^T on MFMA with the G query heads as rows (padded to
// 16): lane (l16, lg) holds heads lg*4..lg*4+3 for key l16, and the softmax
// runs in that layout.  P V runs on the vector units, each lane owning D/64
// output dimensions of every head, with the probabilities and the V row
// addresses broadcast by readlane.  The next tile's K and V are loaded before
// the current one is consumed.
template <int D, int G>
__global__ __launch_bounds__(256) void decode_attend_kernel(DecodeArgs a) {
  constexpr int KS = D / 32;
  constexpr int DPL = D / 64;               // output dims per lane
  constexpr int VW = DPL / 2;               // 32-bit words of V per lane and key
  __shared__ int s_rcum[MAX_C];
  __shared__ int s_rstart[MAX_C];
  __shared__ float s_m[4][G];
  __shared__ float s_l[4][G];
  __shared__ float s_acc[4][G][D];
  __shared__ float s_scale[G][MAX_SPLITS];
  __shared__ int s_last;
  const int h = blockIdx.x;
  const int split = blockIdx.y;
  const int S = a.nsplit + a.ssplit;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t q_pos = *a.pos;
  const bool prompt = split < a.nsplit;

  int count = 0, rcount = 0, t_lo = 0, t_hi = 0;
  if (prompt) {
    count = a.rtokens[h];
    rcount = a.rcount[h];
    for (int i = threadIdx.x; i < rcount; i += 256) {
      s_rcum[i] = a.rcum[h * a.C + i];
      s_rstart[i] = a.rstart[h * a.C + i];
    }
    const int ntiles = (count + 15) / 16;
    const int per = (ntiles + a.nsplit - 1) / a.nsplit;
    t_lo = split * per;
    t_hi = min(t_lo + per, ntiles);
  } else {
    const int s = split - a.nsplit;
    int64_t live64 = (q_pos - a.prompt_len) / 16 + 1;
    live64 = live64 < 1 ? 1 : (live64 > a.max_tiles ? a.max_tiles : live64);
    const int live = (int)live64;
    const int per = (live + a.ssplit - 1) / a.ssplit;
    t_lo = s * per;
    t_hi = min(t_lo + per, live);
  }
  __syncthreads();

  const bf16_t* base = prompt ? a.packed : a.suffix_kv;
  const int64_t vplane = prompt ? a.packed_len * a.Hkv * D : a.suffix_nblk * a.BS * a.Hkv * D;
  // element offset of key l16 of tile t (its K row), or -1
  auto key_elem = [&](int t) -> int {
    if (prompt) {
      const int o = t * 16 + l16;
      if (o >= count) return -1;
      int lo = 0, hi = rcount;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (s_rcum[mid] <= o) lo = mid + 1;
        else hi = mid;
      }
      const int r = lo > 0 ? lo - 1 : 0;
      const int row = s_rstart[r] + (o - s_rcum[r]);
      return (row * a.Hkv + h) * D;
    }
    const int64_t p = a.prompt_len + (int64_t)t * 16 + l16;
    if (p > q_pos) return -1;
    const int64_t blk = p / a.BS;
    const int64_t off = p - blk * a.BS;
    const int64_t phys = a.table[blk];
    return (int)(((phys * a.BS + off) * a.Hkv + h) * D);
  };

  u32x4_t qa[KS];
  {
    const bool ok = l16 < G;
    const bf16_t* src = a.q_post + (int64_t)(h * G + (ok ? l16 : 0)) * a.q_sh + lg * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qa[s] = ok ? *reinterpret_cast<const u32x4_t*>(src + s * 32) : u32x4_t{0, 0, 0, 0};
  }
  float m_run[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};   // heads lg*4 + i
  float l_run[4] = {0.f, 0.f, 0.f, 0.f};
  float acc[G][DPL];
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[j][e] = 0.f;

  u32x4_t kb[KS];
  uint32_t vreg[16][VW];
  int elem = -1;
  auto load_tile = [&](int t) {
    elem = key_elem(t);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      kb[s] = elem >= 0 ? *reinterpret_cast<const u32x4_t*>(base + elem + s * 32 + lg * 8) : u32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      const int rn = __builtin_amdgcn_readlane(elem, n);
      const bf16_t* src = base + vplane + rn + lane * DPL;
      if constexpr (VW == 2) {
        u32x2_t w = rn >= 0 ? *reinterpret_cast<const u32x2_t*>(src) : u32x2_t{0, 0};
        vreg[n][0] = w.x;
        vreg[n][1] = w.y;
      } else {
        vreg[n][0] = rn >= 0 ? *reinterpret_cast<const uint32_t*>(src) : 0u;
      }
    }
  };

  int t = t_lo + wave;
  if (t < t_hi) load_tile(t);
  for (; t < t_hi; t += 4) {
    // S tile of the loaded keys
    f32x4_t sacc = f32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < KS; ++s) sacc = mfma16x16x32(as_bf16x8(qa[s]), as_bf16x8(kb[s]), sacc);
    const bool kvalid = elem >= 0;
    uint32_t vcur[16][VW];
#pragma unroll
    for (int n = 0; n < 16; ++n)
#pragma unroll
      for (int w = 0; w < VW; ++w) vcur[n][w] = vreg[n][w];
    if (t + 4 < t_hi) load_tile(t + 4);        // next tile in flight
    // softmax bookkeeping for this lane's heads (lg*4 + i), over the 16 keys
    float alpha[4], p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = kvalid ? sacc[i] * a.scale_log2 : -INFINITY;
      float mx = v;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      const float m_new = fmaxf(m_run[i], mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      alpha[i] = exp2f(m_run[i] - m_use);
      p[i] = exp2f(v - m_use);
      float sum = p[i];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) sum += __shfl_xor(sum, o, 64);
      l_run[i] = l_run[i] * alpha[i] + sum;
      m_run[i] = m_new;
    }
    // P V: every lane, every head, its own dims
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float al = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha[j & 3]), (j >> 2) * 16));
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[j][e] *= al;
#pragma unroll
      for (int n = 0; n < 16; ++n) {
        const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[j & 3]), (j >> 2) * 16 + n));
#pragma unroll
        for (int w = 0; w < VW; ++w) {
          acc[j][2 * w] += pj * __uint_as_float(vcur[n][w] << 16);
          acc[j][2 * w + 1] += pj * __uint_as_float(vcur[n][w] & 0xffff0000u);
        }
      }
    }
  }
  // the wave's partial -> LDS
  if (l16 == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = lg * 4 + i;
      if (j < G) {
        s_m[wave][j] = m_run[i];
        s_l[wave][j] = l_run[i];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < DPL; ++e) s_acc[wave][j][lane * DPL + e] = acc[j][e];
  __syncthreads();
  // combine the four waves into this split's partial
  for (int e = threadIdx.x; e < G * D; e += 256) {
    const int j = e / D, d = e % D;
    const float mx = fmaxf(fmaxf(s_m[0][j], s_m[1][j]), fmaxf(s_m[2][j], s_m[3][j]));
    const float mu = (mx == -INFINITY) ? 0.f : mx;
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = (s_m[w][j] == -INFINITY) ? 0.f : exp2f(s_m[w][j] - mu);
      num += s_acc[w][j][d] * sc;
      den += s_l[w][j] * sc;
    }
    const int hq = h * G + j;
    a.pacc[((int64_t)hq * S + split) * D + d] = num;
    if (d == 0) {
      a.pm[(int64_t)hq * S + split] = mx;
      a.pl[(int64_t)hq * S + split] = den;
    }
  }
  // the last block of this head merges every split into the output
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) s_last = (atomicAdd(&a.done[h], 1) == S - 1) ? 1 : 0;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  float* m_sh = &s_m[0][0];
  float* den_sh = &s_l[0][0];
  // split scales: wave w takes heads w, w+4, ..; its lanes stride the splits
  for (int j = wave; j < G; j += 4) {
    const int hq = h * G + j;
    const float* pm = a.pm + (int64_t)hq * S;
    const float* pl = a.pl + (int64_t)hq * S;
    float mx = -INFINITY;
    for (int s = lane; s < S; s += 64) mx = fmaxf(mx, __builtin_nontemporal_load(pm + s));
    mx = wave_max(mx);
    const float mu = (mx == -INFINITY) ? 0.f : mx;
    float den = 0.f;
    for (int s = lane; s < S; s += 64) {
      const float pmv = __builtin_nontemporal_load(pm + s);
      const float sc = (pmv == -INFINITY) ? 0.f : exp2f(pmv - mu);
      s_scale[j][s] = sc;
      den += __builtin_nontemporal_load(pl + s) * sc;
    }
    den = wave_sum(den);
    if (lane == 0) {
      m_sh[j] = mu;
      den_sh[j] = den;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G * D; e += 256) {
    const int j = e / D, d = e % D;
    const int hq = h * G + j;
    const float* src = a.pacc + (int64_t)hq * S * D + d;
    float num0 = 0.f, num1 = 0.f, num2 = 0.f, num3 = 0.f;
    int s = 0;
    for (; s + 4 <= S; s += 4) {
      num0 += __builtin_nontemporal_load(src + (int64_t)s * D) * s_scale[j][s];
      num1 += __builtin_nontemporal_load(src + (int64_t)(s + 1) * D) * s_scale[j][s + 1];
      num2 += __builtin_nontemporal_load(src + (int64_t)(s + 2) * D) * s_scale[j][s + 2];
      num3 += __builtin_nontemporal_load(src + (int64_t)(s + 3) * D) * s_scale[j][s + 3];
    }
    for (; s < S; ++s) num0 += __builtin_nontemporal_load(src + (int64_t)s * D) * s_scale[j][s];
    const float num = (num0 + num1) + (num2 + num3);
    const float den = den_sh[j];
    a.out[(int64_t)hq * a.out_sh + d] = f2bf(den == 0.f ? 0.f : num / den);
    if (d == 0 && a.out_lse)
      a.out_lse[hq] = (den > 0.f) ? (m_sh[j] + log2f(den)) * 0.69314718055994531f : -INFINITY;
  }
  if (threadIdx.x == 0) a.done[h] = 0;
}

template <int D>
int launch_select(const DecodeArgs& a, hipStream_t stream) {
  size_t lds = 16 * (D + 8) * 2 + (size_t)a.G * a.C * 4;
  hipLaunchKernelGGL(decode_select_kernel<D>, dim3(a.Hkv), dim3(256), lds, stream, a);
  return SBSA_OK;
}

template <int D, int G>
int launch_attend(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((decode_attend_kernel<D, G>), dim3(a.Hkv, a.nsplit + a.ssplit), dim3(256), 0,
                     stream, a);
  return SBSA_OK;
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

int sbsa_decode_step(const void* q_post, int64_t q_sh, const void* q_pre, int64_t qp_sh,
                     int router_pass, const void* k_new, const void* v_new, int64_t kn_sh,
                     const int32_t* pos, const void* codebooks, const int32_t* sizes,
                     const int32_t* indptr, const void* packed, int64_t packed_len,
                     void* suffix_kv, int64_t suffix_nblk, int suffix_block, const int32_t* table,
                     int64_t prompt_len, int max_tiles, int num_q_heads, int num_kv_heads,
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
  if (q_sh % 8 || qp_sh % 8) return SBSA_ERR_ARG;
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
  int32_t* w = (int32_t*)workspace;
  a.rstart = w;
  a.rlen = w + num_kv_heads * C;
  a.rcum = w + 2 * num_kv_heads * C;
  a.rcount = w + 3 * num_kv_heads * C;
  a.rtokens = a.rcount + num_kv_heads;
  a.done = a.rtokens + num_kv_heads;
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
  if (dim == 128) rc = launch_select<128>(a, stream);
  else if (dim == 256) rc = launch_select<256>(a, stream);
  if (rc) return rc;
  rc = SBSA_ERR_UNSUPPORTED;
#define SBSA_ATT(D_, G_) if (dim == D_ && G == G_) rc = launch_attend<D_, G_>(a, stream);
  SBSA_ATT(128, 1) SBSA_ATT(128, 2) SBSA_ATT(128, 4) SBSA_ATT(128, 8)
  SBSA_ATT(256, 1) SBSA_ATT(256, 2) SBSA_ATT(256, 4) SBSA_ATT(256, 8)
#undef SBSA_ATT
  if (rc) return rc;
  if (csr_out) {
    hipMemcpyAsync(csr_out, workspace, ((size_t)3 * num_kv_heads * C + 2 * num_kv_heads) * 4,
                   hipMemcpyDeviceToDevice, stream);
  }
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

}  // extern "C"
