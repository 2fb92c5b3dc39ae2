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
// Three launches, no host reads, no allocation: every size the kernels need
// (the position, the selected token count) is read on the device, so a HIP
// graph can capture the step and replay it at fixed addresses.
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

// ---------------------------------------------------------------- select ---
template <int D>
__global__ __launch_bounds__(256) void decode_select_kernel(DecodeArgs a) {
  constexpr int KS = D / 32;
  constexpr int LDQ = D + 8;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  bf16_t* svec = reinterpret_cast<bf16_t*>(smem);                   // [16][LDQ]
  float* ssc = reinterpret_cast<float*>(smem + 16 * LDQ * 2);        // [G][C]
  float* sprob = ssc + a.G * a.C;                                    // [C]
  const int h = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int C = a.C, G = a.G;
  const int half = D / 2;

  // 0. suffix write of this KV head
  // (a position past the reservation is not written: the table does not cover it)
  if (a.k_new && *a.pos - a.prompt_len < (int64_t)a.max_tiles * 16 && *a.pos >= a.prompt_len) {
    const int64_t p = *a.pos;
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
  // 1. routing vectors of the G query heads (rows >= G are zero)
  for (int e = threadIdx.x; e < 16 * (D / 8); e += 256) {
    int r = e / (D / 8), ch = e % (D / 8);
    *reinterpret_cast<u32x4_t*>(&svec[r * LDQ + ch * 8]) = u32x4_t{0, 0, 0, 0};
  }
  __syncthreads();
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
    f32x4_t acc = f32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      int d = s * 32 + (lane >> 4) * 8;
      int part = d / half;
      u32x4_t b = *reinterpret_cast<const u32x4_t*>(cb + ((int64_t)part * C + cc) * half + (d - part * half));
      acc = mfma16x16x32(as_bf16x8(aop[s]), as_bf16x8(b), acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int t = (lane >> 4) * 4 + i;
      if (t < G) ssc[t * C + cc] = acc[i] * a.inv_temp;
    }
  }
  __syncthreads();
  // 3. per component LSE, then prob[c] = sum_t exp(s - lse)
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
  for (int c = threadIdx.x; c < C; c += 256) {
    float p = 0.f;
    for (int t = 0; t < G; ++t) p += ssc[t * C + c];
    sprob[c] = p;
  }
  __syncthreads();
  // 4. bisection and CSR emission (wave 0)
  if (wave != 0) return;
  const float NEG = -3.4e38f, POS = 3.4e38f;
  const int nk = C / 64;
  float score[16], size[16], real_size[16];
  float hi = -INFINITY, lo = INFINITY;
  long long live_total = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    score[k] = NEG;
    size[k] = 0.f;
    real_size[k] = 0.f;
    if (k < nk) {
      int c = lane + 64 * k;
      float rs = (float)a.sizes[h * C + c];
      float s = (a.sink > 0 && c == 0) ? 0.f : rs;
      real_size[k] = rs;
      size[k] = s;
      bool live = s > 0.f;
      float sc = logf(fmaxf(sprob[c], 1e-38f));
      if (a.beta != 0.f) sc = sc - a.beta * logf(1.0f + s);
      sc = live ? sc : NEG;
      score[k] = sc;
      hi = fmaxf(hi, sc);
      lo = fminf(lo, live ? sc : POS);
      if (live) live_total += (long long)s;
    }
  }
  hi = wave_max(hi) + 1e-6f;
  lo = wave_min(lo) - 1e-6f;
  lo = fminf(lo, hi - 1e-5f);
  live_total = wave_sum_i64(live_total);
  const float budget = (a.sink > 0) ? fmaxf(a.target - (float)a.sink, 0.f) : a.target;
  const bool all_fit = (float)live_total < budget;
  for (int it = 0; it < a.iters; ++it) {
    float mid = (lo + hi) * 0.5f;
    long long above = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k)
      if (k < nk && score[k] >= mid) above += (long long)size[k];
    above = wave_sum_i64(above);
    bool reach = (float)above >= budget;
    lo = reach ? mid : lo;
    hi = reach ? hi : mid;
  }
  const float theta = all_fit ? NEG : lo;
  int carry_n = 0, carry_tok = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    if (k < nk) {
      int c = lane + 64 * k;
      bool sel = (size[k] > 0.f && score[k] >= theta) || (a.sink > 0 && c == 0 && real_size[k] > 0.f);
      int si = sel ? 1 : 0;
      int sl = sel ? (int)real_size[k] : 0;
      int pi = wave_incl_scan(si);
      int pt = wave_incl_scan(sl);
      if (sel) {
        int p = carry_n + pi - 1;
        a.rstart[h * C + p] = a.indptr[h * (C + 1) + c];
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

// ---------------------------------------------------------------- attend ---
// One wave per (KV head, split).  A 16-key tile: S = Q K^T on MFMA with the G
// query heads as rows (padded to 16), then the softmax bookkeeping and
// P V on the vector units, each lane owning D/64 output dimensions of every
// head.  K and V of the next tile are loaded before the current one is
// consumed.
template <int D, int G>
__global__ __launch_bounds__(64) void decode_attend_kernel(DecodeArgs a) {
  constexpr int KS = D / 32;
  constexpr int DPL = D / 64;               // output dims per lane
  __shared__ float sp[16 * 17];             // scaled scores [row][key]
  __shared__ int srow[16];
  const int h = blockIdx.x;
  const int split = blockIdx.y;
  const int S = a.nsplit + a.ssplit;
  const int lane = threadIdx.x;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t q_pos = *a.pos;

  u32x4_t qa[KS];
  {
    const bool ok = l16 < G;
    const bf16_t* src = a.q_post + (int64_t)(h * G + (ok ? l16 : 0)) * a.q_sh + lg * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qa[s] = ok ? *reinterpret_cast<const u32x4_t*>(src + s * 32) : u32x4_t{0, 0, 0, 0};
  }
  float m[G], l[G], acc[G][DPL];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[j][e] = 0.f;
  }

  // tile range and addressing
  const bool prompt = split < a.nsplit;
  int t_lo, t_hi;     // tile indices
  int rcount = 0;
  if (prompt) {
    const int count = a.rtokens[h];
    rcount = a.rcount[h];
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
  const int count = prompt ? a.rtokens[h] : 0;
  const int* rcum = a.rcum + h * a.C;
  const int* rstart = a.rstart + h * a.C;
  const int64_t plane_p = a.packed_len * a.Hkv * D;
  const int64_t plane_s = a.suffix_nblk * a.BS * a.Hkv * D;

  // address of key l16 of tile t (element offset of its K row, or -1)
  auto key_addr = [&](int t) -> int64_t {
    if (prompt) {
      const int o = t * 16 + l16;
      if (o >= count) return -1;
      int lo = 0, hi = rcount;
      while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (rcum[mid] <= o) lo = mid + 1;
        else hi = mid;
      }
      const int r = lo > 0 ? lo - 1 : 0;
      const int64_t row = (int64_t)rstart[r] + (o - rcum[r]);
      return (row * a.Hkv + h) * D;
    } else {
      const int64_t p = a.prompt_len + (int64_t)t * 16 + l16;
      if (p > q_pos) return -1;
      const int64_t blk = p / a.BS;
      const int64_t off = p - blk * a.BS;
      const int64_t phys = a.table[blk];
      return ((phys * a.BS + off) * a.Hkv + h) * D;
    }
  };
  const bf16_t* kbase = prompt ? a.packed : a.suffix_kv;
  const int64_t vplane = prompt ? plane_p : plane_s;

  u32x4_t kb[KS];
  int64_t addr = -1;
  if (t_lo < t_hi) {
    addr = key_addr(t_lo);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      kb[s] = addr >= 0 ? *reinterpret_cast<const u32x4_t*>(kbase + addr + s * 32 + lg * 8) : u32x4_t{0, 0, 0, 0};
  }
  for (int t = t_lo; t < t_hi; ++t) {
    // S tile
    f32x4_t sacc = f32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < KS; ++s) sacc = mfma16x16x32(as_bf16x8(qa[s]), as_bf16x8(kb[s]), sacc);
    // publish scores and rows
    if (lg * 4 < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = lg * 4 + i;
        sp[row * 17 + l16] = (addr >= 0) ? sacc[i] * a.scale_log2 : -INFINITY;
      }
    }
    if (lg == 0) srow[l16] = (int)(addr >= 0 ? addr / D : -1);
    __syncthreads();
    // V rows of this tile (each lane its DPL dims), and the next tile's K
    uint32_t vreg[16][DPL / 2];
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      const int r = srow[n];
      if (r >= 0) {
        const bf16_t* src = kbase + vplane + (int64_t)r * D + lane * DPL;
        if constexpr (DPL == 4) {
          u32x2_t w = *reinterpret_cast<const u32x2_t*>(src);
          vreg[n][0] = w.x;
          vreg[n][1] = w.y;
        } else {
          vreg[n][0] = *reinterpret_cast<const uint32_t*>(src);
        }
      } else {
#pragma unroll
        for (int e = 0; e < DPL / 2; ++e) vreg[n][e] = 0;
      }
    }
    if (t + 1 < t_hi) {
      addr = key_addr(t + 1);
#pragma unroll
      for (int s = 0; s < KS; ++s)
        kb[s] = addr >= 0 ? *reinterpret_cast<const u32x4_t*>(kbase + addr + s * 32 + lg * 8) : u32x4_t{0, 0, 0, 0};
    }
    // softmax bookkeeping (lane-uniform) and P V
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float sv[16];
      float mx = -INFINITY;
#pragma unroll
      for (int n = 0; n < 16; ++n) {
        sv[n] = sp[j * 17 + n];
        mx = fmaxf(mx, sv[n]);
      }
      const float m_new = fmaxf(m[j], mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m[j] - m_use);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[j][e] *= alpha;
#pragma unroll
      for (int n = 0; n < 16; ++n) {
        const float p = exp2f(sv[n] - m_use);
        sum += p;
#pragma unroll
        for (int e = 0; e < DPL / 2; ++e) {
          const uint32_t w = vreg[n][e];
          acc[j][2 * e] += p * __uint_as_float(w << 16);
          acc[j][2 * e + 1] += p * __uint_as_float(w & 0xffff0000u);
        }
      }
      l[j] = l[j] * alpha + sum;
      m[j] = m_new;
    }
    __syncthreads();
  }
  // partials
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const int hq = h * G + j;
    float* dst = a.pacc + ((int64_t)hq * S + split) * D + lane * DPL;
#pragma unroll
    for (int e = 0; e < DPL; ++e) dst[e] = acc[j][e];
    if (lane == 0) {
      a.pm[(int64_t)hq * S + split] = m[j];
      a.pl[(int64_t)hq * S + split] = l[j];
    }
  }
}

// ----------------------------------------------------------------- merge ---
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a, int D) {
  const int hq = blockIdx.x;
  const int S = a.nsplit + a.ssplit;
  __shared__ float s_scale[256];
  __shared__ float s_den;
  __shared__ float s_m;
  if (threadIdx.x < 64) {
    float mx = -INFINITY;
    for (int s = threadIdx.x; s < S; s += 64) mx = fmaxf(mx, a.pm[(int64_t)hq * S + s]);
    mx = wave_max(mx);
    const float m_use = (mx == -INFINITY) ? 0.f : mx;
    float den = 0.f;
    for (int s = threadIdx.x; s < S; s += 64) {
      const float pmv = a.pm[(int64_t)hq * S + s];
      const float sc = (pmv == -INFINITY) ? 0.f : exp2f(pmv - m_use);
      s_scale[s] = sc;
      den += a.pl[(int64_t)hq * S + s] * sc;
    }
    den = wave_sum(den);
    if (threadIdx.x == 0) {
      s_den = den;
      s_m = m_use;
    }
  }
  __syncthreads();
  const float den = s_den;
  const float inv = (den == 0.f) ? 1.f : 1.f / den;
  for (int d = threadIdx.x; d < D; d += 256) {
    float num = 0.f;
    for (int s = 0; s < S; ++s) num += a.pacc[((int64_t)hq * S + s) * D + d] * s_scale[s];
    a.out[(int64_t)hq * a.out_sh + d] = f2bf(num * inv);
  }
  if (threadIdx.x == 0 && a.out_lse)
    a.out_lse[hq] = (den > 0.f) ? (s_m + log2f(den)) * 0.69314718055994531f : -INFINITY;
}

template <int D>
int launch_select(const DecodeArgs& a, hipStream_t stream) {
  size_t lds = 16 * (D + 8) * 2 + (size_t)a.G * a.C * 4 + (size_t)a.C * 4;
  hipLaunchKernelGGL(decode_select_kernel<D>, dim3(a.Hkv), dim3(256), lds, stream, a);
  return SBSA_OK;
}

template <int D, int G>
int launch_attend(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((decode_attend_kernel<D, G>), dim3(a.Hkv, a.nsplit + a.ssplit), dim3(64), 0,
                     stream, a);
  return SBSA_OK;
}

}  // namespace

extern "C" {

size_t sbsa_decode_workspace_bytes(int num_q_heads, int num_kv_heads, int num_clusters, int dim,
                                   int num_splits, int suffix_splits) {
  size_t s = (size_t)num_splits + suffix_splits;
  size_t ints = (size_t)3 * num_kv_heads * num_clusters + 2 * (size_t)num_kv_heads;
  ints = (ints + 63) / 64 * 64;
  return ints * 4 + (size_t)num_q_heads * s * dim * 4 + 2 * (size_t)num_q_heads * s * 4;
}

int sbsa_decode_step(const void* q_post, int64_t q_sh, const void* q_pre, int64_t qp_sh,
                     int router_pass, const void* k_new, const void* v_new, int64_t kn_sh, const int32_t* pos,
                     const void* codebooks, const int32_t* sizes, const int32_t* indptr,
                     const void* packed, int64_t packed_len, void* suffix_kv, int64_t suffix_nblk,
                     int suffix_block, const int32_t* table, int64_t prompt_len, int max_tiles,
                     int num_q_heads, int num_kv_heads, int num_clusters, int dim,
                     float inv_temperature, float beta, float target_tokens, int iters,
                     int sink_tokens, float sm_scale, int num_splits, int suffix_splits,
                     void* workspace, size_t workspace_bytes, void* out, int64_t out_sh,
                     float* out_lse, int32_t* csr_out, hipStream_t stream) {
  if (!q_post || !q_pre || !pos || !codebooks || !sizes || !indptr || !packed || !suffix_kv ||
      !table || !workspace || !out)
    return SBSA_ERR_ARG;
  if ((k_new == nullptr) != (v_new == nullptr)) return SBSA_ERR_ARG;
  if (num_kv_heads < 1 || num_q_heads % num_kv_heads || num_splits < 1 || suffix_splits < 1)
    return SBSA_ERR_ARG;
  if (q_sh % 8 || qp_sh % 8) return SBSA_ERR_ARG;
  const int G = num_q_heads / num_kv_heads;
  const int C = num_clusters;
  if (C % 64 || C > 1024) return SBSA_ERR_UNSUPPORTED;
  if (num_splits + suffix_splits > 256) return SBSA_ERR_UNSUPPORTED;
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
  size_t ints = (size_t)3 * num_kv_heads * C + 2 * (size_t)num_kv_heads;
  ints = (ints + 63) / 64 * 64;
  const int S = num_splits + suffix_splits;
  a.pacc = (float*)(w + ints);
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
  hipLaunchKernelGGL(decode_merge_kernel, dim3(num_q_heads), dim3(256), 0, stream, a, dim);
  if (csr_out) {
    hipMemcpyAsync(csr_out, workspace, ((size_t)3 * num_kv_heads * C + 2 * num_kv_heads) * 4,
                   hipMemcpyDeviceToDevice, stream);
  }
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

}  // extern "C"
