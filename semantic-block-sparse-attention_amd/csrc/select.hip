// S2 centroid scoring + S3 budget selection, S3c causal snapshot, and S4 the
// reverse index with the work list of the KV-outer prefill, for gfx950.
//
// Reference behaviour (pfnet-research/semantic-block-sparse-attention):
//   fused_select.py:1062-1247  _flat_scores_qtiled_kernel (score, LSE, mixture prob)
//   fused_select.py:604-646    _streaming_select_kernel RESIDENT (bisection, bitmask, qmask)
//   fused_select.py:806-919    theta_select_bitmask_flat (the contract)
//   fused_prefill.py:126-135   CausalSnapshot.advance
//   kv_outer.py:41-173, 254-329 build_reverse_index
#include "sbsa_common.h"

namespace {

// ------------------------------------------------------------- S2 + S3 -----
// One block = QT queries x one KV head.  Rows of the score GEMM are
// (query, component) pairs, R = QT * G of them; the four waves split the
// clusters.  Scores live in LDS; each wave then selects for its queries.
struct SelectArgs {
  const bf16_t* vectors;   // [Q, Hq, D] routing vectors
  int64_t v_sq, v_sh;      // element strides
  const float* logmix;     // [Q, Hq] or null (uniform: 0)
  const bf16_t* codebooks; // [Hkv, 2, C, D/2]
  const int32_t* sizes;    // sizes[b * s_nb + h * s_h + c]
  int64_t s_nb, s_h;
  int32_t* bitmask;        // [NB, Hkv, C/32] (atomic OR) or null
  int32_t* qmask;          // [Q, Hkv, C/32] or null
  int32_t* counts;         // [Q, Hkv] or null
  int32_t* tokens;         // [Q, Hkv] or null
  float* prob_out;         // [Q, Hkv, C] or null
  float* theta_out;        // [Q, Hkv] or null
  int Q, Hq, Hkv, C, G, g_union, iters, sink;
  float inv_temp, beta, target;
};

template <int D, int NK>
__global__ __launch_bounds__(256) void score_select_kernel(SelectArgs a, int R) {
  constexpr int KS = D / 32;
  constexpr int LDQ = D + 8;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  bf16_t* sq = reinterpret_cast<bf16_t*>(smem);                      // [R][LDQ]
  float* ssc = reinterpret_cast<float*>(smem + (size_t)R * LDQ * 2);  // [R][C+1]
  const int C = a.C, G = a.G;
  const int LDS_C = C + 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.y;
  const int QT = R / G;
  const int q0 = blockIdx.x * QT;
  const int half = D / 2;

  // Q tile -> LDS (rows r = query*G + component)
  for (int e = threadIdx.x; e < R * (D / 8); e += 256) {
    int r = e / (D / 8), ch = e % (D / 8);
    int q = q0 + r / G, t = r % G;
    u32x4_t v = u32x4_t{0, 0, 0, 0};
    if (q < a.Q)
      v = *reinterpret_cast<const u32x4_t*>(a.vectors + (int64_t)q * a.v_sq + (int64_t)(h * G + t) * a.v_sh + ch * 8);
    *reinterpret_cast<u32x4_t*>(&sq[r * LDQ + ch * 8]) = v;
  }
  __syncthreads();

  // scores: each wave takes C/4 clusters (a multiple of 16)
  const int cols_per_wave = C / 4;
  const bf16_t* cb = a.codebooks + (int64_t)h * 2 * C * half;
  for (int cbk = 0; cbk < cols_per_wave / 16; ++cbk) {
    const int col0 = wave * cols_per_wave + cbk * 16;
    const int cc = col0 + (lane & 15);
    u32x4_t bop[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      int d = s * 32 + (lane >> 4) * 8;
      int part = d / half;
      bop[s] = *reinterpret_cast<const u32x4_t*>(cb + ((int64_t)part * C + cc) * half + (d - part * half));
    }
    for (int rb = 0; rb < R / 16; ++rb) {
      f32x4_t acc = f32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        u32x4_t aop = *reinterpret_cast<const u32x4_t*>(&sq[(rb * 16 + (lane & 15)) * LDQ + s * 32 + (lane >> 4) * 8]);
        acc = mfma16x16x32(as_bf16x8(aop), as_bf16x8(bop[s]), acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) ssc[(rb * 16 + (lane >> 4) * 4 + i) * LDS_C + cc] = acc[i] * a.inv_temp;
    }
  }
  __syncthreads();

  // per row: lse over C, then w = exp(s - lse + logmix) in place (base-2
  // hardware exp/log: about 1 ulp, far below the selection's near-tie margin)
  constexpr float LOG2E = 1.4426950408889634f;
  for (int r = wave; r < R; r += 4) {
    float* row = ssc + r * LDS_C;
    float m = -INFINITY;
    for (int c = lane; c < C; c += 64) m = fmaxf(m, row[c]);
    m = wave_max_dpp(m);
    float l = 0.f;
    for (int c = lane; c < C; c += 64) l += __builtin_amdgcn_exp2f((row[c] - m) * LOG2E);
    l = wave_sum_dpp(l);
    int q = q0 + r / G, t = r % G;
    float lm = 0.f;
    if (a.logmix && q < a.Q) lm = a.logmix[(int64_t)q * a.Hq + h * G + t];
    // log2 of exp(lm) / (sum exp(s))
    const float off2 = (lm - m) * LOG2E - __builtin_amdgcn_logf(l);
    for (int c = lane; c < C; c += 64) row[c] = __builtin_amdgcn_exp2f(__builtin_fmaf(row[c], LOG2E, off2));
  }
  __syncthreads();

  // selection, one wave per query; lane holds clusters lane + 64k
  const int W = C / 32;
  const float NEG = -3.4e38f, POS = 3.4e38f;
  for (int qi = wave; qi < QT; qi += 4) {
    const int q = q0 + qi;
    if (q >= a.Q) break;
    const int b = q / a.g_union;
    const int32_t* sz = a.sizes + (int64_t)b * a.s_nb + (int64_t)h * a.s_h;
    float score[NK], size[NK];
    float real_size[NK];
    int size_i[NK];
    const int nk = C / 64;
    float hi = -INFINITY, lo = INFINITY;
    int live_total = 0;      // token counts: sizes sum to at most the prompt length
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      score[k] = NEG;
      size[k] = 0.f;
      size_i[k] = 0;
      real_size[k] = 0.f;
      if (k < nk) {
        int c = lane + 64 * k;
        float p = 0.f;
        for (int t = 0; t < G; ++t) p += ssc[(qi * G + t) * LDS_C + c];
        if (a.prob_out) a.prob_out[((int64_t)q * a.Hkv + h) * C + c] = p;
        float rs = (float)sz[c];
        float s = (a.sink > 0 && c == 0) ? 0.f : rs;  // the sink is hidden from the search
        real_size[k] = rs;
        size[k] = s;
        size_i[k] = (int)s;
        bool live = s > 0.f;
        constexpr float LN2 = 0.69314718055994531f;
        float sc = __builtin_amdgcn_logf(fmaxf(p, 1e-38f)) * LN2;
        if (a.beta != 0.f) sc = sc - a.beta * (__builtin_amdgcn_logf(1.0f + s) * LN2);
        sc = live ? sc : NEG;
        score[k] = sc;
        hi = fmaxf(hi, sc);
        lo = fminf(lo, live ? sc : POS);
        if (live) live_total += (int)s;
      }
    }
    hi = wave_max_dpp(hi) + 1e-6f;
    lo = wave_min_dpp(lo) - 1e-6f;
    lo = fminf(lo, hi - 1e-5f);
    live_total = wave_sum_i32_dpp(live_total);
    float budget = a.target;
    if (a.sink > 0) budget = fmaxf(a.target - (float)a.sink, 0.f);
    const bool all_fit = (float)live_total < budget;
    const int bud_i = budget_count(budget);
    // two bisection steps per round: the first step's mid and both possible
    // second mids are counted together (the same fp32 mids as one step at a time)
    for (int it = 0; it < a.iters; it += 2) {
      const float m0 = (lo + hi) * 0.5f;
      const float m1 = (m0 + hi) * 0.5f;     // second mid if m0 reaches the budget
      const float m2 = (lo + m0) * 0.5f;     // second mid otherwise
      int c0 = 0, c1 = 0, c2 = 0;
#pragma unroll
      for (int k = 0; k < NK; ++k) {         // size_i[k] is 0 past the C clusters
        c0 += score[k] >= m0 ? size_i[k] : 0;
        c1 += score[k] >= m1 ? size_i[k] : 0;
        c2 += score[k] >= m2 ? size_i[k] : 0;
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
    const float theta = all_fit ? NEG : lo;
    int nsel = 0;
    int ntok = 0;
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      if (k < nk) {
        int c = lane + 64 * k;
        bool sel = (size[k] > 0.f && score[k] >= theta) || (a.sink > 0 && c == 0 && real_size[k] > 0.f);
        nsel += sel ? 1 : 0;
        ntok += sel ? (int)real_size[k] : 0;
        uint64_t ball = __ballot(sel);
        if (lane < 2) {
          uint32_t word = (uint32_t)(ball >> (32 * lane));
          int wi = 2 * k + lane;
          if (a.qmask) a.qmask[((int64_t)q * a.Hkv + h) * W + wi] = (int32_t)word;
          if (a.bitmask && word) atomicOr((unsigned int*)&a.bitmask[((int64_t)b * a.Hkv + h) * W + wi], word);
        }
      }
    }
    nsel = wave_sum_i32_dpp(nsel);
    ntok = wave_sum_i32_dpp(ntok);
    if (lane == 0) {
      if (a.counts) a.counts[(int64_t)q * a.Hkv + h] = nsel;
      if (a.tokens) a.tokens[(int64_t)q * a.Hkv + h] = (int32_t)ntok;
      if (a.theta_out) a.theta_out[(int64_t)q * a.Hkv + h] = theta;
    }
  }
}

// ---------------------------------------------------------------- S3c ------
// |{keys of cluster c with position < limit}|: the run is position-sorted.
__global__ void causal_sizes_kernel(const int32_t* __restrict__ posting, int64_t width,
                                    const int32_t* __restrict__ indptr,
                                    const int32_t* __restrict__ sizes, int hkv, int C,
                                    int64_t limit, int32_t* __restrict__ out) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= hkv * C) return;
  int h = e / C, c = e % C;
  const int32_t* run = posting + (int64_t)h * width + indptr[h * (C + 1) + c];
  int lo = 0, hi = sizes[e];
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if ((int64_t)run[mid] < limit) lo = mid + 1;
    else hi = mid;
  }
  out[e] = lo;
}

// ----------------------------------------------------------------- S4 ------
// Per (head, cluster): the queries whose qmask has the cluster (and the
// cluster has visible rows), in query order.  Pass 0 counts, pass 1 fills
// qvals[rev_indptr + rank] and qrank[q, h, c] = rank.
__global__ __launch_bounds__(256) void rev_pass_kernel(int pass, const int32_t* __restrict__ qmask,
                                                       int Q, int hkv, int C,
                                                       const int32_t* __restrict__ nvis,
                                                       int32_t* __restrict__ rev_counts,
                                                       const int32_t* __restrict__ rev_indptr,
                                                       int32_t* __restrict__ qvals,
                                                       int32_t* __restrict__ qrank) {
  __shared__ int wcnt[4];
  const int hc = blockIdx.x;
  const int h = hc / C, c = hc % C;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int W = C / 32;
  const bool live = nvis[hc] > 0;
  int run = 0;
  const int base_out = (pass == 1) ? rev_indptr[hc] : 0;
  for (int q0 = 0; q0 < Q; q0 += 256) {
    int q = q0 + threadIdx.x;
    bool bit = false;
    if (live && q < Q) bit = (qmask[((int64_t)q * hkv + h) * W + (c >> 5)] >> (c & 31)) & 1;
    uint64_t ball = __ballot(bit);
    if (lane == 0) wcnt[wave] = __popcll(ball);
    __syncthreads();
    int off = run;
    for (int w = 0; w < wave; ++w) off += wcnt[w];
    int before = __popcll(ball & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
    if (pass == 1 && bit) {
      int rank = off + before;
      qvals[base_out + rank] = q;
      qrank[((int64_t)q * hkv + h) * C + c] = rank;
    }
    run += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
    __syncthreads();
  }
  if (pass == 0 && threadIdx.x == 0) rev_counts[hc] = run;
}

// Exclusive scan of the Hkv*C counts (one block), total into rev_indptr[n].
__global__ __launch_bounds__(1024) void rev_scan_kernel(const int32_t* __restrict__ counts, int n,
                                                        int32_t* __restrict__ indptr,
                                                        int64_t* __restrict__ nnz) {
  __shared__ int wsum[16];
  __shared__ int carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int base = 0; base < n; base += 1024) {
    int i = base + threadIdx.x;
    int v = (i < n) ? counts[i] : 0;
    int incl = wave_incl_scan(v);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int off = carry;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    if (i < n) indptr[i] = off + incl - v;
    __syncthreads();
    if (threadIdx.x == 1023) carry = off + incl;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    indptr[n] = carry;
    *nnz = carry;
  }
}

// Work list of the KV-outer body, one segment per XCD so that the items that
// read the same K/V (the query tiles of one KV head's window, the query tiles
// of one cluster) run on one XCD and share its L2.  Items within a segment:
// local-window items first (longest first), then cluster items, longest
// cluster first (visible rows descending, ties in (head, cluster) order), so
// that the items claimed last, when the queues run dry, are the shortest.  Item = {head, cluster or -1, first query slot, query
// count}.  queue = {n[8], off[8], counter[8]}; the counters are zeroed here.
// One block: per-XCD counts, each source's first item (one pass of eight
// per-segment wave scans over each round of 1024 sources), then one thread
// per source writes its items (a window tile, or the query tiles of one
// (head, cluster)).
__device__ __forceinline__ int local_xcd(int h, int tile, int hkv) {
  const int per = hkv >= 8 ? 1 : 8 / hkv;      // XCDs per KV head
  return ((h * per) + (tile % per)) & 7;
}
__device__ __forceinline__ int cluster_xcd(int h, int c, int C) { return (h * C + c) & 7; }

struct ItemSource {
  int x, n, h, c, qb, qn;
};

// order: cluster sources by enumeration position e' = 8 r + x, the source of
// rank r in segment x (every segment's sources keep their segment)
__device__ __forceinline__ ItemSource item_source(const int32_t* rev_counts, const int* order, int s,
                                                  int nloc, int hkv, int C, int Qc, int QT) {
  ItemSource r;
  const int nl = nloc * hkv;
  if (s < nl) {
    const int k = s / hkv, tile = nloc - 1 - k;
    r.h = s % hkv;
    r.c = -1;
    r.qb = tile * QT;
    r.qn = min(QT, Qc - r.qb);
    r.n = 1;
    r.x = local_xcd(r.h, tile, hkv);
  } else {
    const int e = order[s - nl];
    r.h = e / C;
    r.c = e % C;
    r.qb = 0;
    r.qn = rev_counts[e];
    r.n = (r.qn + QT - 1) / QT;
    r.x = cluster_xcd(r.h, r.c, C);
  }
  return r;
}

// queue[QUEUE_OVERFLOW]: 1 when the chunk's partial entries pass the partial
// buffer's capacity (the list is then empty)
constexpr int QUEUE_OVERFLOW = 24;

__global__ __launch_bounds__(1024) void build_items_kernel(const int32_t* __restrict__ rev_counts,
                                                           int hkv, int C, int Qc, int QT,
                                                           int has_local, const int32_t* __restrict__ indptr,
                                                           const int32_t* __restrict__ nvis,
                                                           const int32_t* __restrict__ rev_indptr,
                                                           PrefillItem* __restrict__ items,
                                                           int32_t* __restrict__ queue,
                                                           int64_t cap, int64_t partials_cap) {
  extern __shared__ int s_first[];     // [nsrc] first item of each source, then
                                       // [hkv C] sort keys and [hkv C] source order
  __shared__ int cnt[8];
  __shared__ int base[8];
  __shared__ int wsum[16][8];
  const int nloc = has_local ? (Qc + QT - 1) / QT : 0;
  const int ncl = hkv * C;
  const int nsrc = nloc * hkv + ncl;
  int* s_key = s_first + nsrc;
  int* s_order = s_key + ncl;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x < 8) cnt[threadIdx.x] = 0;
  // cluster sources ranked within their segment (e & 7) by visible rows,
  // descending; sources without queries last
  for (int e = threadIdx.x; e < ncl; e += 1024) s_key[e] = rev_counts[e] > 0 ? nvis[e] : -1;
  __syncthreads();
  for (int e = threadIdx.x; e < ncl; e += 1024) {
    const int k = s_key[e];
    int rank = 0;
    for (int e2 = e & 7; e2 < ncl; e2 += 8) {
      const int k2 = s_key[e2];
      rank += (k2 > k || (k2 == k && e2 < e)) ? 1 : 0;
    }
    s_order[8 * rank + (e & 7)] = e;
  }
  __syncthreads();
  for (int s = threadIdx.x; s < nsrc; s += 1024) {
    const ItemSource si = item_source(rev_counts, s_order, s, nloc, hkv, C, Qc, QT);
    if (si.n) atomicAdd(&cnt[si.x], si.n);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int x = 0; x < 8; ++x) {
      base[x] = run;        // the segment's offset, then its running fill
      run += cnt[x];
    }
  }
  __syncthreads();
  // a chunk whose partial entries (rev_indptr[hkv C]) pass the partial
  // buffer's capacity gets an empty list and the overflow flag: nothing of it
  // is written, and the caller runs it again with a buffer of its exact size
  const bool overflow = partials_cap > 0 && (int64_t)rev_indptr[ncl] > partials_cap;
  if (threadIdx.x < 8) {
    const int x = threadIdx.x;
    const int64_t end = min((int64_t)base[x] + cnt[x], cap);
    queue[x] = overflow ? 0 : (int32_t)max((int64_t)0, end - base[x]);   // n
    queue[8 + x] = base[x];                              // offset
    queue[16 + x] = 0;                                   // counter
    if (x == 0) queue[QUEUE_OVERFLOW] = overflow ? 1 : 0;
  }
  if (overflow) return;
  // each source's first item: the segment's fill plus the items of the
  // segment's earlier sources, by one scan per segment over each round of
  // 1024 sources (sources keep their order within a segment)
  for (int r0 = 0; r0 < nsrc; r0 += 1024) {
    const int s = r0 + threadIdx.x;
    int n = 0, x = 0;
    if (s < nsrc) {
      const ItemSource si = item_source(rev_counts, s_order, s, nloc, hkv, C, Qc, QT);
      n = si.n;
      x = si.x;
    }
    int mine = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int incl = wave_incl_scan_dpp(x == k ? n : 0);
      if (x == k) mine = incl - n;
      if (lane == 63) wsum[wave][k] = incl;
    }
    __syncthreads();
    if (n) {
      int o = base[x] + mine;
      for (int w = 0; w < wave; ++w) o += wsum[w][x];
      s_first[s] = o;
    }
    __syncthreads();
    if (threadIdx.x < 8) {
      int t = 0;
      for (int w = 0; w < 16; ++w) t += wsum[w][threadIdx.x];
      base[threadIdx.x] += t;
    }
    __syncthreads();
  }
  // expansion: one thread per source writes its items
  for (int s = threadIdx.x; s < nsrc; s += 1024) {
    const ItemSource si = item_source(rev_counts, s_order, s, nloc, hkv, C, Qc, QT);
    if (!si.n) continue;
    int64_t f0 = s_first[s];
    int64_t rel = 0;
    int ent = 0, row = 0, nk = 0;
    if (si.c >= 0) {
      nk = nvis[si.h * C + si.c];
      ent = rev_indptr[si.h * C + si.c];
      row = indptr[si.h * (C + 1) + si.c];
    }
    for (int j = 0; j < si.n; ++j, ++rel) {
      const int64_t pos = f0 + rel;
      if (pos >= cap) break;
      const int qb = si.c >= 0 ? j * QT : si.qb;
      const int qn = si.c >= 0 ? min(QT, si.qn - qb) : si.qn;
      PrefillItem it{si.h, si.c, qb, qn, 0, 0, 0, 0};
      if (si.c >= 0) {
        it.nkeys = nk;
        it.entry0 = ent + qb;
        it.row0 = row;
      }
      items[pos] = it;
    }
  }
}


}  // namespace

// One instantiation per bound on the clusters a lane holds (C <= 64 NK).
template <int D, int NK>
int launch_select_nk(const SelectArgs& a, dim3 grid, size_t lds, int R, hipStream_t stream) {
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute((const void*)score_select_kernel<D, NK>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return SBSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((score_select_kernel<D, NK>), grid, dim3(256), lds, stream, a, R);
  return SBSA_OK;
}
template <int D>
int launch_select(const SelectArgs& a, dim3 grid, size_t lds, int R, hipStream_t stream) {
  const int nk = a.C / 64;
  if (nk <= 1) return launch_select_nk<D, 1>(a, grid, lds, R, stream);
  if (nk <= 2) return launch_select_nk<D, 2>(a, grid, lds, R, stream);
  if (nk <= 4) return launch_select_nk<D, 4>(a, grid, lds, R, stream);
  return launch_select_nk<D, 16>(a, grid, lds, R, stream);
}

extern "C" {

int sbsa_score_select(const void* vectors, int64_t v_sq, int64_t v_sh, const float* logmix,
                      const void* codebooks, const int32_t* sizes, int64_t s_nb, int64_t s_h,
                      int num_queries, int num_q_heads, int num_kv_heads, int num_clusters,
                      int dim, int g_union, float inv_temperature, float beta,
                      float target_tokens, int iters, int sink_tokens, int32_t* bitmask,
                      int32_t* qmask, int32_t* counts, int32_t* tokens, float* prob_out,
                      float* theta_out, hipStream_t stream) {
  if (!vectors || !codebooks || !sizes || num_queries < 0 || num_kv_heads < 1) return SBSA_ERR_ARG;
  if (num_q_heads % num_kv_heads || g_union < 1 || iters < 0) return SBSA_ERR_ARG;
  if (v_sh % 8 || v_sq % 8) return SBSA_ERR_ARG;
  const int G = num_q_heads / num_kv_heads;
  const int C = num_clusters;
  if (C % 64 || C > 1024 || C < 64) return SBSA_ERR_UNSUPPORTED;
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) return SBSA_ERR_UNSUPPORTED;
  if (num_queries == 0) return SBSA_OK;
  // rows (query, component) per block: 32 keep a block's LDS near 50 KB at
  // C <= 256, so three blocks share a CU and hide each other's reduction
  // chains (C = 256, 8192 queries: 373 us with 64 rows, 173 us with 32, 205 with 16)
  int R = (C <= 256) ? 32 : (C <= 512 ? 32 : 16);
  if (R < G) R = G;
  if (R % 16) R = 16;
  SelectArgs a;
  a.vectors = (const bf16_t*)vectors;
  a.v_sq = v_sq;
  a.v_sh = v_sh;
  a.logmix = logmix;
  a.codebooks = (const bf16_t*)codebooks;
  a.sizes = sizes;
  a.s_nb = s_nb;
  a.s_h = s_h;
  a.bitmask = bitmask;
  a.qmask = qmask;
  a.counts = counts;
  a.tokens = tokens;
  a.prob_out = prob_out;
  a.theta_out = theta_out;
  a.Q = num_queries;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.C = C;
  a.G = G;
  a.g_union = g_union;
  a.iters = iters;
  a.sink = sink_tokens;
  a.inv_temp = inv_temperature;
  a.beta = beta;
  a.target = target_tokens;
  const int QT = R / G;
  dim3 grid((num_queries + QT - 1) / QT, num_kv_heads);
  size_t lds = (size_t)R * (dim + 8) * 2 + (size_t)R * (C + 1) * 4;
  if (lds > 160 * 1024) return SBSA_ERR_UNSUPPORTED;
  int rc = SBSA_ERR_UNSUPPORTED;
  switch (dim) {
    case 64: rc = launch_select<64>(a, grid, lds, R, stream); break;
    case 128: rc = launch_select<128>(a, grid, lds, R, stream); break;
    case 256: rc = launch_select<256>(a, grid, lds, R, stream); break;
    default: break;
  }
  if (rc) return rc;
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_causal_sizes(const int32_t* posting, int64_t width, const int32_t* indptr,
                      const int32_t* sizes, int num_kv_heads, int num_clusters,
                      int64_t pos_limit, int32_t* out, hipStream_t stream) {
  if (!posting || !indptr || !sizes || !out || num_kv_heads < 1 || num_clusters < 1) return SBSA_ERR_ARG;
  int n = num_kv_heads * num_clusters;
  hipLaunchKernelGGL(causal_sizes_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, posting,
                     width, indptr, sizes, num_kv_heads, num_clusters, pos_limit, out);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_reverse_index(const int32_t* qmask, int num_queries, int num_kv_heads, int num_clusters,
                       const int32_t* nvis, int32_t* rev_counts, int32_t* rev_indptr,
                       int64_t* nnz, int32_t* qvals, int64_t qvals_cap, int32_t* qrank,
                       hipStream_t stream) {
  if (!qmask || !nvis || !rev_counts || !rev_indptr || !nnz || !qvals || !qrank) return SBSA_ERR_ARG;
  if (num_clusters % 32 || num_clusters < 32 || num_queries < 0) return SBSA_ERR_ARG;
  int64_t bound = (int64_t)num_queries * num_kv_heads * num_clusters;
  if (qvals_cap < bound) return SBSA_ERR_CAPACITY;
  int n = num_kv_heads * num_clusters;
  hipLaunchKernelGGL(rev_pass_kernel, dim3(n), dim3(256), 0, stream, 0, qmask, num_queries,
                     num_kv_heads, num_clusters, nvis, rev_counts, rev_indptr, qvals, qrank);
  hipLaunchKernelGGL(rev_scan_kernel, dim3(1), dim3(1024), 0, stream, rev_counts, n, rev_indptr, nnz);
  hipLaunchKernelGGL(rev_pass_kernel, dim3(n), dim3(256), 0, stream, 1, qmask, num_queries,
                     num_kv_heads, num_clusters, nvis, rev_counts, rev_indptr, qvals, qrank);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int64_t sbsa_prefill_items_bound(int64_t nnz, int num_queries, int num_kv_heads, int num_clusters,
                                 int queries_per_item) {
  int64_t qt = queries_per_item;
  return (int64_t)num_kv_heads * ((num_queries + qt - 1) / qt) +
         (int64_t)num_kv_heads * num_clusters + (nnz + qt - 1) / qt;
}

int sbsa_prefill_items(const int32_t* rev_counts, int num_kv_heads, int num_clusters,
                       int num_queries, int queries_per_item, int has_local,
                       const int32_t* indptr, const int32_t* nvis, const int32_t* rev_indptr,
                       void* items, int64_t items_cap, int64_t partials_cap, int32_t* queue,
                       hipStream_t stream) {
  if (!rev_counts || !items || !queue || queries_per_item < 1) return SBSA_ERR_ARG;
  if (!indptr || !nvis || !rev_indptr) return SBSA_ERR_ARG;
  const int nloc = has_local ? (num_queries + queries_per_item - 1) / queries_per_item : 0;
  const size_t lds = (size_t)(nloc * num_kv_heads + 3 * num_kv_heads * num_clusters) * 4;
  if (lds > 150 * 1024) return SBSA_ERR_UNSUPPORTED;
  static size_t configured = 0;
  if (lds > configured) {
    if (hipFuncSetAttribute((const void*)build_items_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return SBSA_ERR_UNSUPPORTED;
    configured = lds;
  }
  hipLaunchKernelGGL(build_items_kernel, dim3(1), dim3(1024), lds, stream, rev_counts, num_kv_heads,
                     num_clusters, num_queries, queries_per_item, has_local, indptr, nvis, rev_indptr,
                     (PrefillItem*)items, queue,
                     items_cap, partials_cap);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

}  // extern "C"
