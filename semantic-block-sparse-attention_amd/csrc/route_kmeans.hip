// S0 routing normalisation and S1 block build (spherical k-means, bucket
// layout, packed K/V) for gfx950.
//
// Reference behaviour (pfnet-research/semantic-block-sparse-attention):
//   trivial_router.py:48-75        query routing vectors
//   routing_map.py:35-64           key router, whole-vector mode
//   flat_index.py:144-166, 300-302 routing space / fit space
//   flat_index.py:193-289          fit_flat_codebook (random init, cosine)
//   flat_index.py:356-383          bf16 argmax assignment
//   state.py:545-948               ProductPostingIndex._build_flat
//   state.py:44-84                 page-aligned bucket order
//   state.py:950-997               pack_prompt_kv
#include "sbsa_common.h"

namespace {

// ---------------------------------------------------------------- S0 -------
// One wave per row: normalise in fp32, round to bf16, renormalise, round.
// F.normalize divides by max(norm, 1e-12).
__global__ void route_vectors_kernel(const bf16_t* __restrict__ x, int64_t rows, int64_t ld_x,
                                     int dim, int factors, bf16_t* __restrict__ out,
                                     int64_t ld_out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int part = dim / factors;
  const bf16_t* src = x + row * ld_x;
  bf16_t* dst = out + row * ld_out;
  for (int f = 0; f < factors; ++f) {
    float v[8];
    const int per = (part + 63) / 64;  // <= 8 for dim <= 512
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int d = lane + i * 64;
      v[i] = (i < per && d < part) ? bf2f(src[f * part + d]) : 0.f;
      ss += v[i] * v[i];
    }
    float n1 = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
    float ss2 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[i] = round_bf16(v[i] / n1);
      ss2 += v[i] * v[i];
    }
    float n2 = fmaxf(sqrtf(wave_sum(ss2)), 1e-12f);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int d = lane + i * 64;
      if (i < per && d < part) dst[f * part + d] = f2bf(v[i] / n2);
    }
  }
}

// ---------------------------------------------------------------- S1 -------
// Key routing space of one KV head: p = bf16(normalize(k)) (the key router,
// skipped when the input already is its output), s1 = normalize(p)
// (routing_space), s2 = normalize(s1) (the fit space the k-means and the
// assignment work in).  Writes s2 in fp32 and in bf16.
__global__ void key_space_kernel(const bf16_t* __restrict__ k, int64_t length, int64_t ld_k,
                                 int dim, int router_pass, float* __restrict__ space_f32,
                                 bf16_t* __restrict__ space_bf16) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= length) return;
  const int per = (dim + 63) / 64;
  float v[8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int d = lane + i * 64;
    v[i] = (i < per && d < dim) ? bf2f(k[row * ld_k + d]) : 0.f;
    ss += v[i] * v[i];
  }
  if (router_pass) {
    float n0 = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
    ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[i] = round_bf16(v[i] / n0);
      ss += v[i] * v[i];
    }
  }
  float n1 = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
  ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = v[i] / n1;
    ss += v[i] * v[i];
  }
  float n2 = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int d = lane + i * 64;
    if (i < per && d < dim) {
      float s = v[i] / n2;
      space_f32[row * dim + d] = s;
      space_bf16[row * dim + d] = f2bf(s);
    }
  }
}

// Argmax over centroids of round_bf16(x . c) with fp32 accumulation: the bf16
// GEMM of flat_index.py:369 returns bf16 similarities, and torch.argmax takes
// the first of equal maxima.
//
// Block: 4 waves, 32 rows per wave (two 16-row MFMA blocks).  Centroids are
// staged through LDS 64 at a time; rows stay in registers (A operand).
template <int D>
__global__ __launch_bounds__(256) void kmeans_assign_kernel(
    const bf16_t* __restrict__ x, int64_t ld_x, const int32_t* __restrict__ row_index, int64_t n,
    const bf16_t* __restrict__ cent, int num_clusters, int32_t* __restrict__ assign) {
  constexpr int KS = D / 32;           // k-steps of 32
  constexpr int LDR = D + 8;           // padded LDS row (bf16 elements)
  __shared__ __attribute__((aligned(16))) bf16_t sc[64 * LDR];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * 128 + wave * 32;

  // A operands: rows rb*16 + lane%16, k = s*32 + (lane/16)*8 .. +8
  u32x4_t a[2][KS];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    int64_t r = row0 + rb * 16 + (lane & 15);
    bool ok = r < n;
    int64_t src = ok ? (row_index ? (int64_t)row_index[r] : r) : 0;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (ok)
        a[rb][s] = *reinterpret_cast<const u32x4_t*>(x + src * ld_x + s * 32 + (lane >> 4) * 8);
      else
        a[rb][s] = u32x4_t{0, 0, 0, 0};
    }
  }
  // running best per (rb, i): rows rb*16 + (lane/16)*4 + i
  float best[2][4];
  int bidx[2][4];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      best[rb][i] = -INFINITY;
      bidx[rb][i] = 0;
    }

  for (int c0 = 0; c0 < num_clusters; c0 += 64) {
    __syncthreads();
    // stage 64 centroids: 64 rows x D bf16
    for (int e = threadIdx.x; e < 64 * (D / 8); e += 256) {
      int r = e / (D / 8), ch = e % (D / 8);
      u32x4_t v = u32x4_t{0, 0, 0, 0};
      if (c0 + r < num_clusters) v = *reinterpret_cast<const u32x4_t*>(cent + (int64_t)(c0 + r) * D + ch * 8);
      *reinterpret_cast<u32x4_t*>(&sc[r * LDR + ch * 8]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      f32x4_t acc[2] = {f32x4_t{0, 0, 0, 0}, f32x4_t{0, 0, 0, 0}};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        u32x4_t b = *reinterpret_cast<const u32x4_t*>(&sc[(cb * 16 + (lane & 15)) * LDR + s * 32 + (lane >> 4) * 8]);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) acc[rb] = mfma16x16x32(as_bf16x8(a[rb][s]), as_bf16x8(b), acc[rb]);
      }
      const int col = c0 + cb * 16 + (lane & 15);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = (col < num_clusters) ? round_bf16(acc[rb][i]) : -INFINITY;
          // within a lane columns increase with cb: strict > keeps the first
          if (v > best[rb][i]) {
            best[rb][i] = v;
            bidx[rb][i] = col;
          }
        }
    }
  }
  // reduce over the 16 lanes of each group (different columns)
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = best[rb][i];
      int ix = bidx[rb][i];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        float ov = __shfl_xor(v, o, 64);
        int oi = __shfl_xor(ix, o, 64);
        if (ov > v || (ov == v && oi < ix)) {
          v = ov;
          ix = oi;
        }
      }
      int64_t r = row0 + rb * 16 + (lane >> 4) * 4 + i;
      if ((lane & 15) == 0 && r < n) assign[r] = ix;
    }
}

// Per-cluster fp32 sums of the member rows, in row order (deterministic), in
// two launches whose traffic grows with the rows, not with rows x clusters.
//
// kmeans_members_kernel writes one bitmap row per cluster: bit i of bits[c] is
// set iff assign[i] == c.  A block takes 512 rows (16 words of 32 bits), ORs
// their bits into an LDS table [C][16] (the OR commutes, so the result does not
// depend on the order of the LDS atomics) and writes the whole table out, zero
// words included, as 64-byte pieces of each cluster's row: no state is kept
// from call to call.  Words per cluster W = ceil(n / 512) * 16.
constexpr int KB_ROWS = 512;
constexpr int KB_WORDS = KB_ROWS / 32;

__global__ __launch_bounds__(256) void kmeans_members_kernel(const int32_t* __restrict__ assign,
                                                              int64_t n, int num_clusters,
                                                              int64_t words, uint32_t* __restrict__ bits) {
  extern __shared__ u32x4_t tab4[];          // [C][16] words as [C][4] 16-byte pieces
  uint32_t* tab = reinterpret_cast<uint32_t*>(tab4);
  const int64_t r0 = (int64_t)blockIdx.x * KB_ROWS;
  int a[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int64_t i = r0 + threadIdx.x + 256 * k;
    a[k] = i < n ? assign[i] : -1;
  }
  for (int i = threadIdx.x; i < num_clusters * 4; i += 256) tab4[i] = u32x4_t{0u, 0u, 0u, 0u};
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int local = threadIdx.x + 256 * k;
    if ((unsigned)a[k] < (unsigned)num_clusters)
      atomicOr(&tab[a[k] * KB_WORDS + (local >> 5)], 1u << (local & 31));
  }
  __syncthreads();
  u32x4_t* out = reinterpret_cast<u32x4_t*>(bits);
  for (int i = threadIdx.x; i < num_clusters * 4; i += 256) {
    const int c = i >> 2, q = i & 3;
    out[((int64_t)c * words + (int64_t)blockIdx.x * KB_WORDS) / 4 + q] = tab4[i];
  }
}

// kmeans_update_kernel: one block per cluster reads its bitmap row, 4 words a
// thread per segment of 1024 words (32768 rows).  A block-wide prefix sum of the
// threads' bit counts places each member at its rank in an LDS list, so the list
// holds the cluster's rows in row order; the list is mapped through the row map
// in one pass.  Wave w then adds list entries w, w+4, w+8, ... (4 dims a lane,
// 16-byte loads), the loads of KU_BATCH entries issued before any of them is
// added, so one round trip covers 4 * KU_BATCH rows.  A segment with more members
// than the list holds is taken in windows.  The four waves' sums are added in
// wave order at the end: the result depends on the assignment only.
constexpr int KU_LIST = 8192;
constexpr int KU_SEG = 1024;     // words per segment, 4 a thread
constexpr int KU_BATCH = 16;     // entries per wave per round trip

template <int NJ>  // dims 4*lane + 256*j .. +3 for j < NJ
__global__ __launch_bounds__(256) void kmeans_update_kernel(
    const float* __restrict__ x, int64_t ld_x, const int32_t* __restrict__ row_index,
    const uint32_t* __restrict__ bits, int64_t words, int dim, float* __restrict__ sums,
    int32_t* __restrict__ counts) {
  __shared__ int members[KU_LIST];
  __shared__ __attribute__((aligned(16))) float red[4][256 * NJ];
  __shared__ int wsum[4];
  const int c = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const uint32_t* row = bits + (int64_t)c * words;
  f32x4_t acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int total = 0;
  for (int64_t w0 = 0; w0 < words; w0 += KU_SEG) {
    u32x4_t q = {0u, 0u, 0u, 0u};
    const int64_t w = w0 + 4 * t;
    if (w < words) q = *reinterpret_cast<const u32x4_t*>(row + w);   // words is a multiple of 16
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const int cnt = __builtin_popcount(q.x) + __builtin_popcount(q.y) + __builtin_popcount(q.z) +
                    __builtin_popcount(q.w);
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int excl = incl - cnt;
    for (int v = 0; v < wave; ++v) excl += wsum[v];
    const int seg_total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    for (int lo = 0; lo < seg_total; lo += KU_LIST) {
      if (excl < lo + KU_LIST && excl + cnt > lo) {
        int pos = excl;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t m = qw[k];
          while (m) {
            const int bit = __builtin_ctz(m);
            m &= m - 1;
            if (pos >= lo && pos < lo + KU_LIST) members[pos - lo] = (int)((w + k) * 32 + bit);
            ++pos;
          }
        }
      }
      __syncthreads();
      const int listed = min(KU_LIST, seg_total - lo);
      if (row_index) {
        for (int i = t; i < listed; i += 256) members[i] = row_index[members[i]];
        __syncthreads();
      }
      for (int m = wave; m < listed; m += 4 * KU_BATCH) {
        f32x4_t v[KU_BATCH][NJ];
#pragma unroll
        for (int u = 0; u < KU_BATCH; ++u) {
          const bool ok = m + 4 * u < listed;
          const int64_t src = ok ? members[m + 4 * u] : 0;
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int d = 4 * lane + 256 * j;
            v[u][j] = (ok && d < dim) ? *reinterpret_cast<const f32x4_t*>(x + src * ld_x + d)
                                      : f32x4_t{0.f, 0.f, 0.f, 0.f};
          }
        }
#pragma unroll
        for (int u = 0; u < KU_BATCH; ++u)
          if (m + 4 * u < listed)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[j] += v[u][j];
      }
      __syncthreads();  // the list is free for the next window
    }
    total += seg_total;
    __syncthreads();    // wsum may be rewritten
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    *reinterpret_cast<f32x4_t*>(&red[wave][4 * lane + 256 * j]) = acc[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = t + 256 * j;
    if (d < dim) sums[(int64_t)c * dim + d] = ((red[0][d] + red[1][d]) + red[2][d]) + red[3][d];
  }
  if (t == 0) counts[c] = total;
}

// Centroid step, one wave per cluster.
//  mode 0 (init):       cent = x[row_index[src[c]]]                  flat_index.py:260-262
//  mode 1 (update):     cent = normalize(sums / counts), an empty cluster
//                       (src[c] >= 0) restarts on sample row src[c]  flat_index.py:277-288
//  mode 2 (descriptor): out = bf16(normalize(sums)) as [2, C, dim/2] state.py:883-886
//  mode 3 (update with restarts drawn ahead): mode 1, where the empty clusters
//                       of the k-th iteration that has any (k < draws) restart
//                       on the sample rows src[k * C + rank], rank counting the
//                       empty clusters in cluster order (src holds the restart
//                       draws, made ahead).  flags[0] = k, the number of earlier
//                       iterations with an empty cluster; block 0 writes
//                       flags[1] = k + (this iteration has one), for the next
//                       iteration's launch.
__global__ void kmeans_centroids_kernel(int mode, const float* __restrict__ sums,
                                        const int32_t* __restrict__ counts,
                                        const int32_t* __restrict__ src,
                                        const float* __restrict__ x, int64_t ld_x,
                                        const int32_t* __restrict__ row_index, int num_clusters,
                                        int dim, float* __restrict__ cent_f32,
                                        bf16_t* __restrict__ cent_bf16, int32_t* flags,
                                        int draws) {
  const int lane = threadIdx.x & 63;
  const int c = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const bool update = mode == 1 || mode == 3;
  int used = 0;
  if (mode == 3) {
    used = flags[0];
    if (blockIdx.x == 0 && threadIdx.x < 64) {
      int any = 0;
      for (int i = lane; i < num_clusters; i += 64) any |= counts[i] == 0;
      any = __ballot(any) != 0ull;
      if (lane == 0) flags[1] = used + any;
    }
  }
  if (c >= num_clusters) return;
  const int per = (dim + 63) / 64;
  float v[16];
  int64_t r = -1;
  if (mode == 0 || mode == 1) {
    r = src[c];
  } else if (mode == 3 && used < draws && counts[c] == 0) {
    int rank = 0;
    for (int b = 0; b < c; b += 64) rank += __popcll(__ballot(b + lane < c && counts[b + lane] == 0));
    r = src[(int64_t)used * num_clusters + rank];
  }
  if (r >= 0) {
    int64_t srow = row_index ? (int64_t)row_index[r] : r;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int d = lane + 64 * i;
      v[i] = (i < per && d < dim) ? x[srow * ld_x + d] : 0.f;
    }
  } else {
    float cnt = update ? (float)counts[c] : 1.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int d = lane + 64 * i;
      float s = (i < per && d < dim) ? sums[(int64_t)c * dim + d] : 0.f;
      v[i] = update ? s / cnt : s;
    }
  }
  if (mode != 0) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ss += v[i] * v[i];
    float nrm = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = v[i] / nrm;
  }
  const int half = dim / 2;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int d = lane + 64 * i;
    if (i < per && d < dim) {
      if (mode == 2) {
        int part = d / half;
        cent_bf16[((int64_t)part * num_clusters + c) * half + (d - part * half)] = f2bf(v[i]);
      } else {
        cent_f32[(int64_t)c * dim + d] = v[i];
        cent_bf16[(int64_t)c * dim + d] = f2bf(v[i]);
      }
    }
  }
}

// ------------------------------------------------------- bucket layout -----
// Stable counting sort of positions by cluster with page-aligned runs.
constexpr int LAYOUT_CHUNK = 1024;

__global__ __launch_bounds__(256) void layout_hist_kernel(const int32_t* __restrict__ assign,
                                                          int64_t length, int num_clusters,
                                                          int32_t* __restrict__ chunk_counts) {
  extern __shared__ int cnt[];
  for (int c = threadIdx.x; c < num_clusters; c += 256) cnt[c] = 0;
  __syncthreads();
  int64_t base = (int64_t)blockIdx.x * LAYOUT_CHUNK;
  for (int j = threadIdx.x; j < LAYOUT_CHUNK; j += 256) {
    int64_t p = base + j;
    if (p < length) atomicAdd(&cnt[assign[p]], 1);
  }
  __syncthreads();
  for (int c = threadIdx.x; c < num_clusters; c += 256)
    chunk_counts[(int64_t)blockIdx.x * num_clusters + c] = cnt[c];
}

// One block: sizes, padded exclusive scan (indptr), per-chunk bases, first
// non-empty cluster.  num_clusters <= 1024.
__global__ __launch_bounds__(1024) void layout_scan_kernel(int32_t* __restrict__ chunk_counts,
                                                           int nchunks, int num_clusters,
                                                           int align, int32_t* __restrict__ sizes,
                                                           int32_t* __restrict__ indptr,
                                                           int32_t* __restrict__ total_out,
                                                           int32_t* __restrict__ first_cluster) {
  __shared__ int wsum[16];
  __shared__ int s_first;
  const int c = threadIdx.x;
  const int lane = c & 63, wave = c >> 6;
  int size = 0;
  if (c < num_clusters)
    for (int k = 0; k < nchunks; ++k) size += chunk_counts[(int64_t)k * num_clusters + c];
  int padded = (c < num_clusters) ? ((size + align - 1) / align) * align : 0;
  int incl = wave_incl_scan(padded);
  if (lane == 63) wsum[wave] = incl;
  if (c == 0) s_first = 0x7fffffff;
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; ++w) off += wsum[w];
  int excl = off + incl - padded;
  if (c < num_clusters) {
    sizes[c] = size;
    indptr[c] = excl;
    if (size > 0) atomicMin(&s_first, c);
    int run = excl;
    for (int k = 0; k < nchunks; ++k) {
      int64_t at = (int64_t)k * num_clusters + c;
      int v = chunk_counts[at];
      chunk_counts[at] = run;
      run += v;
    }
  }
  if (c == num_clusters - 1) {
    indptr[num_clusters] = excl + padded;
    *total_out = excl + padded;
  }
  __syncthreads();
  if (c == 0) *first_cluster = s_first;
}

// Scatter: each position goes to its cluster's next row, in position order.
__global__ __launch_bounds__(256) void layout_scatter_kernel(const int32_t* __restrict__ assign,
                                                             int64_t length, int num_clusters,
                                                             const int32_t* __restrict__ chunk_base,
                                                             int32_t* __restrict__ posting,
                                                             int32_t* __restrict__ inverse) {
  extern __shared__ int next[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int c = threadIdx.x; c < num_clusters; c += 256)
    next[c] = chunk_base[(int64_t)blockIdx.x * num_clusters + c];
  __syncthreads();
  int64_t base = (int64_t)blockIdx.x * LAYOUT_CHUNK;
  for (int round = 0; round < LAYOUT_CHUNK / 256; ++round) {
    int64_t p = base + round * 256 + threadIdx.x;
    int a = (p < length) ? assign[p] : -1;
    // earlier lanes of this wave with the same cluster, and whether this lane
    // is the last of its cluster in the wave
    int before = 0, after = 0;
    for (int j = 0; j < 64; ++j) {
      int o = __shfl(a, j, 64);
      before += (j < lane && o == a) ? 1 : 0;
      after += (j > lane && o == a) ? 1 : 0;
    }
    for (int w = 0; w < 4; ++w) {
      if (wave == w && a >= 0) {
        int row = next[a] + before;
        posting[row] = (int32_t)p;
        inverse[p] = row;
      }
      __syncthreads();
      if (wave == w && a >= 0 && after == 0) next[a] += before + 1;
      __syncthreads();
    }
  }
}

// Padding rows repeat the first sorted key's position (state.py:73 and 906-913).
__global__ void layout_pad_kernel(const int32_t* __restrict__ sizes,
                                  const int32_t* __restrict__ indptr, int num_clusters,
                                  const int32_t* __restrict__ first_cluster,
                                  int32_t* __restrict__ posting, int64_t posting_cap) {
  const int fc = *first_cluster;
  const int32_t first_pos = posting[indptr[fc]];
  if ((int)blockIdx.x < num_clusters) {
    int c = blockIdx.x;
    int lo = indptr[c] + sizes[c], hi = indptr[c + 1];
    for (int r = lo + threadIdx.x; r < hi; r += blockDim.x) posting[r] = first_pos;
  } else {
    int64_t total = indptr[num_clusters];
    int64_t stride = (int64_t)(gridDim.x - num_clusters) * blockDim.x;
    for (int64_t r = total + (int64_t)(blockIdx.x - num_clusters) * blockDim.x + threadIdx.x;
         r < posting_cap; r += stride)
      posting[r] = first_pos;
  }
}

// packed[t][r][h][:] = (t ? v : k)[posting[h][r]][h][:]; rows >= width are zero.
__global__ void pack_kv_kernel(const bf16_t* __restrict__ key, const bf16_t* __restrict__ value,
                               int64_t stride_tok, int64_t stride_head, int num_kv_heads, int dim,
                               const int32_t* __restrict__ posting, int64_t width,
                               int64_t packed_len, bf16_t* __restrict__ packed) {
  const int chunks = dim / 8;
  const int64_t per_plane = packed_len * num_kv_heads * chunks;
  const int64_t total = 2 * per_plane;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t t = e / per_plane;
    int64_t rem = e - t * per_plane;
    int64_t r = rem / (num_kv_heads * chunks);
    int64_t hc = rem - r * (num_kv_heads * chunks);
    int h = (int)(hc / chunks);
    int ch = (int)(hc - (int64_t)h * chunks);
    u32x4_t v = u32x4_t{0, 0, 0, 0};
    if (r < width) {
      int64_t pos = posting[(int64_t)h * width + r];
      const bf16_t* src = (t ? value : key) + pos * stride_tok + (int64_t)h * stride_head + ch * 8;
      v = *reinterpret_cast<const u32x4_t*>(src);
    }
    *reinterpret_cast<u32x4_t*>(packed + ((t * packed_len + r) * num_kv_heads + h) * dim + ch * 8) = v;
  }
}

// Vectorised forms of the two kernels above for rows of 64..512 elements with
// 16-byte-aligned rows: each lane owns 8 consecutive elements (one 16-byte
// load), LPR = dim / 8 lanes hold a row, and a norm is reduced over the
// lanes of its row (or of its factor's part).
template <int LPR>
__device__ __forceinline__ float row_sum(float v, int group) {
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1)
    if (o < group) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ void unpack8(u32x4_t w, float (&v)[8]) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float(ww[j] << 16);
    v[2 * j + 1] = __uint_as_float(ww[j] & 0xffff0000u);
  }
}

template <int LPR>
__global__ __launch_bounds__(256) void route_vectors_vec_kernel(const bf16_t* __restrict__ x, int64_t rows,
                                                                int64_t ld_x, int factors,
                                                                bf16_t* __restrict__ out, int64_t ld_out) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
  const int sub = lane % LPR;
  const int group = LPR / factors;            // lanes of one factor's part
  const bool ok = row < rows;
  float v[8];
  unpack8(ok ? *reinterpret_cast<const u32x4_t*>(x + row * ld_x + sub * 8) : u32x4_t{0, 0, 0, 0}, v);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  const float n1 = fmaxf(sqrtf(row_sum<LPR>(ss, group)), 1e-12f);
  float ss2 = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v[e] = round_bf16(v[e] / n1);
    ss2 += v[e] * v[e];
  }
  const float n2 = fmaxf(sqrtf(row_sum<LPR>(ss2, group)), 1e-12f);
  if (ok) {
    u32x4_t w;
    w.x = pack2bf(v[0] / n2, v[1] / n2);
    w.y = pack2bf(v[2] / n2, v[3] / n2);
    w.z = pack2bf(v[4] / n2, v[5] / n2);
    w.w = pack2bf(v[6] / n2, v[7] / n2);
    *reinterpret_cast<u32x4_t*>(out + row * ld_out + sub * 8) = w;
  }
}

template <int LPR>
__global__ __launch_bounds__(256) void key_space_vec_kernel(const bf16_t* __restrict__ k, int64_t length,
                                                            int64_t ld_k, int router_pass,
                                                            float* __restrict__ space_f32,
                                                            bf16_t* __restrict__ space_bf16) {
  constexpr int RPW = 64 / LPR;
  constexpr int D = LPR * 8;
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
  const int sub = lane % LPR;
  const bool ok = row < length;
  float v[8];
  unpack8(ok ? *reinterpret_cast<const u32x4_t*>(k + row * ld_k + sub * 8) : u32x4_t{0, 0, 0, 0}, v);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  if (router_pass) {
    const float n0 = fmaxf(sqrtf(row_sum<LPR>(ss, LPR)), 1e-12f);
    ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = round_bf16(v[e] / n0);
      ss += v[e] * v[e];
    }
  }
  const float n1 = fmaxf(sqrtf(row_sum<LPR>(ss, LPR)), 1e-12f);
  ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v[e] = v[e] / n1;
    ss += v[e] * v[e];
  }
  const float n2 = fmaxf(sqrtf(row_sum<LPR>(ss, LPR)), 1e-12f);
  if (ok) {
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = v[e] / n2;
    float* df = space_f32 + row * D + sub * 8;
    *reinterpret_cast<f32x4_t*>(df) = f32x4_t{s[0], s[1], s[2], s[3]};
    *reinterpret_cast<f32x4_t*>(df + 4) = f32x4_t{s[4], s[5], s[6], s[7]};
    *reinterpret_cast<u32x4_t*>(space_bf16 + row * D + sub * 8) =
        u32x4_t{pack2bf(s[0], s[1]), pack2bf(s[2], s[3]), pack2bf(s[4], s[5]), pack2bf(s[6], s[7])};
  }
}

bool vec_rows_ok(const void* p, int64_t ld, int dim) {
  return ((uintptr_t)p & 15) == 0 && ld % 8 == 0 && (dim == 64 || dim == 128 || dim == 256 || dim == 512);
}

}  // namespace

extern "C" {

int sbsa_route_vectors(const void* x, int64_t rows, int64_t ld_x, int dim, int factors, void* out,
                       int64_t ld_out, hipStream_t stream) {
  if (!x || !out || rows < 0 || factors < 1 || dim % factors || dim / factors > 512 || dim < 1)
    return SBSA_ERR_ARG;
  if (rows == 0) return SBSA_OK;
  const int lpr = dim / 8;
  if (vec_rows_ok(x, ld_x, dim) && vec_rows_ok(out, ld_out, dim) && lpr % factors == 0 &&
      (dim / factors) % 8 == 0) {
    const int64_t per_block = 4 * (64 / lpr);
    const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
    switch (lpr) {
      case 8: hipLaunchKernelGGL(route_vectors_vec_kernel<8>, grid, dim3(256), 0, stream, (const bf16_t*)x, rows, ld_x, factors, (bf16_t*)out, ld_out); break;
      case 16: hipLaunchKernelGGL(route_vectors_vec_kernel<16>, grid, dim3(256), 0, stream, (const bf16_t*)x, rows, ld_x, factors, (bf16_t*)out, ld_out); break;
      case 32: hipLaunchKernelGGL(route_vectors_vec_kernel<32>, grid, dim3(256), 0, stream, (const bf16_t*)x, rows, ld_x, factors, (bf16_t*)out, ld_out); break;
      default: hipLaunchKernelGGL(route_vectors_vec_kernel<64>, grid, dim3(256), 0, stream, (const bf16_t*)x, rows, ld_x, factors, (bf16_t*)out, ld_out); break;
    }
    SBSA_CHECK_LAUNCH();
    return SBSA_OK;
  }
  int blocks = (int)((rows + 3) / 4);
  hipLaunchKernelGGL(route_vectors_kernel, dim3(blocks), dim3(256), 0, stream,
                     (const bf16_t*)x, rows, ld_x, dim, factors, (bf16_t*)out, ld_out);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_key_space(const void* k, int64_t length, int64_t ld_k, int dim, int router_pass,
                   float* space_f32, void* space_bf16, hipStream_t stream) {
  if (!k || !space_f32 || !space_bf16 || length < 0 || dim < 1 || dim > 512) return SBSA_ERR_ARG;
  if (length == 0) return SBSA_OK;
  if (vec_rows_ok(k, ld_k, dim) && ((uintptr_t)space_f32 & 15) == 0 && ((uintptr_t)space_bf16 & 15) == 0) {
    const int lpr = dim / 8;
    const int64_t per_block = 4 * (64 / lpr);
    const dim3 grid((unsigned)((length + per_block - 1) / per_block));
    switch (lpr) {
      case 8: hipLaunchKernelGGL(key_space_vec_kernel<8>, grid, dim3(256), 0, stream, (const bf16_t*)k, length, ld_k, router_pass, space_f32, (bf16_t*)space_bf16); break;
      case 16: hipLaunchKernelGGL(key_space_vec_kernel<16>, grid, dim3(256), 0, stream, (const bf16_t*)k, length, ld_k, router_pass, space_f32, (bf16_t*)space_bf16); break;
      case 32: hipLaunchKernelGGL(key_space_vec_kernel<32>, grid, dim3(256), 0, stream, (const bf16_t*)k, length, ld_k, router_pass, space_f32, (bf16_t*)space_bf16); break;
      default: hipLaunchKernelGGL(key_space_vec_kernel<64>, grid, dim3(256), 0, stream, (const bf16_t*)k, length, ld_k, router_pass, space_f32, (bf16_t*)space_bf16); break;
    }
    SBSA_CHECK_LAUNCH();
    return SBSA_OK;
  }
  hipLaunchKernelGGL(key_space_kernel, dim3((unsigned)((length + 3) / 4)), dim3(256), 0, stream,
                     (const bf16_t*)k, length, ld_k, dim, router_pass, space_f32,
                     (bf16_t*)space_bf16);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_kmeans_assign(const void* x_bf16, int64_t ld_x, const int32_t* row_index, int64_t n,
                       const void* cent_bf16, int num_clusters, int dim, int32_t* assign,
                       hipStream_t stream) {
  if (!x_bf16 || !cent_bf16 || !assign || n < 0 || num_clusters < 1) return SBSA_ERR_ARG;
  if (ld_x % 8) return SBSA_ERR_ARG;
  if (n == 0) return SBSA_OK;
  dim3 grid((unsigned)((n + 127) / 128));
  switch (dim) {
    case 64:
      hipLaunchKernelGGL(kmeans_assign_kernel<64>, grid, dim3(256), 0, stream, (const bf16_t*)x_bf16,
                         ld_x, row_index, n, (const bf16_t*)cent_bf16, num_clusters, assign);
      break;
    case 128:
      hipLaunchKernelGGL(kmeans_assign_kernel<128>, grid, dim3(256), 0, stream,
                         (const bf16_t*)x_bf16, ld_x, row_index, n, (const bf16_t*)cent_bf16,
                         num_clusters, assign);
      break;
    case 256:
      hipLaunchKernelGGL(kmeans_assign_kernel<256>, grid, dim3(256), 0, stream,
                         (const bf16_t*)x_bf16, ld_x, row_index, n, (const bf16_t*)cent_bf16,
                         num_clusters, assign);
      break;
    default:
      return SBSA_ERR_UNSUPPORTED;
  }
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

size_t sbsa_kmeans_member_bits_bytes(int64_t n, int num_clusters) {
  if (n < 0 || num_clusters < 1) return 0;
  const int64_t words = (n + KB_ROWS - 1) / KB_ROWS * KB_WORDS;
  return (size_t)(words * num_clusters) * sizeof(uint32_t);
}

int sbsa_kmeans_update(const float* x, int64_t ld_x, const int32_t* row_index, int64_t n,
                       const int32_t* assign, int num_clusters, int dim, float* sums,
                       int32_t* counts, uint32_t* member_bits, size_t member_bits_bytes,
                       hipStream_t stream) {
  if (!x || !assign || !sums || !counts || !member_bits || n < 0 || num_clusters < 1)
    return SBSA_ERR_ARG;
  if (dim < 4 || dim > 1024 || dim % 4 || ld_x % 4 || ((uintptr_t)x & 15) || num_clusters > 1024)
    return SBSA_ERR_UNSUPPORTED;
  if (member_bits_bytes < sbsa_kmeans_member_bits_bytes(n, num_clusters)) return SBSA_ERR_CAPACITY;
  if (((uintptr_t)member_bits & 15) != 0) return SBSA_ERR_ARG;
  const int64_t words = (n + KB_ROWS - 1) / KB_ROWS * KB_WORDS;
  if (words > 0)
    hipLaunchKernelGGL(kmeans_members_kernel, dim3((unsigned)(words / KB_WORDS)), dim3(256),
                       (size_t)num_clusters * KB_WORDS * sizeof(uint32_t), stream, assign, n,
                       num_clusters, words, member_bits);
  auto kernel = dim <= 256 ? kmeans_update_kernel<1>
                : dim <= 512 ? kmeans_update_kernel<2>
                : dim <= 768 ? kmeans_update_kernel<3> : kmeans_update_kernel<4>;
  hipLaunchKernelGGL(kernel, dim3(num_clusters), dim3(256), 0, stream, x, ld_x, row_index,
                     (const uint32_t*)member_bits, words, dim, sums, counts);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_kmeans_centroids(int mode, const float* sums, const int32_t* counts,
                          const int32_t* src_rows, const float* x, int64_t ld_x,
                          const int32_t* row_index, int num_clusters, int dim, float* cent_f32,
                          void* cent_bf16, hipStream_t stream) {
  if (mode < 0 || mode > 2 || num_clusters < 1 || !cent_bf16) return SBSA_ERR_ARG;
  if (dim < 2 || dim > 1024 || dim % 2) return SBSA_ERR_UNSUPPORTED;
  if (mode == 0 && (!src_rows || !x || !cent_f32)) return SBSA_ERR_ARG;
  if (mode == 1 && (!sums || !counts || !src_rows || !x || !cent_f32)) return SBSA_ERR_ARG;
  if (mode == 2 && !sums) return SBSA_ERR_ARG;
  hipLaunchKernelGGL(kmeans_centroids_kernel, dim3((num_clusters + 3) / 4), dim3(256), 0, stream,
                     mode, sums, counts, src_rows, x, ld_x, row_index, num_clusters, dim, cent_f32,
                     (bf16_t*)cent_bf16, (int32_t*)nullptr, 0);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_kmeans_iterate(const void* x_bf16, const float* x_f32, int64_t ld_x,
                        const int32_t* row_index, int64_t n, int num_clusters, int dim,
                        int32_t* assign, float* sums_hist, int32_t* counts_hist,
                        const int32_t* no_restart, const int32_t* restart_rows,
                        int restart_draws, int32_t* restart_flags, float* cent_f32,
                        void* cent_bf16, uint32_t* member_bits, size_t member_bits_bytes,
                        int it0, int it1, hipStream_t stream) {
  if (!sums_hist || !counts_hist || it0 < 0 || it1 < it0) return SBSA_ERR_ARG;
  if (restart_rows ? (!restart_flags || restart_draws < 1) : !no_restart) return SBSA_ERR_ARG;
  for (int it = it0; it < it1; ++it) {
    float* sums = sums_hist + (int64_t)it * num_clusters * dim;
    int32_t* counts = counts_hist + (int64_t)it * num_clusters;
    int rc = sbsa_kmeans_assign(x_bf16, ld_x, row_index, n, cent_bf16, num_clusters, dim, assign, stream);
    if (rc == SBSA_OK)
      rc = sbsa_kmeans_update(x_f32, ld_x, row_index, n, assign, num_clusters, dim, sums, counts,
                              member_bits, member_bits_bytes, stream);
    if (rc == SBSA_OK && !restart_rows)
      rc = sbsa_kmeans_centroids(1, sums, counts, no_restart, x_f32, ld_x, row_index, num_clusters,
                                 dim, cent_f32, cent_bf16, stream);
    if (rc == SBSA_OK && restart_rows) {
      if (!cent_f32 || !cent_bf16 || dim < 2 || dim > 1024 || dim % 2) return SBSA_ERR_ARG;
      hipLaunchKernelGGL(kmeans_centroids_kernel, dim3((num_clusters + 3) / 4), dim3(256), 0,
                         stream, 3, sums, counts, restart_rows, x_f32, ld_x, row_index,
                         num_clusters, dim, cent_f32, (bf16_t*)cent_bf16, restart_flags + it,
                         restart_draws);
      SBSA_CHECK_LAUNCH();
    }
    if (rc != SBSA_OK) return rc;
  }
  return SBSA_OK;
}

size_t sbsa_bucket_layout_workspace_bytes(int64_t length, int num_clusters) {
  int64_t nchunks = (length + LAYOUT_CHUNK - 1) / LAYOUT_CHUNK;
  return (size_t)(nchunks * num_clusters + 64) * sizeof(int32_t);
}

int sbsa_bucket_layout(const int32_t* assign, int64_t length, int num_clusters, int align,
                       int32_t* sizes, int32_t* indptr, int32_t* posting, int64_t posting_cap,
                       int32_t* inverse, int32_t* total_out, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  if (!assign || !sizes || !indptr || !posting || !inverse || !total_out || !workspace)
    return SBSA_ERR_ARG;
  if (length < 1 || num_clusters < 1 || num_clusters > 1024 || align < 1) return SBSA_ERR_ARG;
  if (workspace_bytes < sbsa_bucket_layout_workspace_bytes(length, num_clusters)) return SBSA_ERR_CAPACITY;
  int64_t bound = length + (int64_t)num_clusters * (align - 1);
  if (posting_cap < bound) return SBSA_ERR_CAPACITY;
  int nchunks = (int)((length + LAYOUT_CHUNK - 1) / LAYOUT_CHUNK);
  int32_t* chunk = (int32_t*)workspace;
  int32_t* first = chunk + (int64_t)nchunks * num_clusters;
  size_t lds = (size_t)num_clusters * sizeof(int);
  hipLaunchKernelGGL(layout_hist_kernel, dim3(nchunks), dim3(256), lds, stream, assign, length,
                     num_clusters, chunk);
  hipLaunchKernelGGL(layout_scan_kernel, dim3(1), dim3(1024), 0, stream, chunk, nchunks,
                     num_clusters, align, sizes, indptr, total_out, first);
  hipLaunchKernelGGL(layout_scatter_kernel, dim3(nchunks), dim3(256), lds, stream, assign, length,
                     num_clusters, chunk, posting, inverse);
  hipLaunchKernelGGL(layout_pad_kernel, dim3(num_clusters + 64), dim3(256), 0, stream, sizes, indptr,
                     num_clusters, first, posting, posting_cap);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_pack_kv(const void* key, const void* value, int64_t stride_tok, int64_t stride_head,
                 int num_kv_heads, int dim, const int32_t* posting, int64_t width,
                 int64_t packed_len, void* packed, hipStream_t stream) {
  if (!key || !value || !posting || !packed || num_kv_heads < 1 || width < 0) return SBSA_ERR_ARG;
  if (dim % 8 || stride_tok % 8 || stride_head % 8 || packed_len < width) return SBSA_ERR_ARG;
  int64_t total = 2 * packed_len * num_kv_heads * (dim / 8);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536 * 8) blocks = 65536 * 8;
  if (blocks < 1) return SBSA_OK;
  hipLaunchKernelGGL(pack_kv_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     (const bf16_t*)key, (const bf16_t*)value, stride_tok, stride_head,
                     num_kv_heads, dim, posting, width, packed_len, (bf16_t*)packed);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

}  // extern "C"
