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

// Per-cluster fp32 sums of the member rows, in row order (deterministic).
// One block per cluster.  The work per launch is a few MB; what it costs is
// dependent load round trips, so the kernel is shaped to need few of them.
// The assignment is scanned in chunks of 8192 rows: each wave loads the
// assignment (and the row map) of its 2048 contiguous rows in one go, 32
// values a lane, counts its members with ballots, and after one block barrier
// writes them at its offset of a block-wide member list, so the list holds the
// cluster's rows in row order across chunks.  The list is summed only when the
// next chunk could overflow it, or at the end -- for a typical cluster once --
// each thread adding its dimensions of the listed rows in list order, the loads
// of KU_BATCH rows issued before any of them is added.
constexpr int KU_CHUNK = 8192;
constexpr int KU_PER_LANE = KU_CHUNK / 4 / 64;   // 32 rows a lane per chunk
constexpr int KU_LIST = 3 * KU_CHUNK / 2;        // member list capacity (48 KB)
constexpr int KU_BATCH = 32;

template <int NJ>  // dims threadIdx.x + 256*j for j < NJ
__global__ __launch_bounds__(256) void kmeans_update_kernel(
    const float* __restrict__ x, int64_t ld_x, const int32_t* __restrict__ row_index, int64_t n,
    const int32_t* __restrict__ assign, int dim, float* __restrict__ sums,
    int32_t* __restrict__ counts) {
  __shared__ int members[KU_LIST];
  __shared__ int wave_cnt[4];
  const int c = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint64_t below = (1ull << lane) - 1;
  float acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = 0.f;
  int total = 0;     // members summed so far
  int listed = 0;    // members in the list, not yet summed
  for (int64_t base = 0; base < n; base += KU_CHUNK) {
    const int64_t seg = base + wave * (KU_CHUNK / 4);
    int a[KU_PER_LANE], r[KU_PER_LANE];
#pragma unroll
    for (int k = 0; k < KU_PER_LANE; ++k) {
      const int64_t i = seg + k * 64 + lane;
      a[k] = i < n ? assign[i] : -1;
      r[k] = i < n ? (row_index ? row_index[i] : (int)i) : 0;
    }
    int cnt_w = 0;
#pragma unroll
    for (int k = 0; k < KU_PER_LANE; ++k) cnt_w += __popcll(__ballot(a[k] == c));
    if (lane == 0) wave_cnt[wave] = cnt_w;
    __syncthreads();
    int at = listed;
    for (int w = 0; w < wave; ++w) at += wave_cnt[w];
#pragma unroll
    for (int k = 0; k < KU_PER_LANE; ++k) {
      const bool mine = a[k] == c;
      const uint64_t ball = __ballot(mine);
      if (mine) members[at + __popcll(ball & below)] = r[k];
      at += __popcll(ball);
    }
    listed += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();    // the list is complete; wave_cnt may be rewritten
    if (listed > KU_LIST - KU_CHUNK || base + KU_CHUNK >= n) {
      for (int m = 0; m < listed; m += KU_BATCH) {
        float v[KU_BATCH][NJ];
#pragma unroll
        for (int u = 0; u < KU_BATCH; ++u) {
          const bool ok = m + u < listed;
          const int64_t src = ok ? members[m + u] : 0;
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int d = threadIdx.x + 256 * j;
            v[u][j] = (ok && d < dim) ? x[src * ld_x + d] : 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < KU_BATCH; ++u)
          if (m + u < listed)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[j] += v[u][j];
      }
      total += listed;
      listed = 0;
      __syncthreads();  // the list is free for the next chunk
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    int d = threadIdx.x + 256 * j;
    if (d < dim) sums[(int64_t)c * dim + d] = acc[j];
  }
  if (threadIdx.x == 0) counts[c] = total;
}

// Centroid step, one wave per cluster.
//  mode 0 (init):       cent = x[row_index[src[c]]]                  flat_index.py:260-262
//  mode 1 (update):     cent = normalize(sums / counts), an empty cluster
//                       (src[c] >= 0) restarts on sample row src[c]  flat_index.py:277-288
//  mode 2 (descriptor): out = bf16(normalize(sums)) as [2, C, dim/2] state.py:883-886
__global__ void kmeans_centroids_kernel(int mode, const float* __restrict__ sums,
                                        const int32_t* __restrict__ counts,
                                        const int32_t* __restrict__ src,
                                        const float* __restrict__ x, int64_t ld_x,
                                        const int32_t* __restrict__ row_index, int num_clusters,
                                        int dim, float* __restrict__ cent_f32,
                                        bf16_t* __restrict__ cent_bf16) {
  const int lane = threadIdx.x & 63;
  const int c = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (c >= num_clusters) return;
  const int per = (dim + 63) / 64;
  float v[16];
  if (mode == 0 || (mode == 1 && src[c] >= 0)) {
    int64_t r = src[c];
    int64_t srow = row_index ? (int64_t)row_index[r] : r;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int d = lane + 64 * i;
      v[i] = (i < per && d < dim) ? x[srow * ld_x + d] : 0.f;
    }
  } else {
    float cnt = (mode == 1) ? (float)counts[c] : 1.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int d = lane + 64 * i;
      float s = (i < per && d < dim) ? sums[(int64_t)c * dim + d] : 0.f;
      v[i] = (mode == 1) ? s / cnt : s;
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

int sbsa_kmeans_update(const float* x, int64_t ld_x, const int32_t* row_index, int64_t n,
                       const int32_t* assign, int num_clusters, int dim, float* sums,
                       int32_t* counts, hipStream_t stream) {
  if (!x || !assign || !sums || !counts || n < 0 || num_clusters < 1) return SBSA_ERR_ARG;
  if (dim < 1 || dim > 1024) return SBSA_ERR_UNSUPPORTED;
  auto kernel = dim <= 256 ? kmeans_update_kernel<1>
                : dim <= 512 ? kmeans_update_kernel<2>
                : dim <= 768 ? kmeans_update_kernel<3> : kmeans_update_kernel<4>;
  hipLaunchKernelGGL(kernel, dim3(num_clusters), dim3(256), 0, stream, x, ld_x, row_index, n,
                     assign, dim, sums, counts);
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
                     (bf16_t*)cent_bf16);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_kmeans_iterate(const void* x_bf16, const float* x_f32, int64_t ld_x,
                        const int32_t* row_index, int64_t n, int num_clusters, int dim,
                        int32_t* assign, float* sums_hist, int32_t* counts_hist,
                        const int32_t* no_restart, float* cent_f32, void* cent_bf16, int it0,
                        int it1, hipStream_t stream) {
  if (!sums_hist || !counts_hist || !no_restart || it0 < 0 || it1 < it0) return SBSA_ERR_ARG;
  for (int it = it0; it < it1; ++it) {
    float* sums = sums_hist + (int64_t)it * num_clusters * dim;
    int32_t* counts = counts_hist + (int64_t)it * num_clusters;
    int rc = sbsa_kmeans_assign(x_bf16, ld_x, row_index, n, cent_bf16, num_clusters, dim, assign, stream);
    if (rc == SBSA_OK)
      rc = sbsa_kmeans_update(x_f32, ld_x, row_index, n, assign, num_clusters, dim, sums, counts, stream);
    if (rc == SBSA_OK)
      rc = sbsa_kmeans_centroids(1, sums, counts, no_restart, x_f32, ld_x, row_index, num_clusters,
                                 dim, cent_f32, cent_bf16, stream);
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
