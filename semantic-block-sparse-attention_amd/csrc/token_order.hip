// S10: store maintenance of the token-order streamed prefill, for gfx950.
//
// The token-order prefill fits the clusters on the prompt's head, lays the
// packed store out with a reservation per cluster, and appends every later
// slice's keys behind their cluster's last key.  The kernels here are the
// device side of that bookkeeping.
//
// Reference behaviour (pfnet-research/semantic-block-sparse-attention):
//   suffix_flush.py:154-170              _nearest_cluster (cosine in fp32, zero descriptors never chosen)
//   routing_map.py:35-64                 key router (whole-vector mode)
//   flat_index.py:144-166                routing_space
//   token_outer_prefill.py:66-87         append_rows (stable rank in position order)
//   token_outer_prefill.py:339-364       _append (K/V, posting and inverse rows, sizes)
//   token_outer_prefill.py:284-318       _fit_and_pack (fitted keys into the reserved runs)
//   token_outer_prefill.py:366-392       _repack (the runs laid out again; here into the
//                                        other buffer of a double-buffered store)
#include "sbsa_common.h"

namespace {

// ---------------------------------------------------------------- assignment --
// ids[h, i] = argmax_c  s2(k[i, h]) . cat(codebooks[h, 0, c], codebooks[h, 1, c])
// with s2 the key's unit vector after the key router (bf16(normalize(k)), when
// router_pass), routing_space (normalize) and _nearest_cluster's own
// normalize, all in fp32; descriptors with every element zero are skipped and
// the first of equal maxima wins (torch.argmax).
//
// Block: 256 threads, 64 keys.  The unit keys stay in LDS in fp32 for the
// whole block; the descriptors stream through LDS 64 at a time in bf16.  A
// thread tells a dead descriptor from the words it multiplies (no shared
// flag, so nothing is cleared while another thread may still read it).
// Thread t owns keys (t & 15) + 16 i and descriptors (t >> 4) + 16 j of a
// tile, i, j < 4: the key tile's row stride D + 4 puts the 16 rows a wave
// reads on distinct banks.
constexpr int NC_KEYS = 64;
constexpr int NC_CENTS = 64;

template <int D>
constexpr size_t nearest_lds_bytes() {
  return (size_t)NC_KEYS * (D + 4) * 4 + (size_t)NC_CENTS * (D + 8) * 2 + 2 * 16 * NC_KEYS * 4;
}

template <int D>
__global__ __launch_bounds__(256) void nearest_cluster_kernel(
    const bf16_t* __restrict__ k, int64_t n, int64_t s_tok, int64_t s_head, int router_pass,
    const bf16_t* __restrict__ codebooks, int num_clusters, int32_t* __restrict__ ids) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_nc[];
  constexpr int XS = D + 4;
  constexpr int CS = D + 8;
  constexpr int PER = D / 64;
  float* xs = reinterpret_cast<float*>(smem_nc);                     // [64][XS]
  bf16_t* cs = reinterpret_cast<bf16_t*>(xs + NC_KEYS * XS);         // [64][CS]
  float* bv = reinterpret_cast<float*>(cs + NC_CENTS * CS);          // [16][64]
  int* bi = reinterpret_cast<int*>(bv + 16 * NC_KEYS);               // [16][64]

  const int h = blockIdx.y;
  const int64_t key0 = (int64_t)blockIdx.x * NC_KEYS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  // unit keys, one wave per row
  for (int r = wave; r < NC_KEYS; r += 4) {
    const int64_t row = key0 + r;
    float v[PER];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      v[i] = row < n ? bf2f(k[row * s_tok + (int64_t)h * s_head + lane + 64 * i]) : 0.f;
      ss += v[i] * v[i];
    }
    if (router_pass) {
      const float n0 = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
      ss = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        v[i] = round_bf16(v[i] / n0);
        ss += v[i] * v[i];
      }
    }
    const float n1 = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
    ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      v[i] = v[i] / n1;
      ss += v[i] * v[i];
    }
    const float n2 = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
#pragma unroll
    for (int i = 0; i < PER; ++i) xs[r * XS + lane + 64 * i] = v[i] / n2;
  }

  const int kg = threadIdx.x & 15, cg = threadIdx.x >> 4;
  float best[4];
  int besti[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    best[i] = -INFINITY;
    besti[i] = 0;
  }
  const bf16_t* cb = codebooks + (int64_t)h * 2 * num_clusters * (D / 2);
  constexpr int CHUNKS = D / 8;          // 16-byte chunks of one descriptor
  for (int c0 = 0; c0 < num_clusters; c0 += NC_CENTS) {
    __syncthreads();                     // previous tile consumed, keys ready
    for (int e = threadIdx.x; e < NC_CENTS * CHUNKS; e += 256) {
      const int c = e / CHUNKS, q = e - c * CHUNKS;
      const int half = q / (CHUNKS / 2), off = (q - half * (CHUNKS / 2)) * 8;
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(
          cb + ((int64_t)half * num_clusters + c0 + c) * (D / 2) + off);
      *reinterpret_cast<u32x4_t*>(cs + c * CS + q * 8) = w;
    }
    __syncthreads();
    float acc[4][4];
    uint32_t nz[4] = {0, 0, 0, 0};       // any nonzero element of descriptor j (sign bits ignored)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    for (int d = 0; d < D; d += 4) {
      f32x4_t a[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const f32x4_t*>(xs + (kg + 16 * i) * XS + d);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x2_t w = *reinterpret_cast<const u32x2_t*>(cs + (cg + 16 * j) * CS + d);
        nz[j] |= (w.x | w.y) & 0x7fff7fffu;
        const float b0 = __uint_as_float(w.x << 16), b1 = __uint_as_float(w.x & 0xffff0000u);
        const float b2 = __uint_as_float(w.y << 16), b3 = __uint_as_float(w.y & 0xffff0000u);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float s = acc[i][j];
          s = fmaf(a[i].x, b0, s);
          s = fmaf(a[i].y, b1, s);
          s = fmaf(a[i].z, b2, s);
          s = fmaf(a[i].w, b3, s);
          acc[i][j] = s;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!nz[j]) continue;
      const int c = c0 + cg + 16 * j;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (acc[i][j] > best[i]) {
          best[i] = acc[i][j];
          besti[i] = c;
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bv[cg * NC_KEYS + kg + 16 * i] = best[i];
    bi[cg * NC_KEYS + kg + 16 * i] = besti[i];
  }
  __syncthreads();
  if (threadIdx.x < NC_KEYS) {
    const int key = threadIdx.x;
    float b = -INFINITY;
    int id = 0;
    bool any = false;
    for (int g = 0; g < 16; ++g) {
      const float v = bv[g * NC_KEYS + key];
      const int c = bi[g * NC_KEYS + key];
      if (v == -INFINITY) continue;
      if (!any || v > b || (v == b && c < id)) {
        b = v;
        id = c;
        any = true;
      }
    }
    if (key0 + key < n) ids[(int64_t)h * n + key0 + key] = id;
  }
}

// ---------------------------------------------------------------- append rows --
// One block (16 waves) per KV head.  Wave w takes a contiguous segment of the
// slice's positions; the ids of 64 positions at a time are grouped by value
// with ballots, so a key's rank among the earlier keys of its cluster is
//   (keys of that cluster in earlier segments) + (earlier in this segment)
//   + (earlier lanes of this group).
// Pass 1 counts per segment, a scan over the segments gives each cluster's
// counts and each segment's start, pass 2 writes the rows.
//   rows[h, i] = indptr[h, c] + sizes[h, c] + rank,   c = ids[h, i]
// overflow[h] bit 0: sizes + counts exceeds reserve for some cluster; bit 1:
// an id outside [0, C) (that key gets row -1).
constexpr int AR_WAVES = 16;

__global__ __launch_bounds__(1024) void append_rows_kernel(
    const int32_t* __restrict__ ids, int64_t n, int num_clusters, const int32_t* __restrict__ indptr,
    const int32_t* __restrict__ sizes, const int32_t* __restrict__ reserve, int32_t* __restrict__ rows,
    int32_t* __restrict__ counts, int32_t* __restrict__ overflow) {
  extern __shared__ int ar_cnt[];                // [16][C] per-segment counts, then base [C]
  __shared__ int s_flag;
  const int C = num_clusters;
  int* base = ar_cnt + AR_WAVES * C;
  const int h = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int32_t* id_h = ids + (int64_t)h * n;
  for (int i = threadIdx.x; i < AR_WAVES * C; i += blockDim.x) ar_cnt[i] = 0;
  if (threadIdx.x == 0) s_flag = 0;
  __syncthreads();
  const int64_t seg = (((n + AR_WAVES - 1) / AR_WAVES) + 63) / 64 * 64;
  const int64_t lo = wave * seg, hi = lo + seg < n ? lo + seg : n;
  int* mine = ar_cnt + wave * C;
  const uint64_t below = (1ull << lane) - 1;

  for (int pass = 0; pass < 2; ++pass) {
    for (int64_t p0 = lo; p0 < hi; p0 += 64) {
      const int64_t p = p0 + lane;
      int id = p < hi ? id_h[p] : -1;
      const bool bad = p < hi && (id < 0 || id >= C);
      if (bad) {
        id = -1;
        if (pass == 1) rows[(int64_t)h * n + p] = -1;
        else atomicOr(&s_flag, 2);
      }
      bool pending = id >= 0;
      for (;;) {
        const uint64_t act = __ballot(pending);
        if (!act) break;
        const int lead = __ffsll((unsigned long long)act) - 1;
        const int lid = __shfl(id, lead, 64);
        const bool hit = pending && id == lid;
        const uint64_t m = __ballot(hit);
        const int start = pass ? base[lid] + mine[lid] : 0;
        if (hit) {
          if (pass) rows[(int64_t)h * n + p] = start + __popcll(m & below);
          pending = false;
        }
        if (lane == lead) mine[lid] += __popcll(m);
      }
    }
    __syncthreads();
    if (pass == 0) {
      for (int c = threadIdx.x; c < C; c += blockDim.x) {
        int run = 0;
        for (int w = 0; w < AR_WAVES; ++w) {
          const int t = ar_cnt[w * C + c];
          ar_cnt[w * C + c] = run;
          run += t;
        }
        const int sz = sizes[(int64_t)h * C + c];
        counts[(int64_t)h * C + c] = run;
        base[c] = indptr[(int64_t)h * (C + 1) + c] + sz;
        if (reserve && sz + run > reserve[(int64_t)h * C + c]) atomicOr(&s_flag, 1);
      }
      __syncthreads();
    }
  }
  if (threadIdx.x == 0 && overflow) overflow[h] = s_flag;
}

// ---------------------------------------------------------------- row moves --
// packed[t, rows[h, i], h, :] = (t ? value : key)[i, h, :]   (16-byte chunks;
// rows outside [0, packed_len) are skipped).
__global__ void copy_rows_kernel(const bf16_t* __restrict__ key, const bf16_t* __restrict__ value,
                                 int64_t s_tok, int64_t s_head, int64_t n, int hkv, int dim,
                                 const int32_t* __restrict__ rows, int64_t rows_ld,
                                 bf16_t* __restrict__ packed, int64_t packed_len) {
  const int chunks = dim / 8;
  const int64_t per_plane = n * hkv * chunks;
  const int64_t total = 2 * per_plane;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = e / per_plane;
    const int64_t rem = e - t * per_plane;
    const int64_t i = rem / (hkv * chunks);
    const int hc = (int)(rem - i * (hkv * chunks));
    const int h = hc / chunks, ch = hc - h * chunks;
    const int64_t r = rows[(int64_t)h * rows_ld + i];
    if (r < 0 || r >= packed_len) continue;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>((t ? value : key) + i * s_tok +
                                                         (int64_t)h * s_head + ch * 8);
    *reinterpret_cast<u32x4_t*>(packed + ((t * packed_len + r) * hkv + h) * dim + ch * 8) = v;
  }
}

// The index side of an append: posting[h, row] = first + i and
// inverse[h, first + i] = row for the slice's keys; sizes_before = sizes and
// sizes += counts for every (h, c).
__global__ void append_index_kernel(const int32_t* __restrict__ rows, int64_t n, int hkv,
                                    int64_t first, int32_t* __restrict__ posting, int64_t posting_width,
                                    int32_t* __restrict__ inverse, int64_t inverse_len,
                                    int32_t* __restrict__ sizes, const int32_t* __restrict__ counts,
                                    int num_clusters, int32_t* __restrict__ sizes_before) {
  const int64_t nk = n * hkv, nc = (int64_t)hkv * num_clusters;
  const int64_t total = nk > nc ? nk : nc;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    if (e < nk) {
      const int h = (int)(e / n);
      const int64_t i = e - (int64_t)h * n;
      const int32_t r = rows[e];
      if (r >= 0 && r < posting_width) posting[(int64_t)h * posting_width + r] = (int32_t)(first + i);
      if (first + i < inverse_len) inverse[(int64_t)h * inverse_len + first + i] = r;
    }
    if (e < nc) {
      const int32_t s = sizes[e];
      if (sizes_before) sizes_before[e] = s;
      sizes[e] = s + counts[e];
    }
  }
}

// Relayout map: the key at position i of head h sat at old_rows[h, i] in runs
// starting at old_indptr; its cluster b is the last with old_indptr[b] <=
// row (torch.searchsorted(..., right=True) - 1), and it moves to the same
// offset in the run at new_indptr[b].  Writes new_rows[h, i] and
// posting[h, new row] = i.
__global__ void relayout_map_kernel(const int32_t* __restrict__ old_rows, int64_t old_ld, int64_t n,
                                    int hkv, const int32_t* __restrict__ old_indptr,
                                    const int32_t* __restrict__ new_indptr, int num_clusters,
                                    int32_t* __restrict__ new_rows, int64_t new_ld,
                                    int32_t* __restrict__ posting, int64_t posting_width) {
  const int64_t total = n * hkv;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int h = (int)(e / n);
    const int64_t i = e - (int64_t)h * n;
    const int32_t r = old_rows[(int64_t)h * old_ld + i];
    const int32_t* ip = old_indptr + (int64_t)h * (num_clusters + 1);
    int lo = 0, hi = num_clusters + 1;           // first index with ip[idx] > r
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (ip[mid] <= r) lo = mid + 1;
      else hi = mid;
    }
    int b = lo - 1;
    int32_t nr = -1;
    if (b >= 0 && b < num_clusters) nr = r - ip[b] + new_indptr[(int64_t)h * (num_clusters + 1) + b];
    new_rows[(int64_t)h * new_ld + i] = nr;
    if (nr >= 0 && nr < posting_width) posting[(int64_t)h * posting_width + nr] = (int32_t)i;
  }
}

// (t ? value_out : key_out)[i, h, :] = packed[t, inverse[h, first + i], h, :]
__global__ void gather_rows_kernel(const bf16_t* __restrict__ packed, int64_t packed_len, int hkv,
                                   int dim, const int32_t* __restrict__ inverse, int64_t inverse_ld,
                                   int64_t first, int64_t n, bf16_t* __restrict__ key_out,
                                   bf16_t* __restrict__ value_out, int64_t s_tok, int64_t s_head) {
  const int chunks = dim / 8;
  const int64_t per_plane = n * hkv * chunks;
  const int64_t total = 2 * per_plane;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = e / per_plane;
    const int64_t rem = e - t * per_plane;
    const int64_t i = rem / (hkv * chunks);
    const int hc = (int)(rem - i * (hkv * chunks));
    const int h = hc / chunks, ch = hc - h * chunks;
    const int64_t r = inverse[(int64_t)h * inverse_ld + first + i];
    u32x4_t v = u32x4_t{0, 0, 0, 0};
    if (r >= 0 && r < packed_len)
      v = *reinterpret_cast<const u32x4_t*>(packed + ((t * packed_len + r) * hkv + h) * dim + ch * 8);
    *reinterpret_cast<u32x4_t*>((t ? value_out : key_out) + i * s_tok + (int64_t)h * s_head + ch * 8) = v;
  }
}

// dst[t, new_rows[h, i], h, :] = src[t, old_rows[h, i], h, :] (a repack into the
// other buffer of a double-buffered store; rows out of range are skipped).
__global__ void move_rows_kernel(const bf16_t* __restrict__ src, bf16_t* __restrict__ dst,
                                 int64_t packed_len, int hkv, int dim, int64_t n,
                                 const int32_t* __restrict__ old_rows, int64_t old_ld,
                                 const int32_t* __restrict__ new_rows, int64_t new_ld) {
  const int chunks = dim / 8;
  const int64_t per_plane = n * hkv * chunks;
  const int64_t total = 2 * per_plane;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = e / per_plane;
    const int64_t rem = e - t * per_plane;
    const int64_t i = rem / (hkv * chunks);
    const int hc = (int)(rem - i * (hkv * chunks));
    const int h = hc / chunks, ch = hc - h * chunks;
    const int64_t ro = old_rows[(int64_t)h * old_ld + i];
    const int64_t rn = new_rows[(int64_t)h * new_ld + i];
    if (ro < 0 || ro >= packed_len || rn < 0 || rn >= packed_len) continue;
    const int64_t plane = t * packed_len;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src + ((plane + ro) * hkv + h) * dim + ch * 8);
    *reinterpret_cast<u32x4_t*>(dst + ((plane + rn) * hkv + h) * dim + ch * 8) = v;
  }
}

unsigned grid_for(int64_t work, int per_block) {
  int64_t b = (work + per_block - 1) / per_block;
  if (b > 8192) b = 8192;
  return (unsigned)(b > 0 ? b : 1);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" {

int sbsa_nearest_cluster(const void* k, int64_t n, int64_t stride_tok, int64_t stride_head,
                         int num_kv_heads, int dim, int router_pass, const void* codebooks,
                         int num_clusters, int32_t* ids, hipStream_t stream) {
  if (!k || !codebooks || !ids || n < 0 || num_kv_heads < 1) return SBSA_ERR_ARG;
  if (num_clusters < NC_CENTS || num_clusters % NC_CENTS || num_clusters > 1024) return SBSA_ERR_UNSUPPORTED;
  if (!aligned16(codebooks)) return SBSA_ERR_ARG;
  if (n == 0) return SBSA_OK;
  const dim3 grid((unsigned)((n + NC_KEYS - 1) / NC_KEYS), (unsigned)num_kv_heads);
  switch (dim) {
    case 128: {
      const size_t lds = nearest_lds_bytes<128>();
      hipFuncSetAttribute((const void*)nearest_cluster_kernel<128>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      hipLaunchKernelGGL(nearest_cluster_kernel<128>, grid, dim3(256), lds, stream, (const bf16_t*)k, n,
                         stride_tok, stride_head, router_pass, (const bf16_t*)codebooks, num_clusters, ids);
      break;
    }
    case 256: {
      const size_t lds = nearest_lds_bytes<256>();
      hipFuncSetAttribute((const void*)nearest_cluster_kernel<256>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      hipLaunchKernelGGL(nearest_cluster_kernel<256>, grid, dim3(256), lds, stream, (const bf16_t*)k, n,
                         stride_tok, stride_head, router_pass, (const bf16_t*)codebooks, num_clusters, ids);
      break;
    }
    default:
      return SBSA_ERR_UNSUPPORTED;
  }
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_append_rows(const int32_t* ids, int64_t n, int num_kv_heads, int num_clusters,
                     const int32_t* indptr, const int32_t* sizes, const int32_t* reserve,
                     int32_t* rows, int32_t* counts, int32_t* overflow, hipStream_t stream) {
  if (!indptr || !sizes || !counts || n < 0 || num_kv_heads < 1) return SBSA_ERR_ARG;
  if (n > 0 && (!ids || !rows)) return SBSA_ERR_ARG;
  if (num_clusters < 1 || num_clusters > 1024) return SBSA_ERR_UNSUPPORTED;
  if (n > INT32_MAX) return SBSA_ERR_UNSUPPORTED;
  const size_t lds = (size_t)(AR_WAVES + 1) * num_clusters * sizeof(int);
  hipFuncSetAttribute((const void*)append_rows_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                      (int)lds);
  hipLaunchKernelGGL(append_rows_kernel, dim3(num_kv_heads), dim3(64 * AR_WAVES), lds, stream, ids, n,
                     num_clusters, indptr, sizes, reserve, rows, counts, overflow);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_append_kv(const void* key, const void* value, int64_t stride_tok, int64_t stride_head,
                   int64_t n, int num_kv_heads, int dim, const int32_t* rows, int64_t first_position,
                   void* packed, int64_t packed_len, int32_t* posting, int64_t posting_width,
                   int32_t* inverse, int64_t inverse_len, int32_t* sizes, const int32_t* counts,
                   int num_clusters, int32_t* sizes_before, hipStream_t stream) {
  if (!key || !value || !rows || !packed || !posting || !inverse || !sizes || !counts) return SBSA_ERR_ARG;
  if (n < 0 || num_kv_heads < 1 || num_clusters < 1 || first_position < 0) return SBSA_ERR_ARG;
  if (dim % 8 || dim < 8 || stride_tok % 8 || stride_head % 8) return SBSA_ERR_ARG;
  if (!aligned16(key) || !aligned16(value) || !aligned16(packed)) return SBSA_ERR_ARG;
  if (first_position + n > inverse_len) return SBSA_ERR_CAPACITY;
  const int64_t moves = 2 * n * num_kv_heads * (dim / 8);
  if (moves > 0)
    hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(moves, 256)), dim3(256), 0, stream,
                       (const bf16_t*)key, (const bf16_t*)value, stride_tok, stride_head, n, num_kv_heads,
                       dim, rows, n, (bf16_t*)packed, packed_len);
  const int64_t nk = n * num_kv_heads, nc = (int64_t)num_kv_heads * num_clusters;
  hipLaunchKernelGGL(append_index_kernel, dim3(grid_for(nk > nc ? nk : nc, 256)), dim3(256), 0, stream,
                     rows, n, num_kv_heads, first_position, posting, posting_width, inverse, inverse_len,
                     sizes, counts, num_clusters, sizes_before);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_relayout_runs(const void* key, const void* value, int64_t stride_tok, int64_t stride_head,
                       int64_t n, int num_kv_heads, int dim, const int32_t* old_rows, int64_t old_rows_ld,
                       const int32_t* old_indptr, const int32_t* new_indptr, int num_clusters,
                       void* packed, int64_t packed_len, int32_t* posting, int64_t posting_width,
                       int32_t* inverse, int64_t inverse_ld, hipStream_t stream) {
  if (!key || !value || !old_rows || !old_indptr || !new_indptr || !packed || !posting || !inverse)
    return SBSA_ERR_ARG;
  if (n < 0 || num_kv_heads < 1 || num_clusters < 1) return SBSA_ERR_ARG;
  if (dim % 8 || dim < 8 || stride_tok % 8 || stride_head % 8) return SBSA_ERR_ARG;
  if (!aligned16(key) || !aligned16(value) || !aligned16(packed)) return SBSA_ERR_ARG;
  if (old_rows_ld < n || inverse_ld < n) return SBSA_ERR_CAPACITY;
  // the map reads old_rows while other threads write inverse: they must not overlap
  const char* a0 = (const char*)old_rows;
  const char* a1 = a0 + (size_t)num_kv_heads * old_rows_ld * 4;
  const char* b0 = (const char*)inverse;
  const char* b1 = b0 + (size_t)num_kv_heads * inverse_ld * 4;
  if (a0 < b1 && b0 < a1) return SBSA_ERR_ARG;
  if (n == 0) return SBSA_OK;
  hipLaunchKernelGGL(relayout_map_kernel, dim3(grid_for(n * num_kv_heads, 256)), dim3(256), 0, stream,
                     old_rows, old_rows_ld, n, num_kv_heads, old_indptr, new_indptr, num_clusters, inverse,
                     inverse_ld, posting, posting_width);
  const int64_t moves = 2 * n * num_kv_heads * (dim / 8);
  hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(moves, 256)), dim3(256), 0, stream,
                     (const bf16_t*)key, (const bf16_t*)value, stride_tok, stride_head, n, num_kv_heads, dim,
                     inverse, inverse_ld, (bf16_t*)packed, packed_len);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_gather_rows(const void* packed, int64_t packed_len, int num_kv_heads, int dim,
                     const int32_t* inverse, int64_t inverse_ld, int64_t first, int64_t n, void* key_out,
                     void* value_out, int64_t stride_tok, int64_t stride_head, hipStream_t stream) {
  if (!packed || !inverse || !key_out || !value_out || n < 0 || first < 0 || num_kv_heads < 1)
    return SBSA_ERR_ARG;
  if (dim % 8 || dim < 8 || stride_tok % 8 || stride_head % 8) return SBSA_ERR_ARG;
  if (!aligned16(packed) || !aligned16(key_out) || !aligned16(value_out)) return SBSA_ERR_ARG;
  if (first + n > inverse_ld) return SBSA_ERR_CAPACITY;
  if (n == 0) return SBSA_OK;
  const int64_t moves = 2 * n * num_kv_heads * (dim / 8);
  hipLaunchKernelGGL(gather_rows_kernel, dim3(grid_for(moves, 256)), dim3(256), 0, stream,
                     (const bf16_t*)packed, packed_len, num_kv_heads, dim, inverse, inverse_ld, first, n,
                     (bf16_t*)key_out, (bf16_t*)value_out, stride_tok, stride_head);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

int sbsa_repack_runs(const void* src_packed, void* dst_packed, int64_t packed_len, int num_kv_heads,
                     int dim, int64_t n, const int32_t* old_rows, int64_t old_rows_ld,
                     const int32_t* old_indptr, const int32_t* new_indptr, int num_clusters,
                     int32_t* posting, int64_t posting_width, int32_t* inverse, int64_t inverse_ld,
                     hipStream_t stream) {
  if (!src_packed || !dst_packed || !old_rows || !old_indptr || !new_indptr || !posting || !inverse)
    return SBSA_ERR_ARG;
  if (n < 0 || num_kv_heads < 1 || num_clusters < 1 || dim % 8 || dim < 8) return SBSA_ERR_ARG;
  if (!aligned16(src_packed) || !aligned16(dst_packed) || src_packed == dst_packed) return SBSA_ERR_ARG;
  if (old_rows_ld < n || inverse_ld < n) return SBSA_ERR_CAPACITY;
  const char* a0 = (const char*)old_rows;
  const char* a1 = a0 + (size_t)num_kv_heads * old_rows_ld * 4;
  const char* b0 = (const char*)inverse;
  const char* b1 = b0 + (size_t)num_kv_heads * inverse_ld * 4;
  if (a0 < b1 && b0 < a1) return SBSA_ERR_ARG;
  if (n == 0) return SBSA_OK;
  hipLaunchKernelGGL(relayout_map_kernel, dim3(grid_for(n * num_kv_heads, 256)), dim3(256), 0, stream,
                     old_rows, old_rows_ld, n, num_kv_heads, old_indptr, new_indptr, num_clusters, inverse,
                     inverse_ld, posting, posting_width);
  const int64_t moves = 2 * n * num_kv_heads * (dim / 8);
  hipLaunchKernelGGL(move_rows_kernel, dim3(grid_for(moves, 256)), dim3(256), 0, stream,
                     (const bf16_t*)src_packed, (bf16_t*)dst_packed, packed_len, num_kv_heads, dim, n,
                     old_rows, old_rows_ld, inverse, inverse_ld);
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

}  // extern "C"
