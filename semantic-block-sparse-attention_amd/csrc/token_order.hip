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
// The fp32 products run on bf16 MFMA: a unit key is split into three bf16
// terms s2 = hi + mid + lo (each the rounding of what the earlier terms leave,
// so the sum carries s2's 24 significant bits), the descriptors are bf16
// already, every term's product is exact in fp32 and the three MFMAs
// accumulate in fp32.
//
// Block: 4 waves, 16 keys per wave held in registers as MFMA A operands
// (row lane % 16, k = 32 s + 8 (lane / 16) .. +8: the four lanes of a row
// hold a quarter of it each); descriptors are staged through LDS 64 at a time.
// A lane tells a dead descriptor from the words it multiplies, OR-ed over the
// four lanes of its column.
constexpr int NC_WAVE_KEYS = 16;
constexpr int NC_KEYS = 4 * NC_WAVE_KEYS;   // keys per block
constexpr int NC_CENTS = 64;                // descriptors per LDS tile

__device__ __forceinline__ u32x4_t pack8_bf16(const float* v) {
  return u32x4_t{pack2bf(v[0], v[1]), pack2bf(v[2], v[3]), pack2bf(v[4], v[5]), pack2bf(v[6], v[7])};
}

template <int D>
__global__ __launch_bounds__(256) void nearest_cluster_kernel(
    const bf16_t* __restrict__ k, int64_t n, int64_t s_tok, int64_t s_head, int router_pass,
    const bf16_t* __restrict__ codebooks, int num_clusters, int32_t* __restrict__ ids) {
  constexpr int KS = D / 32;
  constexpr int LDR = D + 8;
  __shared__ __attribute__((aligned(16))) bf16_t sc[NC_CENTS * LDR];
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t key = (int64_t)blockIdx.x * NC_KEYS + wave * NC_WAVE_KEYS + (lane & 15);
  const bool ok = key < n;

  // this lane's quarter of its key row, in fp32
  float v[KS][8];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    u32x4_t w = u32x4_t{0, 0, 0, 0};
    if (ok)
      w = *reinterpret_cast<const u32x4_t*>(k + key * s_tok + (int64_t)h * s_head + s * 32 + (lane >> 4) * 8);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[s][2 * j] = __uint_as_float(ww[j] << 16);
      v[s][2 * j + 1] = __uint_as_float(ww[j] & 0xffff0000u);
    }
  }
  auto row_norm = [&]() {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[s][e] * v[s][e];
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    return fmaxf(sqrtf(ss), 1e-12f);
  };
  if (router_pass) {
    const float n0 = row_norm();
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[s][e] = round_bf16(v[s][e] / n0);
  }
  const float n1 = row_norm();
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) v[s][e] = v[s][e] / n1;
  const float n2 = row_norm();
  u32x4_t a_hi[KS], a_mid[KS], a_lo[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    float hi[8], mid[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = v[s][e] / n2;
      hi[e] = round_bf16(x);
      mid[e] = round_bf16(x - hi[e]);
      lo[e] = round_bf16((x - hi[e]) - mid[e]);
    }
    a_hi[s] = pack8_bf16(hi);
    a_mid[s] = pack8_bf16(mid);
    a_lo[s] = pack8_bf16(lo);
  }

  float best[4];
  int bidx[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    best[i] = -INFINITY;
    bidx[i] = 0;
  }
  const bf16_t* cb = codebooks + (int64_t)h * 2 * num_clusters * (D / 2);
  constexpr int CHUNKS = D / 8;
  for (int c0 = 0; c0 < num_clusters; c0 += NC_CENTS) {
    __syncthreads();                    // the previous tile is consumed
    for (int e = threadIdx.x; e < NC_CENTS * CHUNKS; e += 256) {
      const int c = e / CHUNKS, q = e - c * CHUNKS;
      const int half = q / (CHUNKS / 2), off = (q - half * (CHUNKS / 2)) * 8;
      *reinterpret_cast<u32x4_t*>(&sc[c * LDR + q * 8]) = *reinterpret_cast<const u32x4_t*>(
          cb + ((int64_t)half * num_clusters + c0 + c) * (D / 2) + off);
    }
    __syncthreads();
#pragma unroll
    for (int cbk = 0; cbk < NC_CENTS / 16; ++cbk) {
      f32x4_t acc = f32x4_t{0, 0, 0, 0};
      uint32_t nz = 0;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4_t b = *reinterpret_cast<const u32x4_t*>(&sc[(cbk * 16 + (lane & 15)) * LDR + s * 32 + (lane >> 4) * 8]);
        nz |= (b.x | b.y | b.z | b.w) & 0x7fff7fffu;
        acc = mfma16x16x32(as_bf16x8(a_hi[s]), as_bf16x8(b), acc);
        acc = mfma16x16x32(as_bf16x8(a_mid[s]), as_bf16x8(b), acc);
        acc = mfma16x16x32(as_bf16x8(a_lo[s]), as_bf16x8(b), acc);
      }
      nz |= (uint32_t)__shfl_xor((int)nz, 16, 64);
      nz |= (uint32_t)__shfl_xor((int)nz, 32, 64);
      if (nz) {
        const int col = c0 + cbk * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (acc[i] > best[i]) {        // columns rise with cbk and c0: strict > keeps the first
            best[i] = acc[i];
            bidx[i] = col;
          }
      }
    }
  }
  // acc[i] is key row 4 (lane / 16) + i of the wave, column lane % 16: reduce the 16 columns
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float bv = best[i];
    int bi = bidx[i];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    const int64_t r = (int64_t)blockIdx.x * NC_KEYS + wave * NC_WAVE_KEYS + (lane >> 4) * 4 + i;
    if ((lane & 15) == 0 && r < n) ids[(int64_t)h * n + r] = bi;
  }
}

// ---------------------------------------------------------------- append rows --
// One block (16 waves) per KV head.  Wave w takes a contiguous segment of the
// slice's positions; the ids of 64 positions at a time are grouped by value
// with ballots (on the scalar unit, one round per distinct id; the running
// counts are then read once per lane and raised once per id), so a key's rank
// among the earlier keys of its cluster is
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
    // up to 8 chunks of 64 ids are loaded together, then grouped chunk by chunk
    for (int64_t g0 = lo; g0 < hi; g0 += 8 * 64) {
      int idv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t p = g0 + j * 64 + lane;
        idv[j] = p < hi ? id_h[p] : -1;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (g0 + j * 64 >= hi) break;
        const int64_t p = g0 + j * 64 + lane;
        int id = idv[j];
        const bool bad = p < hi && (id < 0 || id >= C);
        if (bad) {
          id = -1;
          if (pass == 1) rows[(int64_t)h * n + p] = -1;
          else atomicOr(&s_flag, 2);
        }
        // the lane's rank among the earlier lanes with its id, and (in the first
        // lane of each id) the id's count in the group: one round per distinct id,
        // on the scalar unit and the lane masks only
        bool pending = id >= 0;
        int rank = 0, lead_count = 0;
        for (;;) {
          const uint64_t act = __ballot(pending);
          if (!act) break;
          const int lead = __ffsll((unsigned long long)act) - 1;
          const int lid = __builtin_amdgcn_readlane(id, lead);
          const bool hit = pending && id == lid;
          const uint64_t m = __ballot(hit);
          if (hit) {
            rank = __popcll(m & below);
            pending = false;
          }
          if (lane == lead) lead_count = __popcll(m);
        }
        // the group's keys follow the segment's earlier keys of their cluster:
        // read the running counts, then add the group's (one lane per id)
        if (id >= 0) {
          if (pass == 1) rows[(int64_t)h * n + p] = base[id] + mine[id] + rank;
        }
        // every lane has read mine[] before the first lanes add to it (in order on
        // the GPU; the barrier keeps the compiler from moving them)
        __builtin_amdgcn_wave_barrier();
        if (lead_count > 0) mine[id] += lead_count;
        __builtin_amdgcn_wave_barrier();
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
  if (!aligned16(codebooks) || !aligned16(k) || stride_tok % 8 || stride_head % 8) return SBSA_ERR_ARG;
  if (n == 0) return SBSA_OK;
  const dim3 grid((unsigned)((n + NC_KEYS - 1) / NC_KEYS), (unsigned)num_kv_heads);
  switch (dim) {
    case 128:
      hipLaunchKernelGGL(nearest_cluster_kernel<128>, grid, dim3(256), 0, stream, (const bf16_t*)k, n,
                         stride_tok, stride_head, router_pass, (const bf16_t*)codebooks, num_clusters, ids);
      break;
    case 256:
      hipLaunchKernelGGL(nearest_cluster_kernel<256>, grid, dim3(256), 0, stream, (const bf16_t*)k, n,
                         stride_tok, stride_head, router_pass, (const bf16_t*)codebooks, num_clusters, ids);
      break;
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
  if (hipFuncSetAttribute((const void*)append_rows_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return SBSA_ERR_UNSUPPORTED;
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
