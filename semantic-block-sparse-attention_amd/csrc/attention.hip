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
// the prompt-order window, causally masked) in 64-key tiles.  Both GEMMs are
// on bf16 MFMA 16x16x32 in the transposed form S^T = K Q^T, O^T = V^T P^T,
// so the softmax probabilities come out of the first MFMA already in the
// B-operand layout of the second and never pass through LDS.
#include "sbsa_common.h"

namespace {

struct AttnArgs {
  const bf16_t* q;          // [Qc, Hq, D] chunk queries
  int64_t q_sq, q_sh;
  const bf16_t* packed;     // [2, Lp, Hkv, D] cluster-ordered K/V
  int64_t packed_len;
  const bf16_t* korig;      // prompt-order keys from position wstart: k[pos - wstart, h, :]
  const bf16_t* vorig;      // prompt-order values, same rows
  int64_t o_st, o_sh;       // their token / head strides (elements)
  const int32_t* indptr;    // [Hkv, C+1] packed run starts
  const int32_t* nvis;      // [Hkv, C] visible rows per cluster
  const int32_t* rev_indptr;// [Hkv*C + 1]
  const int32_t* qvals;     // [nnz] query slots per (head, cluster)
  const int4* items;
  int32_t* queue;           // n[8], offset[8], counter[8]: one work queue per XCD
  bf16_t* part_o;           // [nnz, G, D]
  float* part_lse;          // [nnz, G]
  bf16_t* local_o;          // [Qc, Hq, D] strided
  int64_t lo_sq, lo_sh;
  float* local_lse;         // [Qc, Hq] or null
  int Hkv, C, Hq;
  int64_t chunk_start, wstart;
  float scale_log2;         // sm_scale * log2(e)
};

constexpr int KT = 32;      // keys per tile
constexpr int PREFILL_RB = 2;                       // 16-row blocks per wave
constexpr int PREFILL_ROWS = 4 * 16 * PREFILL_RB;   // (query, head) rows per work item
constexpr int KB = KT / 16; // 16-key blocks per tile
constexpr int T2 = KT / 32; // 32-key MFMA steps of O^T += V^T P^T per tile
// Probabilities are taken against a reference maximum per row and may reach
// 2^OVERFLOW_LOG2 (well inside fp32 and bf16 range) before an item is redone.
constexpr float OVERFLOW_LOG2 = 64.0f;
constexpr int BUFFER_CONFIG = 0x00020000;   // raw buffer resource, 32-bit data format

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// LDS tile layout: K and V rows of D bf16, row-major; the 16-byte chunks of
// row r are permuted by an XOR (K: chunk ^ (r % 16), V: chunk ^ 2 (r % 8)) so
// that the MFMA operand reads of one LDS cycle (16 lanes of 16 bytes for K,
// 32 lanes of 8 bytes for the transposing V reads: 256 bytes, the 64 banks)
// hit distinct banks.  Tiles are filled straight
// from global memory by buffer loads into LDS (lane l writes slot l of a 1 KB
// run; rows past the item's last key are out of the buffer's range and read
// as zero).
template <int D>
struct AttnTileShape {
  static constexpr int CH = D / 8;                    // 16-byte chunks per row
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int TILE_BYTES = KT * ROW_BYTES;   // one of K or V
  static constexpr int BUF_BYTES = 2 * TILE_BYTES;    // K then V
  static constexpr size_t LDS_BYTES = 2 * (size_t)BUF_BYTES;
  static constexpr int ROWS_PER_INST = 64 / CH;       // rows one wave instruction covers
  static constexpr int INSTS = KT / ROWS_PER_INST;    // instructions per K (or V) tile
  static constexpr int PER_WAVE = INSTS / 4;
};

// RB: 16-row blocks per wave (a block's item holds 64 RB (query, head) rows);
// with RB = 1 two blocks share a CU.
template <int D, int G, int RB>
__global__ __launch_bounds__(256, 3 - RB) void attn_items_kernel(AttnArgs a) {
  using S = AttnTileShape<D>;
  constexpr int KS = D / 32;
  constexpr int DB = D / 16;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_attn[];
  __shared__ int s_item;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const float NEG_INF = -INFINITY;
  // blocks are dispatched round-robin over the 8 XCDs: take work from this
  // XCD's queue, then steal from the others
  const int home = blockIdx.x & 7;
  int probe = 0;

  // --- per-lane address bases (fixed for the kernel) ---------------------
  // loads: instruction m of this wave covers rows r0 + m * 4 * ROWS_PER_INST
  const int r0 = wave * S::ROWS_PER_INST + lane / S::CH;
  const int cpos = lane % S::CH;
  // instruction m covers rows r0 + 4 m RPI: (r0 + 4 m RPI) % 8 == r0 % 8, and
  // % 16 alternates with m when 4 RPI == 8
  uint32_t kslot[2], vslot;
  kslot[0] = (uint32_t)((cpos ^ (r0 & 15)) * 16);
  kslot[1] = (uint32_t)((cpos ^ ((r0 + 4 * S::ROWS_PER_INST) & 15)) * 16);
  vslot = (uint32_t)((cpos ^ ((r0 & 7) << 1)) * 16);
  // K operand reads: row kb*16 + l16, chunk (s*4 + lg) ^ l16
  //   = 4 ((s & ~3) | ((s & 3) ^ (l16 >> 2))) + (lg ^ (l16 & 3))
  int kbase[4];
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4)
    kbase[s4] = l16 * S::ROW_BYTES + 64 * (s4 ^ (l16 >> 2)) + 16 * (lg ^ (l16 & 3));
  // V^T operand (transposing reads): row t2*32 + hlf*16 + lg*4 + (l16 >> 2),
  // dims db*16 + (l16 & 3)*4 .. +4: 32-byte pair (db ^ zz) with zz = row % 8
  const int zz = ((lg & 1) << 2) | (l16 >> 2);
  int vbase[8];
#pragma unroll
  for (int dl = 0; dl < 8; ++dl)
    vbase[dl] = (lg * 4 + (l16 >> 2)) * S::ROW_BYTES + 32 * (dl ^ zz) + 16 * ((l16 & 3) >> 1) + 8 * (l16 & 1);

  // LDS: K tiles in buffers 0/1, V tiles in buffers 2/3
  unsigned char* const kbuf[2] = {smem_attn, smem_attn + S::TILE_BYTES};
  unsigned char* const vbuf[2] = {smem_attn + 2 * S::TILE_BYTES, smem_attn + 3 * S::TILE_BYTES};

  while (probe < 8) {
    const int x = (home + probe) & 7;
    if (threadIdx.x == 0) {
      const int v = atomicAdd(&a.queue[16 + x], 1);
      s_item = v < a.queue[x] ? a.queue[8 + x] + v : -1;
    }
    __syncthreads();
    const int idx = s_item;
    __syncthreads();
    if (idx < 0) {
      ++probe;
      continue;
    }
    const int4 it = a.items[idx];
    const int h = it.x, c = it.y, qb = it.z, qn = it.w;
    const bool local = c < 0;
    const bf16_t* kp;
    const bf16_t* vp;
    int64_t rs;
    int nkeys;
    int64_t entry0 = 0;
    if (local) {
      kp = a.korig + (int64_t)h * a.o_sh;   // row 0 is position wstart
      vp = a.vorig + (int64_t)h * a.o_sh;
      rs = a.o_st;
      nkeys = (int)(a.chunk_start + qb + qn - a.wstart);
    } else {
      int64_t r0g = a.indptr[h * (a.C + 1) + c];
      kp = a.packed + r0g * a.Hkv * D + (int64_t)h * D;
      vp = kp + a.packed_len * a.Hkv * D;
      rs = (int64_t)a.Hkv * D;
      nkeys = a.nvis[h * a.C + c];
      entry0 = (int64_t)a.rev_indptr[h * a.C + c] + qb;
    }
    if (nkeys <= 0) continue;
    const int ntiles = (nkeys + KT - 1) / KT;
    const uint32_t rs_bytes = (uint32_t)(rs * 2);
    const uint32_t kvoff = (uint32_t)r0 * rs_bytes;

    // direct loads of the K (or V) rows of tile t into an LDS buffer; rows
    // past the item's last key are outside the buffer range and read as 0
    auto issue = [&](const bf16_t* base, int t, unsigned char* dst_tile, bool is_k) {
      const int t0 = t * KT;
      const uint32_t valid = (uint32_t)(nkeys - t0) * rs_bytes;
      __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(base + (int64_t)t0 * rs), (short)0, (int)valid, BUFFER_CONFIG);
      unsigned char* dst = dst_tile + wave * 1024;
#pragma unroll
      for (int m = 0; m < S::PER_WAVE; ++m) {
        const uint32_t roff = kvoff + (uint32_t)(m * 4 * S::ROWS_PER_INST) * rs_bytes;
        const uint32_t slot = is_k ? kslot[m & 1] : vslot;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(dst + m * 4096), 16, roff + slot, 0, 0, 0);
      }
    };

    // Q rows of this wave: R = wave*16*RB + rb*16 + l16 -> (slot i, head j)
    u32x4_t qr[RB][KS];
    int qlim[RB];
    int qidx_r[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int R = wave * 16 * RB + rb * 16 + l16;
      const int i = R / G, j = R % G;
      const bool ok = i < qn;
      int qidx = 0;
      if (ok) qidx = local ? qb + i : a.qvals[entry0 + i];
      qidx_r[rb] = ok ? qidx : -1;
      qlim[rb] = local ? (int)(a.chunk_start + qidx - a.wstart) : 0x7fffffff;
      const bf16_t* src = a.q + (int64_t)qidx * a.q_sq + (int64_t)(h * G + j) * a.q_sh + lg * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        qr[rb][s] = ok ? *reinterpret_cast<const u32x4_t*>(src + s * 32) : u32x4_t{0, 0, 0, 0};
    }
    // the last key any row of this wave may see, and the last key every row sees
    int wave_lim = qlim[0], wave_min = 0x7fffffff;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      wave_lim = max(wave_lim, qlim[rb]);
      if (qidx_r[rb] >= 0) wave_min = min(wave_min, qlim[rb]);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      wave_lim = max(wave_lim, __shfl_xor(wave_lim, o, 64));
      wave_min = min(wave_min, __shfl_xor(wave_min, o, 64));
    }

    // S^T = K Q^T for one tile: lane holds keys kb*16 + lg*4 + i of row (rb, l16).
    // K fragments (s, kb) are read KA_AHEAD ahead of their MFMAs.
    constexpr int NKF = KS * KB;
    constexpr int KA_AHEAD = 3;
    auto kread = [&](const unsigned char* sK, int f) -> u32x4_t {
      const int s = f / KB, kb = f % KB;
      const unsigned char* kb0 = sK + kbase[s & 3] + 256 * (s >> 2);
      return *reinterpret_cast<const u32x4_t*>(kb0 + kb * 16 * S::ROW_BYTES);
    };
    auto gemm_s_body = [&](f32x4_t (&sacc)[KB][RB], const unsigned char* sK) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) sacc[kb][rb] = f32x4_t{0, 0, 0, 0};
      u32x4_t ka[KA_AHEAD];
#pragma unroll
      for (int f = 0; f < KA_AHEAD; ++f) ka[f] = kread(sK, f);
#pragma unroll
      for (int f = 0; f < NKF; ++f) {
        const u32x4_t cur = ka[f % KA_AHEAD];
        if (f + KA_AHEAD < NKF) ka[f % KA_AHEAD] = kread(sK, f + KA_AHEAD);
        const int s = f / KB, kb = f % KB;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          sacc[kb][rb] = mfma16x16x32(as_bf16x8(cur), as_bf16x8(qr[rb][s]), sacc[kb][rb]);
      }
    };
    auto gemm_s = [&](f32x4_t (&sacc)[KB][RB], const unsigned char* sK) {
      gemm_s_body(sacc, sK);
      __builtin_amdgcn_sched_group_barrier(0x100, KA_AHEAD, 0);
#pragma unroll
      for (int f = 0; f < NKF - KA_AHEAD; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, RB, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, RB * KA_AHEAD, 0);
    };

    // masking of tile t (only tiles that cross the item's end or a row's
    // causal limit) and this lane's running maximum of the raw scores
    float lmax_all[RB];
    auto mask_track = [&](f32x4_t (&sacc)[KB][RB], int t) {
      const int t0 = t * KT;
      if (t0 + KT > nkeys || t0 + KT - 1 > wave_min) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = t0 + kb * 16 + lg * 4 + i;
              if (!(key < nkeys && key <= qlim[rb])) sacc[kb][rb][i] = NEG_INF;
            }
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
          lmax_all[rb] = fmaxf(lmax_all[rb], fmaxf(fmaxf(sacc[kb][rb][0], sacc[kb][rb][1]),
                                                   fmaxf(sacc[kb][rb][2], sacc[kb][rb][3])));
    };

    // probabilities exp2(s - m) of tile t against the row's reference maximum,
    // as the B operand of O^T += V^T P^T: keys {t2*32 + 4 lg..+3,
    // t2*32 + 16 + 4 lg..+3} of row (rb, l16)
    float m_ref[RB], l_part[RB];
    auto exp_pack = [&](f32x4_t (&sacc)[KB][RB], u32x4_t (&pb)[RB][T2]) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][rb][i], a.scale_log2, -m_ref[rb]));
            sacc[kb][rb][i] = p;
            sum += p;
          }
        l_part[rb] += sum;
#pragma unroll
        for (int t2 = 0; t2 < T2; ++t2) {
          pb[rb][t2].x = pack2bf(sacc[2 * t2][rb][0], sacc[2 * t2][rb][1]);
          pb[rb][t2].y = pack2bf(sacc[2 * t2][rb][2], sacc[2 * t2][rb][3]);
          pb[rb][t2].z = pack2bf(sacc[2 * t2 + 1][rb][0], sacc[2 * t2 + 1][rb][1]);
          pb[rb][t2].w = pack2bf(sacc[2 * t2 + 1][rb][2], sacc[2 * t2 + 1][rb][3]);
        }
      }
    };

    // O^T += V^T P^T; transposing LDS reads: lane i of a 16-lane group reads
    // row K0 + i/4, dims 4 (i%4).. of a d-block and receives dim (block + i)
    // of rows K0..K0+3.  The reads run VA_AHEAD fragments ahead of the MFMAs.
    f32x4_t o[DB][RB];
    auto gemm_pv = [&](const u32x4_t (&pb)[RB][T2], const unsigned char* sV) {
      constexpr int NF = DB * T2;         // fragments (db, t2)
      constexpr int VA_AHEAD = 4;
      u32x4_t va[VA_AHEAD];
      auto vread = [&](int f) -> u32x4_t {
        const int db = f / T2, t2 = f % T2;
        s16x4_t part[2];
#pragma unroll
        for (int hlf = 0; hlf < 2; ++hlf) {
          const unsigned char* p = sV + vbase[db & 7] + (t2 * 32 + hlf * 16) * S::ROW_BYTES + 256 * (db >> 3);
          part[hlf] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
        }
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
        const int db = f / T2, t2 = f % T2;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          o[db][rb] = mfma16x16x32(as_bf16x8(cur), as_bf16x8(pb[rb][t2]), o[db][rb]);
      }
      // keep VA_AHEAD fragments of reads in flight ahead of the MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * VA_AHEAD, 0);
#pragma unroll
      for (int f = 0; f < NF - VA_AHEAD; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, RB, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, RB * VA_AHEAD, 0);
    };

    // One step: S(t+1) on the MFMA units while the VALU turns S(t) into
    // probabilities, then O += V(t) P(t).  K(t+2) and V(t+1) stream into the
    // buffers that K(t) and V(t-1) left.
    auto step = [&](int t, f32x4_t (&cur)[KB][RB], f32x4_t (&nxt)[KB][RB]) {
      if (t + 2 < ntiles) issue(kp, t + 2, kbuf[t & 1], true);
      if (t + 1 < ntiles) issue(vp, t + 1, vbuf[(t + 1) & 1], false);
      const bool act = t * KT <= wave_lim;
      const bool act_n = t + 1 < ntiles && (t + 1) * KT <= wave_lim;
      u32x4_t pb[RB][T2];
      if (act) mask_track(cur, t);
      if (act && act_n) {
        gemm_s_body(nxt, kbuf[(t + 1) & 1]);
        exp_pack(cur, pb);
        // the VALU work of exp_pack between the MFMAs of S(t+1)
        __builtin_amdgcn_sched_group_barrier(0x100, KA_AHEAD, 0);
#pragma unroll
        for (int f = 0; f < NKF - KA_AHEAD; ++f) {
          __builtin_amdgcn_sched_group_barrier(0x008, RB, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2 * RB, 0);
        }
#pragma unroll
        for (int f = 0; f < KA_AHEAD; ++f) {
          __builtin_amdgcn_sched_group_barrier(0x008, RB, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2 * RB, 0);
        }
      } else if (act) {
        exp_pack(cur, pb);
      } else if (act_n) {
        gemm_s(nxt, kbuf[(t + 1) & 1]);
      }
      if (act) gemm_pv(pb, vbuf[t & 1]);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    };

    // Each row's probabilities are taken against a reference maximum fixed
    // from the first tile; no accumulator is rescaled in the loop.  A key
    // more than OVERFLOW_LOG2 above the reference (probabilities past 2^64)
    // restarts the item with the rows' true maxima as reference.
    bool forced = false;
    for (int pass = 0; pass < 2; ++pass) {
      issue(kp, 0, kbuf[0], true);
      issue(vp, 0, vbuf[0], false);
      if (ntiles > 1) issue(kp, 1, kbuf[1], true);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) o[db][rb] = f32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        l_part[rb] = 0.f;
        lmax_all[rb] = NEG_INF;
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      f32x4_t sA[KB][RB], sB[KB][RB];
      gemm_s(sA, kbuf[0]);
      mask_track(sA, 0);
      if (!forced) {
        // reference maximum: the row's maximum over the first tile (key 0 of
        // an item is visible to every row, so it is finite)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          float mx = lmax_all[rb];
          mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
          mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
          m_ref[rb] = (mx == NEG_INF) ? 0.f : mx * a.scale_log2;
        }
      }
      for (int t = 0; t < ntiles; t += 2) {
        step(t, sA, sB);
        if (t + 1 < ntiles) step(t + 1, sB, sA);
      }
      // the rows' true maxima; restart if any exceeds its reference by too much
      bool over = false;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float mx = lmax_all[rb];
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        mx = (mx == NEG_INF) ? 0.f : mx * a.scale_log2;
        over |= mx > m_ref[rb] + OVERFLOW_LOG2;
        if (!forced) lmax_all[rb] = mx;     // kept for a second pass
      }
      if (forced || !__syncthreads_or(over ? 1 : 0)) break;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) m_ref[rb] = lmax_all[rb];
      forced = true;
    }

    // epilogue: normalise, write the partial (or the local window) and its LSE
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float l = l_part[rb];
      l += __shfl_xor(l, 16, 64);
      l += __shfl_xor(l, 32, 64);
      const int R = wave * 16 * RB + rb * 16 + l16;
      const int i = R / G, j = R % G;
      if (qidx_r[rb] < 0) continue;
      const float inv = (l > 0.f) ? 1.0f / l : 0.f;
      const float lse = (l > 0.f) ? (m_ref[rb] + log2f(l)) * 0.69314718055994531f : NEG_INF;
      bf16_t* dst;
      float* ldst;
      if (local) {
        dst = a.local_o + (int64_t)qidx_r[rb] * a.lo_sq + (int64_t)(h * G + j) * a.lo_sh;
        ldst = a.local_lse ? a.local_lse + (int64_t)qidx_r[rb] * a.Hq + h * G + j : nullptr;
      } else {
        dst = a.part_o + ((entry0 + i) * G + j) * D;
        ldst = a.part_lse + (entry0 + i) * G + j;
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        u32x2_t w;
        w.x = pack2bf(o[db][rb][0] * inv, o[db][rb][1] * inv);
        w.y = pack2bf(o[db][rb][2] * inv, o[db][rb][3] * inv);
        *reinterpret_cast<u32x2_t*>(dst + db * 16 + lg * 4) = w;
      }
      if (lg == 0 && ldst) *ldst = lse;
    }
  }
}


// S6: per (query, KV head), one wave.  Seeds with the local window, then
// folds the query's cluster partials in cluster order (query-major order of
// the reference's entries).  Each lane owns E = G*D/64 consecutive values of
// one head.
template <int D, int G>
__global__ __launch_bounds__(256) void combine_kernel(
    const int32_t* __restrict__ qmask, const int32_t* __restrict__ nvis,
    const int32_t* __restrict__ rev_indptr, const int32_t* __restrict__ qrank,
    const bf16_t* __restrict__ part_o, const float* __restrict__ part_lse,
    const bf16_t* __restrict__ local_o, int64_t lo_sq, int64_t lo_sh,
    const float* __restrict__ local_lse, bf16_t* __restrict__ out, int64_t out_sq, int64_t out_sh,
    float* __restrict__ out_lse, int Qc, int Hkv, int C) {
  constexpr int E = G * D / 64;
  static_assert(E >= 1 && D % E == 0, "lane share");
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gw >= (int64_t)Qc * Hkv) return;
  const int qi = (int)(gw / Hkv), h = (int)(gw % Hkv);
  const int j = (lane * E) / D, d0 = (lane * E) % D;
  const int Hq = Hkv * G;
  float acc[E];
  float m = local_lse[(int64_t)qi * Hq + h * G + j];
  {
    const bf16_t* src = local_o + (int64_t)qi * lo_sq + (int64_t)(h * G + j) * lo_sh + d0;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = bf2f(src[e]);
  }
  float den = 1.f;
  const int W = C / 32;
  const int32_t* qm = qmask + ((int64_t)qi * Hkv + h) * W;
  const int32_t* qr = qrank + ((int64_t)qi * Hkv + h) * C;
  for (int w = 0; w < W; ++w) {
    uint32_t bits = (uint32_t)qm[w];
    while (bits) {
      const int b = __builtin_ctz(bits);
      bits &= bits - 1;
      const int c = w * 32 + b;
      if (nvis[h * C + c] <= 0) continue;
      const int64_t entry = (int64_t)rev_indptr[h * C + c] + qr[c];
      const float le = part_lse[entry * G + j];
      const float nm = fmaxf(m, le);
      const float sc = expf(m - nm);
      const float wt = expf(le - nm);
      const bf16_t* src = part_o + (entry * G + j) * D + d0;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = acc[e] * sc + bf2f(src[e]) * wt;
      den = den * sc + wt;
      m = nm;
    }
  }
  const float inv = 1.0f / fmaxf(den, 1e-30f);
  bf16_t* dst = out + (int64_t)qi * out_sq + (int64_t)(h * G + j) * out_sh + d0;
#pragma unroll
  for (int e = 0; e < E; ++e) dst[e] = f2bf(acc[e] * inv);
  if (out_lse && (lane * E) % D == 0) out_lse[(int64_t)qi * Hq + h * G + j] = m + logf(den);
}

template <int D, int G>
int launch_attn(const AttnArgs& a, int grid, hipStream_t stream) {
  const size_t lds = AttnTileShape<D>::LDS_BYTES;
  static bool configured = false;
  if (!configured) {
    hipFuncSetAttribute((const void*)attn_items_kernel<D, G, PREFILL_RB>,
                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    configured = true;
  }
  static int auto_grid = 0;
  if (grid <= 0) {
    if (!auto_grid) {
      int dev = 0, cus = 0, occ = 0;
      hipGetDevice(&dev);
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)attn_items_kernel<D, G, PREFILL_RB>,
                                                   256, lds);
      auto_grid = (cus > 0 ? cus : 256) * (occ > 0 ? occ : 1);
    }
    grid = auto_grid;
  }
  hipLaunchKernelGGL((attn_items_kernel<D, G, PREFILL_RB>), dim3(grid), dim3(256), lds, stream, a);
  return SBSA_OK;
}

template <int D, int G>
int launch_combine(const int32_t* qmask, const int32_t* nvis, const int32_t* rev_indptr,
                   const int32_t* qrank, const bf16_t* part_o, const float* part_lse,
                   const bf16_t* local_o, int64_t lo_sq, int64_t lo_sh, const float* local_lse,
                   bf16_t* out, int64_t out_sq, int64_t out_sh, float* out_lse, int Qc, int Hkv,
                   int C, hipStream_t stream) {
  int64_t waves = (int64_t)Qc * Hkv;
  hipLaunchKernelGGL((combine_kernel<D, G>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     stream, qmask, nvis, rev_indptr, qrank, part_o, part_lse, local_o, lo_sq,
                     lo_sh, local_lse, out, out_sq, out_sh, out_lse, Qc, Hkv, C);
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
                     float* out_lse, int Qc, int Hkv, int C, hipStream_t stream) {
  SBSA_DISPATCH_DG(D, G, launch_combine, qmask, nvis, rev_indptr, qrank, part_o, part_lse, local_o,
                   lo_sq, lo_sh, local_lse, out, out_sq, out_sh, out_lse, Qc, Hkv, C, stream);
}

}  // namespace

extern "C" {

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
  AttnArgs a;
  a.q = (const bf16_t*)q;
  a.q_sq = q_sq;
  a.q_sh = q_sh;
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
  a.items = (const int4*)items;
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
  a.chunk_start = chunk_start;
  a.wstart = wstart;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
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
                         int num_clusters, hipStream_t stream) {
  if (!qmask || !nvis || !rev_indptr || !qrank || !local_o || !local_lse || !out) return SBSA_ERR_ARG;
  if (num_kv_heads < 1 || num_q_heads % num_kv_heads || num_clusters % 32) return SBSA_ERR_ARG;
  if (num_queries == 0) return SBSA_OK;
  int rc = combine_dispatch(dim, num_q_heads / num_kv_heads, qmask, nvis, rev_indptr, qrank,
                            (const bf16_t*)part_o, part_lse, (const bf16_t*)local_o, lo_sq, lo_sh,
                            local_lse, (bf16_t*)out, out_sq, out_sh, out_lse, num_queries,
                            num_kv_heads, num_clusters, stream);
  if (rc) return rc;
  SBSA_CHECK_LAUNCH();
  return SBSA_OK;
}

}  // extern "C"
