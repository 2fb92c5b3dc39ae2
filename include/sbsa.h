/*
 * libsbsa: the C ABI of the MI355X (gfx950) semantic block-sparse attention path.
 *
 * Every entry point takes raw device pointers, element strides (int64) and a
 * hipStream_t, allocates nothing, and returns an int status (SBSA_OK or one of
 * the SBSA_ERR_* codes below; nothing is thrown across the ABI).  bf16 tensors
 * are passed as void* and hold IEEE bfloat16 bit patterns.  All launches go to
 * the given stream; no entry point synchronises the device.
 *
 * Each declaration names the reference interface it replaces
 * (pfnet-research/semantic-block-sparse-attention, file:line).
 */
#ifndef SBSA_H
#define SBSA_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SBSA_OK 0
#define SBSA_ERR_ARG 1          /* a null pointer, a bad shape or stride          */
#define SBSA_ERR_UNSUPPORTED 2  /* a shape outside what the kernels are built for */
#define SBSA_ERR_LAUNCH 3       /* the HIP runtime refused a launch               */
#define SBSA_ERR_CAPACITY 4     /* a caller buffer is smaller than the bound      */

/* ABI version of this header (bumped on any signature change). */
int sbsa_abi_version(void);

/* ---- S0: routing normalisation -------------------------------------------
 * Replaces trivial_router_vectors (semblo/vllm_plugin/trivial_router.py:48-75):
 * per row and per factor, normalise in fp32, round to bf16, renormalise,
 * round again.  x and out are [rows, dim] bf16 with row strides ld_x, ld_out. */
int sbsa_route_vectors(const void* x, int64_t rows, int64_t ld_x, int dim, int factors,
                       void* out, int64_t ld_out, hipStream_t stream);

/* ---- S1: block build -------------------------------------------------------
 * Key routing space of one KV head: the identity key router in whole mode
 * (semblo/vllm_plugin/routing_map.py:35-64) followed by routing_space and the
 * k-means fit space (semblo/inference/flat_index.py:144-166, 300-302).
 * k is [length] rows of dim bf16 at stride ld_k: pre-RoPE keys when
 * router_pass is 1, the key router's output (ProductPostingIndex.build's
 * product_keys) when 0.  Writes the unit rows in fp32 and bf16, both
 * [length, dim] contiguous. */
int sbsa_key_space(const void* k, int64_t length, int64_t ld_k, int dim, int router_pass,
                   float* space_f32, void* space_bf16, hipStream_t stream);

/* Nearest centroid by bf16 similarity, the GEMM output rounded to bf16 and the
 * first maximum taken: replaces _argmax_sim_chunked / assign_flat_buckets
 * (semblo/inference/flat_index.py:356-383).  Rows are x_bf16[row_index[i]]
 * (or x_bf16[i] when row_index is null); cent_bf16 is [num_clusters, dim].
 * dim in {64, 128, 256}. */
int sbsa_kmeans_assign(const void* x_bf16, int64_t ld_x, const int32_t* row_index, int64_t n,
                       const void* cent_bf16, int num_clusters, int dim, int32_t* assign,
                       hipStream_t stream);

/* Deterministic per-cluster fp32 sums and counts of the sample rows (the sum
 * order depends on the assignment only): replaces _segment_sum / torch.bincount
 * in fit_flat_codebook (semblo/inference/flat_index.py:87-141, 268-272).
 * sums [C, dim], counts [C]; C <= 1024; dim and ld_x multiples of 4 and x
 * 16-byte aligned (SBSA_ERR_UNSUPPORTED otherwise).  member_bits is device scratch of at
 * least sbsa_kmeans_member_bits_bytes(n, C) bytes, 16-byte aligned (one bitmap
 * of the rows per cluster; overwritten, need not be cleared). */
size_t sbsa_kmeans_member_bits_bytes(int64_t n, int num_clusters);
int sbsa_kmeans_update(const float* x, int64_t ld_x, const int32_t* row_index, int64_t n,
                       const int32_t* assign, int num_clusters, int dim, float* sums,
                       int32_t* counts, uint32_t* member_bits, size_t member_bits_bytes,
                       hipStream_t stream);

/* Centroid step of fit_flat_codebook (semblo/inference/flat_index.py:255-289)
 * and the descriptor of _build_flat (semblo/vllm_plugin/state.py:877-886).
 *   mode 0: cent = x[row_index[src_rows[c]]]  (random init)
 *   mode 1: cent = normalize(sums / counts); src_rows[c] >= 0 restarts an
 *           empty cluster on that sample row
 *   mode 2: cent_bf16 as [2, C, dim/2] = bf16(normalize(sums))  (descriptor)
 * cent_f32 [C, dim] and cent_bf16 [C, dim] (modes 0, 1). */
int sbsa_kmeans_centroids(int mode, const float* sums, const int32_t* counts,
                          const int32_t* src_rows, const float* x, int64_t ld_x,
                          const int32_t* row_index, int num_clusters, int dim, float* cent_f32,
                          void* cent_bf16, hipStream_t stream);

/* Iterations it0 .. it1-1 of fit_flat_codebook's k-means loop
 * (semblo/inference/flat_index.py:264-289) in one call: each is
 * sbsa_kmeans_assign, sbsa_kmeans_update into sums_hist[it] [C, dim] and
 * counts_hist[it] [C], and the centroid step.  The rows are x (bf16 for the
 * assignment, fp32 for the sums, both with row stride ld_x) at row_index [n];
 * assign [n] and member_bits (as for sbsa_kmeans_update) are scratch.
 *   restart_rows null: no restarts (sbsa_kmeans_centroids mode 1 with
 *     no_restart, C entries of -1); an iteration that leaves a cluster empty
 *     is for the caller to find in counts_hist and redo.
 *   restart_rows [restart_draws, C]: the k-th iteration that leaves clusters
 *     empty (k < restart_draws) restarts them on sample rows restart_rows[k][0..],
 *     in cluster order -- the k-th restart draw the reference makes
 *     (flat_index.py:277-283), made ahead by the caller.  restart_flags
 *     [it1 + 1]: restart_flags[it0] must hold the number of iterations before
 *     it0 that left a cluster empty (0 for it0 = 0); iteration it writes
 *     restart_flags[it + 1].  Later empty iterations are not restarted: the
 *     caller finds them in counts_hist and redoes them. */
int sbsa_kmeans_iterate(const void* x_bf16, const float* x_f32, int64_t ld_x,
                        const int32_t* row_index, int64_t n, int num_clusters, int dim,
                        int32_t* assign, float* sums_hist, int32_t* counts_hist,
                        const int32_t* no_restart, const int32_t* restart_rows,
                        int restart_draws, int32_t* restart_flags, float* cent_f32,
                        void* cent_bf16, uint32_t* member_bits, size_t member_bits_bytes,
                        int it0, int it1, hipStream_t stream);

/* Stable counting sort of positions by cluster into page-aligned runs:
 * replaces argsort/bincount + _page_align_order
 * (semblo/vllm_plugin/state.py:850-866, 44-84).  Writes sizes [C], indptr
 * [C+1] (padded), posting [posting_cap] (padding rows repeat the first sorted
 * key's position, as do rows past the total), inverse [length] (position ->
 * padded row) and the padded total (device int).  num_clusters <= 1024. */
size_t sbsa_bucket_layout_workspace_bytes(int64_t length, int num_clusters);
int sbsa_bucket_layout(const int32_t* assign, int64_t length, int num_clusters, int align,
                       int32_t* sizes, int32_t* indptr, int32_t* posting, int64_t posting_cap,
                       int32_t* inverse, int32_t* total_out, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* ---- S1b: packed K/V --------------------------------------------------------
 * Replaces ProductPostingIndex.pack_prompt_kv (semblo/vllm_plugin/state.py:950-997):
 * packed [2, packed_len, Hkv, dim] gathered through posting [Hkv, width];
 * rows >= width are zero. */
int sbsa_pack_kv(const void* key, const void* value, int64_t stride_tok, int64_t stride_head,
                 int num_kv_heads, int dim, const int32_t* posting, int64_t width,
                 int64_t packed_len, void* packed, hipStream_t stream);

/* ---- S2 + S3: scoring and budget selection ----------------------------------
 * Replaces theta_select_bitmask_flat (semblo/vllm_plugin/fused_select.py:806-919)
 * = flat_mixture_scores_qtiled (:1250-1357) + _streaming_select_kernel RESIDENT
 * (:551-647).  vectors [Q, Hq, dim] bf16 (strides v_sq, v_sh), logmix [Q, Hq]
 * fp32 or null, codebooks [Hkv, 2, C, dim/2] bf16, sizes[b*s_nb + h*s_h + c]
 * for union block b = q / g_union (s_nb may be 0).  Outputs (each optional):
 * bitmask [NB, Hkv, C/32] (OR-ed into; pre-zero it), qmask [Q, Hkv, C/32],
 * counts and tokens [Q, Hkv], prob_out [Q, Hkv, C], theta_out [Q, Hkv].
 * sink_tokens > 0 holds cluster 0 out of the search and selects it
 * (fused_prefill.py:202-216).  C a multiple of 64, <= 1024. */
int sbsa_score_select(const void* vectors, int64_t v_sq, int64_t v_sh, const float* logmix,
                      const void* codebooks, const int32_t* sizes, int64_t s_nb, int64_t s_h,
                      int num_queries, int num_q_heads, int num_kv_heads, int num_clusters,
                      int dim, int g_union, float inv_temperature, float beta,
                      float target_tokens, int iters, int sink_tokens, int32_t* bitmask,
                      int32_t* qmask, int32_t* counts, int32_t* tokens, float* prob_out,
                      float* theta_out, hipStream_t stream);

/* ---- S3c: causal snapshot ----------------------------------------------------
 * Replaces CausalSnapshot.advance (semblo/vllm_plugin/fused_prefill.py:126-135):
 * out[h, c] = |{rows of cluster c's run with position < pos_limit}|. */
int sbsa_causal_sizes(const int32_t* posting, int64_t width, const int32_t* indptr,
                      const int32_t* sizes, int num_kv_heads, int num_clusters,
                      int64_t pos_limit, int32_t* out, hipStream_t stream);

/* ---- S4: reverse index ---------------------------------------------------------
 * Replaces build_reverse_index (semblo/vllm_plugin/kv_outer.py:254-329): for
 * each (head, cluster) with nvis > 0, the ascending query ids whose qmask has
 * it.  rev_counts [Hkv*C], rev_indptr [Hkv*C + 1], nnz (device int64), qvals
 * [qvals_cap >= Q*Hkv*C], qrank [Q, Hkv, C] (rank of q in the cluster's list,
 * written where selected).  Deterministic, no atomics. */
int sbsa_reverse_index(const int32_t* qmask, int num_queries, int num_kv_heads, int num_clusters,
                       const int32_t* nvis, int32_t* rev_counts, int32_t* rev_indptr,
                       int64_t* nnz, int32_t* qvals, int64_t qvals_cap, int32_t* qrank,
                       hipStream_t stream);

/* (query, head) rows of one prefill work item: the host tiles each (head,
 * cluster) query list into items of sbsa_prefill_item_rows() / G queries.
 * No counterpart in the reference (its FA3 calls take whole lists). */
int sbsa_prefill_item_rows(void);

/* ---- S5: KV-outer prefill attention ---------------------------------------------
 * The work list replacing the per-(cluster, KV head) FA3 varlen calls and the
 * local-window call of kv_outer_attention (semblo/vllm_plugin/kv_outer.py:661-753).
 * items are 32-byte records {head, cluster or -1 (local window), first query
 * slot, count, visible rows nvis[h, c], first partial slot rev_indptr[h*C+c] +
 * first query slot, first packed row indptr[h, c], 0}, so the attention
 * kernel resolves an item with one load; indptr [Hkv, C+1], nvis [Hkv, C] and
 * rev_indptr [Hkv*C + 1] are those later passed to sbsa_prefill_attend (any
 * valid arrays when no cluster has queries).  Items are grouped in one segment
 * per XCD (the query tiles of a KV head's window, and those of one cluster,
 * share an XCD and its L2), window items first (longest first), then cluster
 * items, longest cluster first; queue (int32[32]) receives the segments' sizes
 * and offsets and zeroed counters in ints 0-23, and in int 24 an overflow
 * flag: with partials_cap > 0 and more partial entries than that
 * (rev_indptr[Hkv*C] > partials_cap) the list is empty and the flag 1, so the
 * attention writes nothing and sbsa_prefill_combine (given the flag) skips the
 * chunk, which the caller runs again with a partial buffer of its exact size
 * (the reference reads the count instead, kv_outer.py:592-613).
 * queries_per_item = 128 / (Hq/Hkv). */
int64_t sbsa_prefill_items_bound(int64_t nnz, int num_queries, int num_kv_heads,
                                 int num_clusters, int queries_per_item);
int sbsa_prefill_items(const int32_t* rev_counts, int num_kv_heads, int num_clusters,
                       int num_queries, int queries_per_item, int has_local,
                       const int32_t* indptr, const int32_t* nvis, const int32_t* rev_indptr,
                       void* items, int64_t items_cap, int64_t partials_cap, int32_t* queue,
                       hipStream_t stream);

/* Attention over the work list (kv_outer.py:482-816; dense chunks:
 * fused_prefill.py:155-189).  q [Qc, Hq, dim] (strides q_sq, q_sh); packed
 * [2, packed_len, Hkv, dim]; k_orig/v_orig the prompt-order window whose row 0
 * is position wstart ([>= chunk_end + 1 - wstart, Hkv, dim] at strides
 * (o_st, o_sh)); a cluster item reads the first nvis[h, c] rows of the run at
 * indptr[h, c]; a local item reads positions wstart..(its last query)
 * causally.  Cluster partials: part_o [nnz, G, dim] bf16, part_lse [nnz, G];
 * the local window: local_o [Qc, Hq, dim] (strides lo_sq, lo_sh) and
 * local_lse [Qc, Hq] (null for a dense chunk, whose local_o is the output).
 * grid: persistent blocks (<= 0: as many as the device holds at once).  dim in {128, 256}, Hq/Hkv
 * in {1, 2, 4, 8}. */
int sbsa_prefill_attend(const void* q, int64_t q_sq, int64_t q_sh, int num_queries,
                        int num_q_heads, int num_kv_heads, int dim, const void* packed,
                        int64_t packed_len, const void* k_orig, const void* v_orig, int64_t o_st,
                        int64_t o_sh, const int32_t* indptr, const int32_t* nvis, int num_clusters,
                        const int32_t* rev_indptr, const int32_t* qvals, const void* items,
                        int32_t* queue, void* part_o, float* part_lse,
                        void* local_o, int64_t lo_sq, int64_t lo_sh, float* local_lse,
                        int64_t chunk_start, int64_t wstart, float sm_scale, int grid,
                        hipStream_t stream);

/* ---- S6: combine ----------------------------------------------------------------
 * Replaces combine_partials / _combine_grouped_kernel
 * (semblo/vllm_plugin/kv_outer.py:370-479): per (query, KV head), seeds with
 * the local window and folds the partials of the query's clusters in cluster
 * order by online log-sum-exp; out [Qc, Hq, dim] bf16, out_lse [Qc, Hq] or null.
 * skip (null, or the work list's overflow flag, queue + 24): a nonzero flag
 * leaves out untouched. */
int sbsa_prefill_combine(const int32_t* qmask, const int32_t* nvis, const int32_t* rev_indptr,
                         const int32_t* qrank, const void* part_o, const float* part_lse,
                         const void* local_o, int64_t lo_sq, int64_t lo_sh, const float* local_lse,
                         void* out, int64_t out_sq, int64_t out_sh, float* out_lse,
                         int num_queries, int num_q_heads, int num_kv_heads, int dim,
                         int num_clusters, const int32_t* skip, hipStream_t stream);

/* ---- S7-S9: decode step ------------------------------------------------------------
 * Replaces fused_decode_step (semblo/vllm_plugin/fused_decode.py:393-521): the
 * suffix write (if k_new/v_new are given), the routing vector, selection
 * against the full bucket sizes with CSR emission, the split attention over
 * the selected packed rows and the suffix store [2, suffix_nblk, suffix_block,
 * Hkv, dim] (through table, positions prompt_len..*pos), and the LSE merge
 * into out [Hq, dim] (row stride out_sh) and out_lse [Hq] (natural log, or
 * null).  q_pre holds pre-RoPE queries to route (router_pass 1) or routing
 * vectors already (router_pass 0).  pos is a device int.  The suffix holds at
 * most 16*max_tiles positions from prompt_len (max_tiles 0: no suffix), and
 * table maps logical blocks prompt_len/suffix_block through
 * (prompt_len + 16*max_tiles - 1)/suffix_block.  prompt_len_dev (optional,
 * int32 [1]): the prompt length read on the device instead of prompt_len, so
 * that a captured step follows a suffix flush (the arena's prompt_length_t,
 * semblo/vllm_plugin/arena.py:118-124, suffix_flush.py:230).  kpre_new /
 * suffix_kpre (optional, [Hkv, dim] at kn_sh / [suffix_nblk, suffix_block,
 * Hkv, dim]): the token's pre-RoPE key is stored beside its K/V, for the
 * flush's routing (arena.py:138-141).  num_splits + suffix_splits
 * <= 512; suffix_block and suffix_nblk at least 1 (else SBSA_ERR_ARG).  No host reads, no allocation: capturable in a HIP graph.  csr_out (optional) receives [rstart, rlen, rcum] ([3, Hkv, C])
 * then rcount [Hkv] and rtokens [Hkv]; of each head's C entries only the first
 * rcount[h] are written by the step (the rest keep earlier contents). */
size_t sbsa_decode_workspace_bytes(int num_q_heads, int num_kv_heads, int num_clusters, int dim,
                                   int num_splits, int suffix_splits);
int sbsa_decode_step(const void* q_post, int64_t q_sh, const void* q_pre, int64_t qp_sh,
                     int router_pass, const void* k_new, const void* v_new, int64_t kn_sh, const int32_t* pos,
                     const void* codebooks, const int32_t* sizes, const int32_t* indptr,
                     const void* packed, int64_t packed_len, void* suffix_kv, int64_t suffix_nblk,
                     int suffix_block, const int32_t* table, int64_t prompt_len, int max_tiles,
                     const int32_t* prompt_len_dev, const void* kpre_new, void* suffix_kpre,
                     int num_q_heads, int num_kv_heads, int num_clusters, int dim,
                     float inv_temperature, float beta, float target_tokens, int iters,
                     int sink_tokens, float sm_scale, int num_splits, int suffix_splits,
                     void* workspace, size_t workspace_bytes, void* out, int64_t out_sh,
                     float* out_lse, int32_t* csr_out, hipStream_t stream);

/* The decode step with no allocation and no workspace argument.  This entry point
 * has no counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as sbsa_decode_step minus the
 * workspace: the step's scratch (the selection's CSR and the splits' partials) is
 * a static device array of the library, sbsa_decode_scratch_bytes() bytes per GPU,
 * held until the process ends; shapes whose sbsa_decode_workspace_bytes exceeds it
 * return SBSA_ERR_CAPACITY.  Its address is looked up once per device, on the
 * first call with that device current (make that call before a capture).  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams, or two processes' threads into one library) race. */
size_t sbsa_decode_scratch_bytes(void);
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
                             hipStream_t stream);

/* ---- S10: token-order streamed prefill (the store behind the fixed clusters) -----
 * Nearest cluster of each new key: replaces _nearest_cluster
 * (semblo/vllm_plugin/suffix_flush.py:154-170) applied to routing_space of the
 * key router's output, as TokenOuterPrefillSession._append does
 * (semblo/vllm_plugin/token_outer_prefill.py:339-348).  k [n, Hkv, dim] bf16 at
 * strides (stride_tok, stride_head): pre-RoPE keys (router_pass 1) or the
 * router's output (0).  Cosine in fp32 against cat(codebooks[h, 0, c],
 * codebooks[h, 1, c]); all-zero descriptors are never chosen; the first of
 * equal maxima wins.  ids [Hkv, n] int32.  dim in {128, 256}, C a multiple
 * of 64 up to 1024. */
int sbsa_nearest_cluster(const void* k, int64_t n, int64_t stride_tok, int64_t stride_head,
                         int num_kv_heads, int dim, int router_pass, const void* codebooks,
                         int num_clusters, int32_t* ids, hipStream_t stream);

/* Destination rows of a slice's keys: replaces append_rows
 * (semblo/vllm_plugin/token_outer_prefill.py:66-87).  ids [Hkv, n] (cluster of
 * each key in position order), indptr [Hkv, C+1], sizes [Hkv, C] (keys
 * already in each run).  rows[h, i] = indptr[h, c] + sizes[h, c] + (earlier
 * keys of the slice in c); counts [Hkv, C].  reserve [Hkv, C] (optional):
 * overflow[h] (optional) gets bit 0 when sizes + counts exceeds it for some
 * cluster, the test of _append (token_outer_prefill.py:350-352); bit 1 flags
 * an id outside [0, C) (its row is -1).  Reads only: sizes are not advanced. */
int sbsa_append_rows(const int32_t* ids, int64_t n, int num_kv_heads, int num_clusters,
                     const int32_t* indptr, const int32_t* sizes, const int32_t* reserve,
                     int32_t* rows, int32_t* counts, int32_t* overflow, hipStream_t stream);

/* The writes of _append (semblo/vllm_plugin/token_outer_prefill.py:353-364):
 * packed[t, rows[h, i], h] = (t ? value : key)[i, h], posting[h, rows[h, i]] =
 * first_position + i, inverse[h, first_position + i] = rows[h, i];
 * sizes_before (optional) = sizes, then sizes += counts.  key/value [n, Hkv,
 * dim] at (stride_tok, stride_head); packed [2, packed_len, Hkv, dim];
 * posting [Hkv, posting_width]; inverse [Hkv, inverse_len]. */
int sbsa_append_kv(const void* key, const void* value, int64_t stride_tok, int64_t stride_head,
                   int64_t n, int num_kv_heads, int dim, const int32_t* rows, int64_t first_position,
                   void* packed, int64_t packed_len, int32_t* posting, int64_t posting_width,
                   int32_t* inverse, int64_t inverse_len, int32_t* sizes, const int32_t* counts,
                   int num_clusters, int32_t* sizes_before, hipStream_t stream);

/* Moves positions 0..n-1 from runs starting at old_indptr to the same offsets
 * in runs starting at new_indptr: the row moves of _fit_and_pack
 * (semblo/vllm_plugin/token_outer_prefill.py:284-312) and _repack (:366-392).
 * old_rows [Hkv, >= n] (row stride old_rows_ld) is each position's row in the
 * old layout; its cluster is the last b with old_indptr[b] <= row.  key/value
 * [n, Hkv, dim] hold the keys in position order (the staged prompt at the
 * fit; sbsa_gather_rows' output at a repack).  Writes inverse [Hkv, >= n]
 * (row stride inverse_ld; must not overlap old_rows), posting[h, new row] =
 * position and the packed rows. */
int sbsa_relayout_runs(const void* key, const void* value, int64_t stride_tok, int64_t stride_head,
                       int64_t n, int num_kv_heads, int dim, const int32_t* old_rows, int64_t old_rows_ld,
                       const int32_t* old_indptr, const int32_t* new_indptr, int num_clusters,
                       void* packed, int64_t packed_len, int32_t* posting, int64_t posting_width,
                       int32_t* inverse, int64_t inverse_ld, hipStream_t stream);

/* Positions first..first+n-1 back in prompt order through the inverse map:
 * (t ? value_out : key_out)[i, h] = packed[t, inverse[h, first + i], h].  The
 * gather of _repack (semblo/vllm_plugin/token_outer_prefill.py:380-383) and of
 * the dense chunks that follow the fit ("read densely by the fused body through
 * the inverse permutation", token_outer_prefill.py:155-159). */
int sbsa_gather_rows(const void* packed, int64_t packed_len, int num_kv_heads, int dim,
                     const int32_t* inverse, int64_t inverse_ld, int64_t first, int64_t n, void* key_out,
                     void* value_out, int64_t stride_tok, int64_t stride_head, hipStream_t stream);

/* The row moves of _repack (semblo/vllm_plugin/token_outer_prefill.py:366-392)
 * into the other buffer of a double-buffered store, in one pass:
 * dst_packed[t, new row, h] = src_packed[t, old_rows[h, i], h] for positions
 * i < n, with the new row found as in sbsa_relayout_runs (written to inverse,
 * which must not overlap old_rows) and posting[h, new row] = i.  Both stores
 * are [2, packed_len, Hkv, dim]; rows of dst that no key lands on keep what
 * they held. */
int sbsa_repack_runs(const void* src_packed, void* dst_packed, int64_t packed_len, int num_kv_heads,
                     int dim, int64_t n, const int32_t* old_rows, int64_t old_rows_ld,
                     const int32_t* old_indptr, const int32_t* new_indptr, int num_clusters,
                     int32_t* posting, int64_t posting_width, int32_t* inverse, int64_t inverse_ld,
                     hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SBSA_H */
