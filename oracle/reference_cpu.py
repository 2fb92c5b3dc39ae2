"""CPU restatement of semblo's semantic block-sparse attention path (the parity oracle).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg use it, and only as the checker or as the timed CPU baseline.

Each function restates one step of the reference (pfnet-research/
semantic-block-sparse-attention, "semblo") in torch on the CPU, op for op where
the reference is itself torch, so that on CPU tensors it reproduces the
reference's results bit for bit:

  S0  routing normalisation        trivial_router.py:55-61, routing_map.py:52-59,
                                   flat_index.py:165-166
  S1  flat k-means block build     state.py:545-948, flat_index.py:81-110,
                                   193-289, 356-383, state.py:44-84
  S1b pack_prompt_kv               state.py:950-997
  S2  centroid scoring             fused_select.py:1062-1247 (qtiled kernel),
                                   fused_select.py:865-906 (torch form)
  S3  budget selection (bisection) fused_select.py:604-646
      sorted-walk selection        fused_select.py:280-300, torch_select.py:39-68
  S3c causal snapshot              fused_prefill.py:44-135, 259-279
  S4  reverse index                kv_outer.py:254-329
  S5  KV-outer prefill attention   kv_outer.py:482-816, fused_prefill.py:155-189
  S6  LSE combine                  kv_outer.py:370-428
  S7-S9 decode step                fused_decode.py:81-358, 393-521
  S8  LSE merge                    paged_attention.py:50-80
  S10 token-order append           token_outer_prefill.py:39-87, 260-392,
                                   suffix_flush.py:154-170

Parity pins (each checked by a test in tests/):
  S0   closed form: unit norm of the bf16 result; reproduces the reference's
       torch fallback op for op.
  S1   golden vectors written by the reference's own ``ProductPostingIndex.build``
       on CPU (tests/golden/make_golden.py) -- bit-exact, with and without an
       attention sink (SEMBLO_SINK_TOKENS); the sink's hold-out and forced bit by
       the known answers of the reference's tests/test_fitted_sink.py:100-117.
  S2   fp64 loop form of the score (tests/test_oracle.py).
  S3   golden vectors of the reference's Triton select kernel run under the
       Triton CPU interpreter, plus the sorted-rule bound (sorted set is a subset
       of the bisection set) and the special cases (all fit, empty clusters).
  S4   brute-force transpose of the selection mask.
  S5/S6 fp64 brute force over the explicit key set S(p, h).
  S7-S9 fp64 brute force over the selected rows plus the visible suffix.
  S10  append_rows: the known answers of the reference's own test
       (tests/test_token_outer_prefill.py:30-38) and a vectorised sort-based
       form on random slices; reserved_layout: the reference test's
       properties (whole pages, at least one page, fits the width, ratio) and
       a hand-computed case; nearest_cluster: fp64 argmax on random keys
       (near-ties excluded) and the dead-descriptor rule.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

NEG_BIG = -3.4e38
POS_BIG = 3.4e38


# ---------------------------------------------------------------- S0 ----------

def trivial_router_vectors(x: torch.Tensor, factors: int = 1) -> torch.Tensor:
    """[Q, Hq, D] -> [Q, Hq, D] in x.dtype: normalise in fp32, round, renormalise, round.

    trivial_router.py:55-61 (the torch fallback, same rounding points as the kernel).
    """
    q, h, d = x.shape
    halves = x.float().view(q, h, factors, d // factors)
    unit = halves / halves.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    unit = unit.to(x.dtype).float()
    unit = unit / unit.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    return unit.to(x.dtype).view(q, h, d)


def routing_normalize_keys(k: torch.Tensor) -> torch.Tensor:
    """The identity key router in whole mode: F.normalize in fp32, cast back.

    routing_map.py:52-59 with SembloKeyRouter.project being the identity
    (routing_map.py:80-87).
    """
    rows = k.reshape(-1, k.shape[-1])
    return F.normalize(rows.float(), dim=-1).reshape_as(k).to(k.dtype)


def routing_space(x: torch.Tensor) -> torch.Tensor:
    """flat_index.py:165-166 (whole mode): fp32 unit vectors."""
    return F.normalize(x.float(), dim=-1)


# ---------------------------------------------------------------- S1 ----------

def flat_cluster_count(length: int, target_size: int, *, min_clusters: int = 64,
                       max_clusters: int = 16384) -> int:
    """flat_index.py:81-84."""
    return int(min(max(length // max(target_size, 1), min_clusters), max_clusters, length))


def num_flat_clusters(length: int, unit_tokens: int = 2048, min_log2: int = 7) -> int:
    """The power-of-two cluster count of state.py:586-597."""
    min_c_log2 = max(3, int(min_log2))
    raw_c = flat_cluster_count(length, unit_tokens)
    c = 1 << max(min_c_log2, (max(raw_c, 1) - 1).bit_length())
    return min(c, 1 << (int(length).bit_length() - 1))


def argmax_sim_chunked(x: torch.Tensor, centroids: torch.Tensor, chunk: int) -> torch.Tensor:
    """flat_index.py:356-373 (cosine): argmax over the bf16 GEMM's bf16 output.

    The GEMM's operands are bf16 and so is its result: the similarities are
    rounded to bf16 before the argmax, and ties go to the first index.
    """
    out = torch.empty(x.shape[0], dtype=torch.int64)
    cb = centroids.to(torch.bfloat16)
    for lo in range(0, x.shape[0], chunk):
        hi = min(lo + chunk, x.shape[0])
        sim = x[lo:hi].to(torch.bfloat16) @ cb.T
        out[lo:hi] = torch.argmax(sim, dim=1)
    return out


def segment_sum_matmul(x: torch.Tensor, assign: torch.Tensor, num_clusters: int,
                       chunk: int = 8192) -> torch.Tensor:
    """flat_index.py:87-110: per-cluster fp32 sums as a chunked one-hot GEMM."""
    sums = torch.zeros(num_clusters, x.shape[1], dtype=torch.float32)
    for lo in range(0, x.shape[0], chunk):
        hi = min(lo + chunk, x.shape[0])
        onehot = torch.zeros(hi - lo, num_clusters, dtype=torch.float32)
        onehot.scatter_(1, assign[lo:hi, None], 1.0)
        sums += onehot.T @ x[lo:hi].float()
    return sums


def fit_flat_codebook(space: torch.Tensor, num_clusters: int, *, num_iters: int,
                      sample_size: int, generator: torch.Generator,
                      chunk: int = 65536, trace: list | None = None,
                      steps: list | None = None) -> torch.Tensor:
    """flat_index.py:193-289 with init="random", metric="cosine", deterministic sums.

    ``space`` is already unit-norm fp32 (routing_space), so _fit_space's
    F.normalize is applied again exactly as the reference does.  ``trace``, if
    given, receives the random draws (sample rows, init rows, and per iteration
    the replacement rows of empty clusters) so a device implementation can be
    fed the identical draws.  ``steps``, if given, receives per iteration the
    fp32 centroids it starts from, its assignment, counts and sums.
    """
    x = F.normalize(space.float(), dim=-1)
    n = x.shape[0]
    fit_n = min(n, int(sample_size))
    if fit_n < num_clusters:
        raise ValueError("sample must be at least as large as num_clusters")
    perm = torch.randperm(n, generator=generator)
    sample = x[perm[:fit_n]]
    init = torch.randperm(fit_n, generator=generator)[:num_clusters]
    centroids = sample[init].clone()
    if trace is not None:
        trace.append(("sample", perm[:fit_n].clone()))
        trace.append(("init", init.clone()))
    for _ in range(num_iters):
        if steps is not None:
            steps.append(dict(entry=centroids.clone()))
        assign = argmax_sim_chunked(sample, centroids, chunk)
        counts = torch.bincount(assign, minlength=num_clusters)
        sums = segment_sum_matmul(sample, assign, num_clusters)
        if steps is not None:
            steps[-1].update(assign=assign.clone(), counts=counts.clone(), sums=sums.clone())
        empty = counts == 0
        if bool(empty.any()):
            repl = torch.randperm(fit_n, generator=generator)[: int(empty.sum())]
            sums[empty] = sample[repl]
            counts = counts.clone()
            counts[empty] = 1
            if trace is not None:
                trace.append(("empty", repl.clone()))
        elif trace is not None:
            trace.append(("empty", torch.zeros(0, dtype=torch.int64)))
        centroids = sums / counts[:, None].float()
        centroids = F.normalize(centroids, dim=-1)
    return centroids.to(space.dtype)


def page_align_order(order: torch.Tensor, counts: torch.Tensor, positions: torch.Tensor,
                     align: int):
    """state.py:44-84: pad each bucket to a page multiple; padding repeats order[0]."""
    length = int(order.numel())
    counts64 = counts.to(torch.int64)
    padded = ((counts64 + align - 1) // align) * align
    zero = counts64.new_zeros(1)
    ip_orig = torch.cat([zero, counts64.cumsum(0)])
    ip_pad = torch.cat([zero, padded.cumsum(0)])
    total = int(ip_pad[-1])
    ar = torch.arange(total)
    bucket = torch.searchsorted(ip_pad, ar, right=True) - 1
    off = ar - ip_pad[bucket]
    real = off < counts64[bucket]
    src = (ip_orig[bucket] + off).clamp_max(length - 1)
    new_order = torch.where(real, order[src], order[0])
    bucket_of_row = torch.searchsorted(ip_orig, torch.arange(length), right=True) - 1
    padded_row = torch.arange(length) + (ip_pad[bucket_of_row] - ip_orig[bucket_of_row])
    inverse = torch.zeros(length, dtype=torch.int32)
    inverse[positions[order].long()] = padded_row.to(torch.int32)
    return new_order, ip_pad.to(torch.int32), inverse


def check_sink_partition(sink: int, length: int, fit_length: int, num_clusters: int) -> None:
    """state.py:26-34: the sink settings the paper path refuses."""
    if sink % 16:
        raise RuntimeError(f"SEMBLO_SINK_TOKENS={sink}: a multiple of 16 keeps the sink cluster page-aligned")
    if length <= sink or fit_length - sink < 2 * num_clusters:
        raise RuntimeError(f"SEMBLO_SINK_TOKENS={sink} leaves too few keys")


def build_flat_index(product_keys: torch.Tensor, positions: torch.Tensor | None = None, *,
                     unit_tokens: int = 2048, min_clusters_log2: int = 7,
                     sample_size: int = 8192, fit_iters: int = 8, per_centroid: int = 32,
                     codebook_seed: int = 0, page_align: int = 16,
                     num_clusters: int | None = None, traces: list | None = None,
                     fit_steps: list | None = None, sink_tokens: int = 0) -> dict:
    """ProductPostingIndex._build_flat, state.py:545-948, on the paper path.

    product_keys [L, Hkv, I] are the router's output (routing_normalize_keys of
    the pre-RoPE keys).  The generator is a CPU torch.Generator seeded with
    ``codebook_seed`` (state.py:520-523), used for every head in turn.
    Returns codebooks [Hkv, 2, C, I/2] (key dtype), posting [Hkv, W] int32,
    indptr [Hkv, C+1] int32, sizes [Hkv, C] int32, inverse [Hkv, L] int32.

    ``sink_tokens`` S > 0 (SEMBLO_SINK_TOKENS, state.py:757-782): positions 0..S-1
    form cluster 0 with a zero centroid; positions S.. are fitted into C-1
    clusters (sample min(fit_sample, L-S)) and assigned to them as ids 1..C-1.
    ``fit_steps`` then describes that fit (rows S..).
    """
    length, num_kv_heads, index_dim = product_keys.shape
    if positions is None:
        positions = torch.arange(length)
    gen = torch.Generator()
    gen.manual_seed(int(codebook_seed))
    c = num_clusters or num_flat_clusters(length, unit_tokens, min_clusters_log2)
    codebooks, posting_rows, indptr_rows, size_rows, inverse_rows = [], [], [], [], []
    sink = int(sink_tokens)
    if sink:
        check_sink_partition(sink, length, length, c)
    for h in range(num_kv_heads):
        keys = product_keys[:, h]
        space = routing_space(keys)
        fit_sample = min(length, max(int(sample_size), per_centroid * c))
        trace = [] if traces is not None else None
        steps = [] if fit_steps is not None else None
        if sink:
            rest = fit_flat_codebook(space[sink:], c - 1, num_iters=fit_iters,
                                     sample_size=min(fit_sample, length - sink), generator=gen,
                                     trace=trace, steps=steps)
            cents = torch.cat([rest.new_zeros(1, rest.shape[1]), rest], dim=0)
            rest_assign = argmax_sim_chunked(F.normalize(space[sink:].float(), dim=-1), rest, 65536)
            assign = torch.cat([torch.zeros(sink, dtype=torch.long), rest_assign.long() + 1])
            fit_cents, fit_assign = rest, rest_assign
        else:
            cents = fit_flat_codebook(space, c, num_iters=fit_iters, sample_size=fit_sample,
                                      generator=gen, trace=trace, steps=steps)
            assign = argmax_sim_chunked(F.normalize(space.float(), dim=-1), cents, 65536)
            fit_cents, fit_assign = cents, assign
        if traces is not None:
            traces.append(trace)
        if fit_steps is not None:
            fit_steps.append(dict(steps=steps, final_centroids=fit_cents, final_assign=fit_assign))
        order = torch.argsort(assign, stable=True)
        counts = torch.bincount(assign, minlength=c).to(torch.int32)
        if page_align > 1:
            order, indptr, inv_row = page_align_order(order, counts, positions, page_align)
        else:
            indptr = torch.cat([torch.zeros(1, dtype=torch.int32), counts.cumsum(0).to(torch.int32)])
            inv_row = torch.empty(length, dtype=torch.int32)
            inv_row[positions[order].long()] = torch.arange(length, dtype=torch.int32)
        inverse_rows.append(inv_row)
        unit = routing_space(cents)
        desc = torch.stack(list(unit.chunk(2, dim=-1)), dim=0).to(product_keys.dtype)
        codebooks.append(desc)
        posting_rows.append(positions[order].to(torch.int32).contiguous())
        indptr_rows.append(indptr.contiguous())
        size_rows.append(counts.contiguous())
    width = max(int(r.numel()) for r in posting_rows)
    posting_rows = [r if r.numel() == width else torch.cat([r, r[:1].expand(width - r.numel())])
                    for r in posting_rows]
    return dict(codebooks=torch.stack(codebooks).contiguous(),
                posting=torch.stack(posting_rows).contiguous(),
                indptr=torch.stack(indptr_rows).contiguous(),
                sizes=torch.stack(size_rows).contiguous(),
                inverse=torch.stack(inverse_rows).contiguous(),
                num_clusters=c, prompt_length=length)


PACK_ALIGN = 256


def pack_prompt_kv(posting: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """state.py:950-997: [2, W padded to 256, Hkv, D], gathered through the posting list."""
    order = posting.to(torch.int64).t().contiguous()
    packed_len, head_dim = order.shape[0], key.shape[-1]
    pad = (-packed_len) % PACK_ALIGN
    packed = torch.zeros(2, packed_len + pad, order.shape[1], head_dim, dtype=key.dtype)
    idx = order.unsqueeze(-1).expand(-1, -1, head_dim)
    packed[0, :packed_len] = torch.gather(key, 0, idx)
    packed[1, :packed_len] = torch.gather(value, 0, idx)
    return packed


# ---------------------------------------------------------------- S2 ----------

def mixture_probs(vectors: torch.Tensor, logmix: torch.Tensor | None, codebooks: torch.Tensor,
                  temperature: float, slab: int = 1024) -> torch.Tensor:
    """[Q, Hkv, C] fp32 mixture probability (fused_select.py:865-906, torch form).

    vectors [Q, Hq, I] (bf16 routing vectors, R = 1), logmix [Q, Hq] fp32 or
    None (uniform: log 1 = 0), codebooks [Hkv, 2, C, I/2].  Per component t:
    s = (q0.c0 + q1.c1) / tau with bf16 values and fp32 sums, log-softmax over
    C, plus logmix, exp, summed over the G components of the KV head.
    """
    q_count, num_q_heads, index_dim = vectors.shape
    num_kv_heads, _, c_dim, df = codebooks.shape
    t_dim = num_q_heads // num_kv_heads
    if logmix is None:
        logmix = torch.zeros(q_count, num_q_heads)
    prob = torch.empty(q_count, num_kv_heads, c_dim, dtype=torch.float32)
    cb = codebooks.float()
    inv_t = 1.0 / float(temperature)
    for lo in range(0, q_count, slab):
        hi = min(lo + slab, q_count)
        n = hi - lo
        q5 = vectors[lo:hi].reshape(n, num_kv_heads, t_dim, 2, df).float()
        lm = logmix[lo:hi].reshape(n, num_kv_heads, t_dim, 1).float()
        for h in range(num_kv_heads):
            a0 = q5[:, h, :, 0].reshape(n * t_dim, df)
            a1 = q5[:, h, :, 1].reshape(n * t_dim, df)
            sc = (a0 @ cb[h, 0].T + a1 @ cb[h, 1].T).view(n, t_dim, c_dim)
            sc *= inv_t
            prob[lo:hi, h] = (sc.log_softmax(dim=-1) + lm[:, h]).exp_().sum(dim=1)
    return prob


def mixture_probs_fp64(vectors, logmix, codebooks, temperature):
    """The same quantity as a float64 loop (the tests' independent form,
    after tests/test_torch_select.py:19-47 of the reference)."""
    q_count, num_q_heads, index_dim = vectors.shape
    num_kv_heads, _, c_dim, df = codebooks.shape
    g = num_q_heads // num_kv_heads
    out = torch.zeros(q_count, num_kv_heads, c_dim, dtype=torch.float64)
    for h in range(num_kv_heads):
        cent = torch.cat([codebooks[h, 0].double(), codebooks[h, 1].double()], dim=-1)
        for t in range(g):
            vec = vectors[:, h * g + t].double()
            logits = (vec @ cent.T) / temperature
            w = 1.0 if logmix is None else logmix[:, h * g + t].double().exp()[:, None]
            out[:, h] += torch.softmax(logits, dim=-1) * w
    return out


# ---------------------------------------------------------------- S3 ----------

def theta_select(prob: torch.Tensor, sizes: torch.Tensor, *, beta: float, target_tokens: float,
                 g_union: int = 1, iters: int = 16) -> dict:
    """The RESIDENT bisection of _streaming_select_kernel, fused_select.py:604-646.

    prob [Q, Hkv, C] fp32; sizes [NB, Hkv, C] int32, query q uses block q // g_union.
    Every step is fp32, in the kernel's order; the size sums are integers below
    2^24 and therefore exact in any order.  Returns the per-query selection
    (bool [Q, Hkv, C]), theta [Q, Hkv], score [Q, Hkv, C], counts, tokens, and
    the union bitmask words [NB, Hkv, C/32] (int32).
    """
    q_count, hkv, c = prob.shape
    blocks = torch.arange(q_count) // g_union
    sz = sizes[blocks].to(torch.float32)                 # [Q, Hkv, C]
    live = sz > 0
    score = torch.log(torch.clamp(prob.float(), min=1e-38))
    if beta != 0.0:
        score = score - torch.tensor(beta, dtype=torch.float32) * torch.log(1.0 + sz)
    score = torch.where(live, score, torch.tensor(NEG_BIG, dtype=torch.float32))
    e6 = torch.tensor(1e-6, dtype=torch.float32)
    e5 = torch.tensor(1e-5, dtype=torch.float32)
    hi = score.max(dim=-1).values + e6
    lo = torch.where(live, score, torch.tensor(POS_BIG, dtype=torch.float32)).min(dim=-1).values - e6
    lo = torch.minimum(lo, hi - e5)
    tgt = torch.tensor(float(target_tokens), dtype=torch.float32)
    all_fit = torch.where(live, sz, torch.zeros_like(sz)).sum(dim=-1) < tgt
    half = torch.tensor(0.5, dtype=torch.float32)
    for _ in range(iters):
        mid = (lo + hi) * half
        above = torch.where(score >= mid[..., None], sz, torch.zeros_like(sz)).sum(dim=-1)
        reach = above >= tgt
        lo = torch.where(reach, mid, lo)
        hi = torch.where(reach, hi, mid)
    theta = torch.where(all_fit, torch.tensor(NEG_BIG, dtype=torch.float32), lo)
    sel = live & (score >= theta[..., None])
    counts = sel.sum(-1).to(torch.int32)
    tokens = torch.where(sel, sz, torch.zeros_like(sz)).sum(-1).to(torch.int32)
    nb = sizes.shape[0]
    union = torch.zeros(nb, hkv, c, dtype=torch.bool)
    for b in range(nb):
        rows = sel[b * g_union:(b + 1) * g_union]
        if rows.numel():
            union[b] = rows.any(dim=0)
    return dict(sel=sel, theta=theta, score=score, counts=counts, tokens=tokens,
                bitmask=pack_bits(union), qmask=pack_bits(sel), all_fit=all_fit)


def hold_out_sink(sizes: torch.Tensor, target_tokens: int, sink: int):
    """fused_prefill.py:202-209: the selector's sizes with cluster 0 hidden (a copy), and
    the budget the other clusters share."""
    held = sizes.clone()
    held[..., 0] = 0
    return held, max(0, int(target_tokens) - int(sink))


def force_sink_bit(*masks) -> None:
    """fused_prefill.py:212-216: cluster 0 selected in every row of every mask, in place."""
    for m in masks:
        if m is not None:
            m[..., 0].bitwise_or_(1)


def sorted_select(score: torch.Tensor, sizes: torch.Tensor, target_tokens: float,
                  g_union: int = 1) -> torch.Tensor:
    """theta_select_reference, fused_select.py:280-300: walk clusters in descending
    score and stop once the causal tokens reach the budget (the crossing cluster
    is included).  score [Q, Hkv, C] (penalty applied, -3.4e38 for dead)."""
    q_count, hkv, c = score.shape
    blocks = torch.arange(q_count) // g_union
    sz = sizes[blocks].to(score.dtype)
    s = score.masked_fill(sz <= 0, float("-inf"))
    order = s.argsort(dim=-1, descending=True, stable=True)
    ssz = sz.gather(-1, order)
    csum = ssz.cumsum(dim=-1)
    take = ((csum - ssz) < target_tokens) & (s.gather(-1, order) > float("-inf"))
    return torch.zeros_like(take).scatter(-1, order, take)


def pack_bits(mask: torch.Tensor) -> torch.Tensor:
    """[.., C] bool -> [.., C/32] int32 with bit (c & 31) of word c >> 5 (fused_select.py:627-629)."""
    *lead, c = mask.shape
    w = mask.reshape(*lead, c // 32, 32).to(torch.int64)
    words = (w << torch.arange(32)).sum(-1)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words)
    return words.to(torch.int32)


def unpack_bits(words: torch.Tensor, c: int) -> torch.Tensor:
    *lead, nw = words.shape
    w = words.to(torch.int64) & 0xFFFFFFFF
    bits = (w[..., None] >> torch.arange(32)) & 1
    return bits.reshape(*lead, nw * 32)[..., :c].bool()


# ---------------------------------------------------------------- S3c ---------

def causal_sizes_at(posting: torch.Tensor, indptr: torch.Tensor, sizes: torch.Tensor,
                    pos_limit: int) -> torch.Tensor:
    """|{keys of cluster c with position < pos_limit}| per (head, cluster).

    CausalSnapshot.advance(pos_limit - 1), fused_prefill.py:126-135.  Keys enter
    a cluster's run in position order, so these are the first rows of the run.
    """
    hkv, c = sizes.shape
    out = torch.zeros(hkv, c, dtype=torch.int32)
    for h in range(hkv):
        for cl in range(c):
            s = int(indptr[h, cl])
            n = int(sizes[h, cl])
            out[h, cl] = int((posting[h, s:s + n] < pos_limit).sum())
    return out


def chunk_window_start(chunk_start: int, target_tokens: int, dense_prefix_x: int = 4,
                       local: int = 0) -> int:
    """fused_prefill.py:263-266: 0 (dense chunk) while the prefix is within x budgets."""
    cap = dense_prefix_x * target_tokens
    return 0 if chunk_start <= cap else max(0, chunk_start - local)


# ---------------------------------------------------------------- S4 ----------

def reverse_index(sel: torch.Tensor, live: torch.Tensor):
    """kv_outer.py:254-329 restated: per (head, cluster) the sorted query ids that
    selected it; entries are numbered head-major, cluster-major, query-ascending.

    sel [Q, Hkv, C] bool, live [Hkv, C] bool.  Returns (counts [Hkv, C],
    indptr [Hkv*C + 1] int64, qvals [nnz] int32).
    """
    q_count, hkv, c = sel.shape
    m = sel & live[None]
    counts = m.sum(0).to(torch.int32)                      # [Hkv, C]
    flat = counts.reshape(-1).to(torch.int64)
    indptr = torch.cat([torch.zeros(1, dtype=torch.int64), flat.cumsum(0)])
    qvals = []
    for h in range(hkv):
        for cl in range(c):
            qvals.append(torch.nonzero(m[:, h, cl]).flatten().to(torch.int32))
    qvals = torch.cat(qvals) if qvals else torch.zeros(0, dtype=torch.int32)
    return counts, indptr, qvals


# ------------------------------------------------------------- S5 / S6 --------

def prefill_chunk_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            posting: torch.Tensor, indptr: torch.Tensor,
                            causal_sizes: torch.Tensor, sel: torch.Tensor | None,
                            chunk_start: int, wstart: int, sm_scale: float) -> torch.Tensor:
    """fp64 attention of the chunk's queries over the explicit key set S(p, h).

    q [Qc, Hq, D] for positions chunk_start.., k/v [L, Hkv, D] in prompt order,
    the packed layout (posting, indptr) and causal_sizes [Hkv, C] taken at
    wstart, sel [Qc, Hkv, C] bool (ignored for a dense chunk, wstart == 0).
    S(p, h) = union over selected c of the first causal_sizes[h, c] rows of
    cluster c's run, plus positions wstart..p (kv_outer.py:482-816 for a sparse
    chunk, fused_prefill.py:155-189 when wstart == 0).
    """
    q_count, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = torch.zeros(q_count, hq, d, dtype=torch.float64)
    kd, vd = k.double(), v.double()
    for h in range(hkv):
        for qi in range(q_count):
            p = chunk_start + qi
            pos = []
            if wstart > 0 and sel is not None:
                for cl in torch.nonzero(sel[qi, h]).flatten().tolist():
                    s = int(indptr[h, cl])
                    n = int(causal_sizes[h, cl])
                    pos.append(posting[h, s:s + n].long())
            pos.append(torch.arange(wstart, p + 1))
            pos = torch.cat(pos)
            kk, vv = kd[pos, h], vd[pos, h]
            for t in range(g):
                s = (kk @ q[qi, h * g + t].double()) * sm_scale
                out[qi, h * g + t] = torch.softmax(s, dim=0) @ vv
    return out


def lse_merge(o_a, lse_a, o_b, lse_b):
    """merge_paged_attention_results, paged_attention.py:70-80 (exact LSE merge)."""
    merged = torch.logaddexp(lse_a.double(), lse_b.double())
    wa = torch.exp(lse_a.double() - merged)
    wb = torch.exp(lse_b.double() - merged)
    return o_a.double() * wa[..., None] + o_b.double() * wb[..., None], merged


# ------------------------------------------------------------- S7 - S9 --------

def decode_reference(q: torch.Tensor, packed: torch.Tensor, indptr: torch.Tensor,
                     sizes: torch.Tensor, sel: torch.Tensor, suffix_k: torch.Tensor,
                     suffix_v: torch.Tensor, sm_scale: float, with_lse: bool = False):
    """fp64 attention of one decode query over the selected clusters' full runs
    plus the visible suffix (tests/test_fused_decode_v3.py:98-124 of the reference).

    q [Hq, D]; packed [2, W, Hkv, D]; sel [Hkv, C] bool; suffix_k/v [S, Hkv, D]
    are the suffix tokens at positions <= the query's.  With ``with_lse`` also
    returns the natural-log log-sum-exp of the scaled scores [Hq]
    (fused_prefill.py:625-718 returns it beside the output).
    """
    hq, d = q.shape
    hkv = packed.shape[2]
    g = hq // hkv
    out = torch.zeros(hq, d, dtype=torch.float64)
    lse = torch.full((hq,), -math.inf, dtype=torch.float64)
    for h in range(hkv):
        rows = [torch.arange(int(indptr[h, cl]), int(indptr[h, cl]) + int(sizes[h, cl]))
                for cl in torch.nonzero(sel[h]).flatten().tolist()]
        rows = torch.cat(rows) if rows else torch.zeros(0, dtype=torch.long)
        kk = torch.cat([packed[0, rows, h].double(), suffix_k[:, h].double()])
        vv = torch.cat([packed[1, rows, h].double(), suffix_v[:, h].double()])
        for t in range(g):
            s = (kk @ q[h * g + t].double()) * sm_scale
            out[h * g + t] = torch.softmax(s, dim=0) @ vv
            if s.numel():
                lse[h * g + t] = torch.logsumexp(s, dim=0)
    return (out, lse) if with_lse else out


# ---------------------------------------------------------------- S10 ---------

def reserved_layout(sizes_ref: torch.Tensor, n_ref: int, total_tokens: int, width: int,
                    align: int) -> torch.Tensor:
    """token_outer_prefill.py:39-63: rows reserved per cluster, [Hkv, C] int64.

    Each cluster's expected share of ``total_tokens`` (its fraction of the
    ``n_ref`` reference keys), rounded up to whole pages of ``align`` rows,
    never below one page; the pages left in ``width`` are then handed out in
    the same proportions, rounded down.  Raises when the rounded shares alone
    do not fit.
    """
    align = max(int(align), 1)
    want = sizes_ref.double() * (float(total_tokens) / float(max(int(n_ref), 1)))
    pages = torch.ceil(want / align).to(torch.int64).clamp_min(1)
    rows = pages * align
    for h in range(rows.shape[0]):
        left = int(width) - int(rows[h].sum())
        if left < 0:
            raise RuntimeError(f"head {h}: the reserved layout needs {int(rows[h].sum())} rows, "
                               f"the store holds {width}")
        if left >= align:
            frac = want[h] / max(float(want[h].sum()), 1.0)
            rows[h] += torch.floor(frac * (left // align)).to(torch.int64) * align
    return rows


def append_rows(ids: torch.Tensor, indptr: torch.Tensor, sizes: torch.Tensor):
    """token_outer_prefill.py:66-87, as a scan in position order.

    ids [Hkv, n] (cluster of each new key), indptr [Hkv, C+1], sizes [Hkv, C].
    A key goes to the row after the last key of its cluster: the run start,
    plus the keys already there, plus the slice's earlier keys of that
    cluster.  Returns rows [Hkv, n] int64 and counts [Hkv, C] int64.
    """
    hkv, n = ids.shape
    c = sizes.shape[1]
    rows = torch.empty(hkv, n, dtype=torch.int64)
    counts = torch.zeros(hkv, c, dtype=torch.int64)
    for h in range(hkv):
        nxt = (indptr[h, :c].to(torch.int64) + sizes[h].to(torch.int64)).tolist()
        cnt = [0] * c
        for i, b in enumerate(ids[h].tolist()):
            rows[h, i] = nxt[b]
            nxt[b] += 1
            cnt[b] += 1
        counts[h] = torch.tensor(cnt, dtype=torch.int64)
    return rows, counts


def nearest_cluster(keys: torch.Tensor, codebooks_h: torch.Tensor, *, router_pass: bool = True,
                    return_sim: bool = False):
    """The cluster of each new key in _append (token_outer_prefill.py:339-348).

    keys [n, I] of one KV head: pre-RoPE keys, through the identity key router
    (routing_normalize_keys) when ``router_pass``.  routing_space
    (flat_index.py:165-166), then _nearest_cluster (suffix_flush.py:154-170):
    F.normalize in fp32 against cat(codebooks_h[0], codebooks_h[1]) in fp32,
    all-zero descriptors at -inf, torch.argmax (first maximum).
    """
    product = routing_normalize_keys(keys) if router_pass else keys
    space = routing_space(product)
    cents = torch.cat([codebooks_h[0], codebooks_h[1]], dim=-1).float()
    sim = F.normalize(space.float(), dim=-1) @ cents.t()
    sim[:, cents.norm(dim=-1) == 0] = -float("inf")
    ids = sim.argmax(dim=-1)
    return (ids, sim) if return_sim else ids


def relayout_rows(old_rows: torch.Tensor, old_indptr: torch.Tensor,
                  new_indptr: torch.Tensor) -> torch.Tensor:
    """The row moves of _fit_and_pack / _repack (token_outer_prefill.py:287-292, 376-379).

    A key at row r of the old layout belongs to the last cluster b with
    old_indptr[b] <= r and keeps its offset in that cluster's new run.
    old_rows [Hkv, n]; returns new rows [Hkv, n] int64.
    """
    out = torch.empty(old_rows.shape, dtype=torch.int64)
    for h in range(old_rows.shape[0]):
        ip = old_indptr[h].to(torch.int64).contiguous()
        r = old_rows[h].to(torch.int64).contiguous()
        b = torch.searchsorted(ip, r, right=True) - 1
        out[h] = r - ip[b] + new_indptr[h].to(torch.int64)[b]
    return out


# ------------------------------------------------------------ suffix flush -----

def flush_range(prompt_len: int, written: int, plen_cur: int, keep: int, every: int):
    """suffix_flush.py:140-152: the positions [frm, to) to move, or None.  ``written``
    generated tokens sit at [prompt_len, prompt_len + written); those below ``plen_cur``
    were moved already.  Once keep + every tokens are exact, all but the newest keep move."""
    live = prompt_len + written - plen_cur
    if live >= keep + every:
        return plen_cur, prompt_len + written - keep
    return None


def flush_store(posting: torch.Tensor, indptr: torch.Tensor, sizes: torch.Tensor,
                ids: torch.Tensor, first_position: int, align: int):
    """The layout after a flush (repack_plan / repack_apply, suffix_flush.py:55-137).

    posting [Hkv, W], indptr [Hkv, C+1], sizes [Hkv, C] of the store before; ids [Hkv, n]
    the clusters of positions first_position .. first_position + n - 1.  Every cluster
    keeps its rows in order and takes its newcomers after them in position order; the
    runs are laid out again from row 0, each padded to a whole number of ``align`` rows.
    Returns (runs, new_sizes [Hkv, C], new_indptr [Hkv, C+1]) with runs[h][c] the
    positions of cluster c's rows in row order."""
    hkv, c = sizes.shape
    align = max(int(align), 1)
    runs = []
    new_sizes = torch.zeros(hkv, c, dtype=torch.int64)
    new_indptr = torch.zeros(hkv, c + 1, dtype=torch.int64)
    for h in range(hkv):
        lists = []
        for b in range(c):
            st = int(indptr[h, b])
            lists.append([int(x) for x in posting[h, st:st + int(sizes[h, b])].tolist()])
        for i, b in enumerate(ids[h].tolist()):
            lists[b].append(int(first_position) + i)
        runs.append(lists)
        row = 0
        for b in range(c):
            new_sizes[h, b] = len(lists[b])
            new_indptr[h, b] = row
            row += -(-len(lists[b]) // align) * align
        new_indptr[h, c] = row
    return runs, new_sizes, new_indptr
