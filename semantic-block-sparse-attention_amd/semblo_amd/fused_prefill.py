"""Per-chunk prefill and the prompt part of a decode step (the reference's
semblo/vllm_plugin/fused_prefill.py seams, paper path: FA3 page 16, KV-outer).

  CausalSnapshot          cluster sizes at a position       (fused_prefill.py:44-135)
  fused_chunk_attention   dense prefix or select + KV-outer (fused_prefill.py:219-482),
                          also as its two halves: fused_chunk_plan (selection and
                          reverse index) and fused_chunk_execute (the attention)
  fused_decode_attention  one query over the packed prompt  (fused_prefill.py:625-718)
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .config import fitted_sink_tokens
from .fused_select import theta_select_bitmask_flat
from .kv_outer import dense_causal_attention, kv_outer_execute, kv_outer_plan


@dataclass(frozen=True)
class PagedSparseAttentionResult:
    """paged_attention.py:44-47."""

    output: torch.Tensor             # [Q, Hq, D]
    logsumexp: torch.Tensor | None   # [Q, Hq]


class CausalSnapshot:
    """Per-cluster counts of keys at positions <= p (fused_prefill.py:44-135).

    Keys enter a cluster's run in position order, so the count at p is found
    by a binary search in each run (one small kernel) instead of the
    reference's running bincount.
    """

    def __init__(self, index) -> None:
        self.index = index
        self.length = int(index.prompt_length)
        hkv, c = index.bucket_sizes.shape
        self.sizes = torch.zeros(hkv, c, dtype=torch.int32, device=index.bucket_sizes.device)
        self.next_pos = 0

    def advance(self, last_pos: int) -> torch.Tensor:
        """Counts at positions <= last_pos (calls must be non-decreasing)."""
        hi = min(int(last_pos) + 1, self.length)
        if hi > self.next_pos:
            self.index.causal_sizes(hi, out=self.sizes)
            self.next_pos = hi
        return self.sizes


class ChunkPlan:
    """The selection side of one sparse chunk: its causal snapshot, the per-query
    cluster masks and the reverse index, all on the device."""

    def __init__(self, chunk_start, chunk_end, wstart, causal_sizes, tokens, kv, theta=None):
        self.chunk_start, self.chunk_end, self.wstart = chunk_start, chunk_end, wstart
        self.causal_sizes, self.tokens, self.kv = causal_sizes, tokens, kv
        self.theta = theta

    def record(self, log: list | None) -> None:
        """Append what decided this chunk's key sets to ``log`` (a test hook: the per-query
        cluster masks, the causal sizes and the cut theta, device tensors)."""
        if log is not None:
            log.append(dict(chunk_start=self.chunk_start, chunk_end=self.chunk_end,
                            wstart=self.wstart, causal_sizes=self.causal_sizes,
                            qmask=self.kv.qmask, theta=self.theta))

    def tensors(self):
        return (self.causal_sizes, self.tokens, *self.kv.tensors())


def chunk_window_start(chunk_start: int, target_tokens: int, dense_prefix_x: int = 4,
                       local: int = 0) -> int:
    """0 for a dense-prefix chunk (chunk_start <= x * K), else the window's first
    position (fused_prefill.py:259-279)."""
    cap = dense_prefix_x * target_tokens
    return 0 if chunk_start <= cap else max(0, chunk_start - local)


def hold_out_sink(sizes: torch.Tensor, target_tokens: int, sink: int) -> tuple[torch.Tensor, int]:
    """The sizes the selection sees with the sink cluster 0 hidden (a copy: the attention
    still reads cluster 0's rows), and the budget the other clusters share
    (fused_prefill.py:202-209)."""
    held = sizes.clone()
    held[..., 0] = 0
    return held, max(0, int(target_tokens) - int(sink))


def force_sink_bit(*masks: torch.Tensor | None) -> None:
    """Select cluster 0 in every row of every mask, in place (fused_prefill.py:212-216)."""
    for m in masks:
        if m is not None:
            m[..., 0].bitwise_or_(1)


def fused_chunk_plan(q_chunk: torch.Tensor, query_state, index, snapshot_state, chunk_start: int,
                     chunk_end: int, *, temperature: float, beta: float, target_tokens: int,
                     queries_per_block: int = 32, iters: int = 16, local: int = 0,
                     dense_prefix_x: int = 4, keep_theta: bool = False) -> ChunkPlan:
    """Selection and reverse index of a sparse chunk (fused_prefill.py:281-482 up to
    the attention calls); no host read.  ``keep_theta`` also keeps each query's cut
    (for ChunkPlan.record)."""
    q_count = q_chunk.shape[0]
    hkv = index.num_kv_heads
    c = index.num_buckets
    wstart = chunk_window_start(chunk_start, target_tokens, dense_prefix_x, local)
    if wstart == 0:
        raise ValueError("a dense-prefix chunk has no selection to plan")
    sizes = snapshot_state.advance(wstart - 1)
    causal_sizes = sizes.clone()
    vectors = query_state.vectors[0]
    logmix = query_state.mixture_weights[0].float().clamp_min(1e-12).log()
    g_union = min(queries_per_block, q_count)
    nb = (q_count + g_union - 1) // g_union
    bitmask = torch.zeros(nb, hkv, c // 32, dtype=torch.int32, device=q_chunk.device)
    qmask = torch.empty(q_count, hkv, c // 32, dtype=torch.int32, device=q_chunk.device)
    theta = torch.empty(q_count, hkv, dtype=torch.float32, device=q_chunk.device) if keep_theta else None
    # a sink (cluster 0, positions 0..S-1) is hidden from the search, which shares
    # K - S among the other clusters, and then read by every query
    # (fused_prefill.py:382-405)
    sink = fitted_sink_tokens()
    select_sizes, select_target = (hold_out_sink(causal_sizes, target_tokens, sink) if sink
                                   else (causal_sizes, target_tokens))
    _, tokens = theta_select_bitmask_flat(vectors, logmix, index.codebooks, select_sizes[None],
                                          bitmask, temperature=temperature, beta=beta,
                                          target_tokens=select_target, g_union=g_union,
                                          iters=iters, qmask=qmask, theta_out=theta)
    if sink:
        force_sink_bit(bitmask, qmask)
    kv = kv_outer_plan(qmask, causal_sizes, num_queries=q_count)
    return ChunkPlan(chunk_start, chunk_end, wstart, causal_sizes, tokens, kv, theta)


def fused_chunk_execute(plan: ChunkPlan, q_chunk: torch.Tensor, index, nnz: int | None = None, *,
                        sm_scale: float, fa3_page_size: int = 16, out: torch.Tensor | None = None,
                        timing=None, window_kv=None, guard=None) -> torch.Tensor:
    """The attention of a planned sparse chunk.  ``nnz`` (its partial count, read on the
    host) sizes the partial rows exactly; None sizes them by the capacity bound, capped
    in bytes, so the chunk is enqueued without waiting for its plan (kv_outer_execute;
    ``guard``, a kv_outer.PartialsGuard, then settles a capped chunk later)."""
    q_count, hq, d = q_chunk.shape
    hkv = index.num_kv_heads
    wstart, chunk_start, chunk_end = plan.wstart, plan.chunk_start, plan.chunk_end
    if timing is not None and timing.counts_flops:
        # selected rows of every (query, KV head), each read by its G query heads,
        # plus the causal window (p - chunk_start + 1 keys per query and head)
        g = hq // hkv
        window = q_count * (q_count + 1) // 2
        timing.add_flops(4.0 * d * (g * plan.tokens.to(torch.float64).sum() + hq * window))
    if window_kv is not None:
        if window_kv[0].shape[0] != chunk_end + 1 - wstart:
            raise ValueError("window_kv must hold positions wstart..chunk_end")
        window = window_kv
    else:
        if index.original_kv is None:
            raise RuntimeError("the prefill reads the chunk's window from the prompt-order K/V "
                               "(index.original_kv), which this index no longer holds")
        k_orig, v_orig = index.original_kv
        window = (k_orig[wstart:chunk_end + 1], v_orig[wstart:chunk_end + 1])
    res, _ = kv_outer_execute(q_chunk, index.packed_kv, plan.kv, nnz, index.bucket_indptr,
                              sm_scale=sm_scale, local_kv=window, chunk_start=chunk_start,
                              wstart=wstart, out=out, timing=timing, guard=guard)
    return res


def fused_chunk_attention(q_chunk: torch.Tensor, query_state, index, q_positions: torch.Tensor,
                          snapshot_state: CausalSnapshot, chunk_start: int, chunk_end: int, *,
                          temperature: float, beta: float, target_tokens: int,
                          queries_per_block: int = 32, sm_scale: float, iters: int = 16,
                          fa3_page_size: int = 16, kv_outer_default: bool = True,
                          dense_prefix_x: int = 4, local: int = 0, out: torch.Tensor | None = None,
                          timing=None, window_kv=None, plan_log: list | None = None,
                          guard=None, **unused) -> torch.Tensor:
    """Attention of one query chunk [chunk_start, chunk_end] (fused_prefill.py:219-482).

    While chunk_start <= dense_prefix_x * K the chunk is dense and causal over
    the whole prefix (fused_prefill.py:259-279); otherwise every cluster's
    rows before wstart = chunk_start are read sparsely, per query, and the
    chunk's own tokens through the exact causal window.  ``window_kv`` (k, v),
    rows wstart..chunk_end in prompt order, replaces the slice of
    ``index.original_kv`` for that window (the token-order prefill, whose
    store has no prompt-order copy).  One host read (the partial count).
    ``plan_log``: a test hook, see ChunkPlan.record.  ``guard``: a kv_outer.PartialsGuard
    that settles the chunk later if its partial rows were capped (with none, a capped
    chunk is settled before returning: one host read).
    """
    if not kv_outer_default or not fa3_page_size:
        raise NotImplementedError("only the paper path (FA3 page body, KV-outer) is built")
    q_count = q_chunk.shape[0]
    wstart = chunk_window_start(chunk_start, target_tokens, dense_prefix_x, local)
    if wstart == 0:
        if index.original_kv is None:
            raise RuntimeError("the prefill reads the chunk's window from the prompt-order K/V "
                               "(index.original_kv), which this index no longer holds")
        k_orig, v_orig = index.original_kv
        hq, d = q_chunk.shape[1], q_chunk.shape[2]
        if timing is not None:
            # sum over p in the chunk of (p + 1) keys, every query head, 4 D FLOPs per key
            n = q_count
            keys = n * (chunk_start + 1) + n * (n - 1) // 2
            timing.add_flops(4.0 * d * hq * keys)
        return dense_causal_attention(q_chunk, k_orig, v_orig, sm_scale=sm_scale,
                                      chunk_start=chunk_start, out=out, timing=timing)
    plan = fused_chunk_plan(q_chunk, query_state, index, snapshot_state, chunk_start, chunk_end,
                            temperature=temperature, beta=beta, target_tokens=target_tokens,
                            queries_per_block=queries_per_block, iters=iters, local=local,
                            dense_prefix_x=dense_prefix_x, keep_theta=plan_log is not None)
    plan.record(plan_log)
    # no host read: the partial rows are sized by the capacity bound
    return fused_chunk_execute(plan, q_chunk, index, None, sm_scale=sm_scale,
                               fa3_page_size=fa3_page_size, out=out, timing=timing,
                               window_kv=window_kv, guard=guard)


def fused_decode_attention(q_chunk: torch.Tensor, query_state, index, q_positions: torch.Tensor, *,
                           temperature: float, beta: float, target_tokens: int, sm_scale: float,
                           iters: int = 16, num_splits: int = 64, csr_out=None,
                           **unused) -> PagedSparseAttentionResult:
    """One decode query over the packed prompt, selection against the full cluster
    sizes (fused_prefill.py:625-718).  The generated suffix is merged by the caller."""
    from .fused_decode import decode_prompt_only
    return decode_prompt_only(q_chunk, query_state.vectors[0], index, temperature=temperature,
                              beta=beta, target_tokens=target_tokens, sm_scale=sm_scale,
                              iters=iters, num_splits=num_splits, csr_out=csr_out)


def merge_paged_attention_results(left: PagedSparseAttentionResult,
                                  right: PagedSparseAttentionResult) -> PagedSparseAttentionResult:
    """Exact LSE merge of two disjoint key sets (paged_attention.py:50-80)."""
    if left.logsumexp is None or right.logsumexp is None:
        raise ValueError("attention-state merge requires logsumexp from both inputs")
    merged = torch.logaddexp(left.logsumexp.float(), right.logsumexp.float())
    wl = torch.exp(left.logsumexp.float() - merged)
    wr = torch.exp(right.logsumexp.float() - merged)
    out = (left.output.float() * wl.unsqueeze(-1) + right.output.float() * wr.unsqueeze(-1))
    return PagedSparseAttentionResult(output=out.to(left.output.dtype), logsumexp=merged)
