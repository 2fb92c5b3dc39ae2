"""KV-outer sparse prefill attention (S4 + S5 + S6) on HIP.

The reference (semblo/vllm_plugin/kv_outer.py:482-816) builds a reverse index
from each query's selected clusters, makes one FA3 varlen call per
(cluster, KV head) whose query rows are the queries that picked it, one FA3
call over the chunk's own causal window, and folds the partials per query by
log-sum-exp.  Here the same three steps are three libsbsa calls:

  sbsa_reverse_index    the CSR (query ids per (head, cluster)) and each
                        query's rank in its clusters' lists     (kv_outer.py:254-329)
  sbsa_prefill_items +  one persistent MFMA kernel over a work list of
  sbsa_prefill_attend   (head, cluster | window, 128/G queries) items,
                        partials in bf16 with their LSE        (kv_outer.py:661-753)
  sbsa_prefill_combine  window first, then the clusters in order (kv_outer.py:370-479)

One host read per call (the entry count, which sizes the partial buffer), as
in the reference (kv_outer.py:604-613), or none: the partial rows are then
sized by a bound known on the host, capped in bytes (PartialsGuard).
"""
from __future__ import annotations

import os

import torch

from . import _lib

# int32 fields of one work item {head, cluster, first query slot, count,
# visible rows, first partial slot, first packed row, 0}
ITEM_INTS = 8


def queries_per_item(q_per_kv: int) -> int:
    """Queries of one work item: the kernel's (query, head) rows per item over G."""
    return _lib.query("sbsa_prefill_item_rows") // q_per_kv


def build_reverse_index(qmask: torch.Tensor, live: torch.Tensor, *, num_queries: int,
                        block_q: int = 64, capacity=None):
    """qmask [Q, H, C/32] int32, live [H, C] int32 (> 0: the cluster has visible rows).

    Returns (qvals, counts [H, C], indptr [H*C + 1] int32, nnz (device int64),
    qrank [Q, H, C] int32): qvals lists, per (head, cluster), the ascending
    query ids that selected it; qrank[q, h, c] is q's place in that list.
    """
    q_all, hkv, nw = qmask.shape
    c = nw * 32
    dev = qmask.device
    counts = torch.empty(hkv, c, dtype=torch.int32, device=dev)
    indptr = torch.empty(hkv * c + 1, dtype=torch.int32, device=dev)
    nnz = torch.empty(1, dtype=torch.int64, device=dev)
    cap = max(num_queries * hkv * c, 1)
    qvals = torch.empty(cap, dtype=torch.int32, device=dev)
    qrank = torch.empty(num_queries, hkv, c, dtype=torch.int32, device=dev)
    live32 = live if live.dtype == torch.int32 and live.is_contiguous() else live.to(torch.int32).contiguous()
    _lib.call("sbsa_reverse_index", _lib.ptr(qmask), num_queries, hkv, c, _lib.ptr(live32),
              _lib.ptr(counts), _lib.ptr(indptr), _lib.ptr(nnz), _lib.ptr(qvals), cap,
              _lib.ptr(qrank), _lib.stream(dev))
    return qvals, counts, indptr, nnz, qrank


def kv_outer_attention(q: torch.Tensor, packed_kv: torch.Tensor, qmask: torch.Tensor,
                       causal_sizes: torch.Tensor, bucket_indptr: torch.Tensor, *, sm_scale: float,
                       page_size: int = 16, aligned: bool = True, local_kv=None,
                       chunk_start: int | None = None, wstart: int | None = None,
                       out: torch.Tensor | None = None, want_stats: bool = False,
                       grid: int | None = None, timing=None, **unused):
    """Attention with the cluster outside and its queries gathered (kv_outer.py:482-499).

    q [Q, Hq, D] bf16; packed_kv [2, Lp, Hkv, D]; qmask [Q, Hkv, C/32];
    causal_sizes [Hkv, C] (visible rows per cluster: every visible row of a
    selected cluster precedes the chunk); bucket_indptr [Hkv, C+1];
    local_kv = (k, v), each [n_local, Hkv, D], the prompt-order window whose
    first row is position ``wstart`` and whose last is the chunk's last query.
    Returns (out [Q, Hq, D], stats).
    """
    if not aligned:
        raise NotImplementedError("the packed layout is always page-aligned (SEMBLO_FA3_ALIGN=16)")
    if local_kv is None:
        raise NotImplementedError("the KV-outer body always merges the chunk's causal window")
    qn, hq, d = q.shape
    hkv = packed_kv.shape[2]
    g = hq // hkv
    c = qmask.shape[2] * 32
    dev = q.device
    _lib.require_device(q, packed_kv, qmask, causal_sizes, bucket_indptr)
    k_loc, v_loc = local_kv
    n_local = k_loc.shape[0]
    if wstart is None:
        wstart = 0
    if chunk_start is None:
        chunk_start = wstart + n_local - qn
    if n_local != chunk_start + qn - wstart:
        raise ValueError("the local window must run from wstart to the chunk's last query")
    if k_loc.stride() != v_loc.stride():
        raise ValueError("the window's K and V must share a layout")
    plan = kv_outer_plan(qmask, causal_sizes, num_queries=qn)
    nnz = int(plan.nnz_d.item())                  # the one host read of the chunk
    return kv_outer_execute(q, packed_kv, plan, nnz, bucket_indptr, sm_scale=sm_scale,
                            local_kv=local_kv, chunk_start=chunk_start, wstart=wstart, out=out,
                            want_stats=want_stats, grid=grid, timing=timing)


class KVOuterPlan:
    """The reverse index of one chunk (kv_outer.py:254-329): everything the
    attention needs from the selection, built before the one host read.  ``work``:
    the chunk's work list and queue when ``prepare_work`` built them ahead, on the
    plan's stream, with the partial capacity they were built for."""

    def __init__(self, qmask, nvis, qvals, counts, rev_indptr, nnz_d, qrank):
        self.qmask, self.nvis, self.qvals, self.counts = qmask, nvis, qvals, counts
        self.rev_indptr, self.nnz_d, self.qrank = rev_indptr, nnz_d, qrank
        self.work = None

    def prepare_work(self, q: torch.Tensor, hkv: int, bucket_indptr: torch.Tensor,
                     guard: "PartialsGuard | None" = None) -> None:
        """Build the work list ``kv_outer_execute`` would build for this chunk, with
        its capacity bound (nothing is read on the host), on the current stream."""
        qn, hq, d = q.shape
        c = self.qmask.shape[2] * 32
        cap, capped = partials_room(qn, hkv, c, hq // hkv, d, q.element_size(), guard)
        items, queue = build_work_list(self, hkv, c, qn, queries_per_item(hq // hkv), bucket_indptr,
                                       cap, capped, q.device)
        arrived = None
        if capped:
            # the overflow flag is final once the work list is built: copied to the host
            # here, the chunk can be settled as soon as its plan is done, not after its
            # attention
            flag = torch.empty(1, dtype=torch.int32, pin_memory=True)
            flag.copy_(queue[QUEUE_OVERFLOW:QUEUE_OVERFLOW + 1], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            arrived = (ev, flag)
        self.work = (cap, capped, items, queue, arrived)

    def tensors(self):
        """The device tensors a chunk's execution reads (for record_stream)."""
        t = [self.qmask, self.nvis, self.qvals, self.counts, self.rev_indptr, self.nnz_d, self.qrank]
        if self.work is not None:
            t += [self.work[2], self.work[3]]
        return t


def kv_outer_plan(qmask: torch.Tensor, causal_sizes: torch.Tensor, *, num_queries: int) -> KVOuterPlan:
    """The reverse index of a chunk's selection (no host read)."""
    nvis = causal_sizes if causal_sizes.dtype == torch.int32 else causal_sizes.to(torch.int32)
    nvis = nvis.contiguous()
    qvals, counts, rev_indptr, nnz_d, qrank = build_reverse_index(qmask, nvis, num_queries=num_queries)
    return KVOuterPlan(qmask, nvis, qvals, counts, rev_indptr, nnz_d, qrank)


# int32 words of a work queue: per-XCD counts, offsets and counters, then the
# overflow flag (word QUEUE_OVERFLOW)
QUEUE_INTS = 32
QUEUE_OVERFLOW = 24


def partials_capacity(num_queries: int, num_kv_heads: int, num_clusters: int) -> int:
    """A bound of a chunk's partial count known without reading the device: a query
    selects at most every cluster of each KV head (one partial per selected,
    visible (query, KV head, cluster))."""
    return int(num_queries) * int(num_kv_heads) * int(num_clusters)


def partials_cap_bytes() -> int:
    """SEMBLO_KV_OUTER_PARTIALS_CAP_MB (default 4096): the most bytes of partial rows a
    chunk enqueued without a host read may take.  Past it the rows are sized to this
    cap, and a chunk with more entries is run again at its exact count (the reference
    caps its index buffers the same way and reads the count above the cap,
    kv_outer.py:592-600)."""
    return int(float(os.environ.get("SEMBLO_KV_OUTER_PARTIALS_CAP_MB", "4096")) * (1 << 20))


class PartialsGuard:
    """The chunks enqueued with a capped partial buffer, each with its overflow flag.

    ``watch`` copies a chunk's flag to pinned memory behind its work (no wait);
    ``poll`` settles the chunks whose flag has arrived, ``finish`` waits for the rest.
    A chunk that overflowed ran nothing (its work list was empty and its combine
    skipped): it is run again with its exact partial count, read on the host, and the
    guard's later chunks get room for 1.25 times that count (``cap_entries``), since
    the counts grow along a prompt."""

    def __init__(self):
        self._pending = []
        self._next = 0
        self.reruns = 0
        self.cap_entries = 0

    def watch(self, queue: torch.Tensor, rerun, arrived=None) -> None:
        """``arrived``: (event, pinned flag) when the flag was copied already, on the
        stream that built the work list; else it is copied here, behind the chunk."""
        if arrived is None:
            flag = torch.empty(1, dtype=torch.int32, pin_memory=True)
            flag.copy_(queue[QUEUE_OVERFLOW:QUEUE_OVERFLOW + 1], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
        else:
            ev, flag = arrived
        self._pending.append((self._next, ev, flag, rerun))
        self._next += 1

    def mark(self) -> int:
        """A mark: the chunks watched from now on are not below it."""
        return self._next

    def poll(self, wait: bool = False, wait_below: int | None = None) -> None:
        """Settle chunks: with ``wait`` every one; with ``wait_below`` exactly those watched
        before that mark (waiting for them), so that which chunks run again, and the room
        the later ones get, does not depend on timing; otherwise those whose flags have
        arrived."""
        keep = []
        for seq, ev, flag, rerun in self._pending:
            if wait_below is not None and not wait:
                if seq >= wait_below:
                    keep.append((seq, ev, flag, rerun))
                    continue
                ev.synchronize()
            elif wait:
                ev.synchronize()
            elif not ev.query():
                keep.append((seq, ev, flag, rerun))
                continue
            if int(flag[0]):
                self.reruns += 1
                rerun()
        self._pending = keep

    def finish(self) -> None:
        self.poll(wait=True)


def partials_room(qn: int, hkv: int, c: int, g: int, d: int, elem_size: int,
                  guard: PartialsGuard | None = None) -> tuple[int, bool]:
    """(entries of the chunk's partial rows, capped): the capacity bound, capped at
    ``partials_cap_bytes`` (or at the guard's room for the counts seen so far)."""
    cap = partials_capacity(qn, hkv, c)
    entry_bytes = g * d * elem_size + g * 4
    limit = max(1, partials_cap_bytes() // entry_bytes)
    if guard is not None:
        limit = max(limit, guard.cap_entries)
    return (limit, True) if cap > limit else (cap, False)


def build_work_list(plan: KVOuterPlan, hkv: int, c: int, qn: int, qt: int, bucket_indptr: torch.Tensor,
                    cap: int, capped: bool, dev):
    """The chunk's work items (sbsa_prefill_items) and its claim queue, on the
    current stream."""
    bound = _lib.query("sbsa_prefill_items_bound", cap, qn, hkv, c, qt)
    items = torch.empty(max(bound, 1), ITEM_INTS, dtype=torch.int32, device=dev)
    queue = torch.empty(QUEUE_INTS, dtype=torch.int32, device=dev)
    _lib.call("sbsa_prefill_items", _lib.ptr(plan.counts), hkv, c, qn, qt, 1, _lib.ptr(bucket_indptr),
              _lib.ptr(plan.nvis), _lib.ptr(plan.rev_indptr), _lib.ptr(items), bound,
              cap if capped else 0, _lib.ptr(queue), _lib.stream(dev))
    return items, queue


def kv_outer_execute(q: torch.Tensor, packed_kv: torch.Tensor, plan: KVOuterPlan, nnz: int | None,
                     bucket_indptr: torch.Tensor, *, sm_scale: float, local_kv, chunk_start: int,
                     wstart: int, out: torch.Tensor | None = None, want_stats: bool = False,
                     grid: int | None = None, timing=None, guard: PartialsGuard | None = None):
    """The work list, the attention and the combine of one chunk, given its plan and
    its partial count ``nnz`` read on the host, or None: the partial rows are then
    sized by ``partials_capacity``, capped at ``partials_cap_bytes``, and nothing
    waits for the plan on the host (the kernels take the count and the entries from
    the plan's device arrays).  A capped chunk is settled through ``guard`` (its
    overflow flag is read later, and the chunk run again if it overflowed), or, with
    no guard, at once (one host read)."""
    qn, hq, d = q.shape
    hkv = packed_kv.shape[2]
    g = hq // hkv
    qmask, nvis, qvals, counts = plan.qmask, plan.nvis, plan.qvals, plan.counts
    rev_indptr, qrank = plan.rev_indptr, plan.qrank
    c = qmask.shape[2] * 32
    dev = q.device
    k_loc, v_loc = local_kv
    capped = False
    if nnz is not None:
        cap = nnz
    else:
        cap, capped = partials_room(qn, hkv, c, g, d, q.element_size(), guard)
    if out is None:
        out = torch.empty_like(q)
    part_o = torch.empty(max(cap, 1), g, d, dtype=q.dtype, device=dev)
    part_lse = torch.empty(max(cap, 1), g, dtype=torch.float32, device=dev)
    local_o = torch.empty_like(q)
    local_lse = torch.empty(qn, hq, dtype=torch.float32, device=dev)
    s = _lib.stream(dev)
    arrived = None
    if plan.work is not None and nnz is None and plan.work[:2] == (cap, capped):
        # built ahead on the plan's stream (KVOuterPlan.prepare_work); used once
        items, queue, arrived = plan.work[2], plan.work[3], plan.work[4]
        plan.work = None
    else:
        items, queue = build_work_list(plan, hkv, c, qn, queries_per_item(g), bucket_indptr, cap, capped,
                                       dev)
    if timing is not None:
        timing.begin(s, "sparse")
    _lib.call("sbsa_prefill_attend", _lib.ptr(q), q.stride(0), q.stride(1), qn, hq, hkv, d,
              _lib.ptr(packed_kv), packed_kv.shape[1], _lib.ptr(k_loc), _lib.ptr(v_loc),
              k_loc.stride(0), k_loc.stride(1), _lib.ptr(bucket_indptr), _lib.ptr(nvis), c,
              _lib.ptr(rev_indptr), _lib.ptr(qvals), _lib.ptr(items), _lib.ptr(queue),
              _lib.ptr(part_o), _lib.ptr(part_lse), _lib.ptr(local_o),
              local_o.stride(0), local_o.stride(1), _lib.ptr(local_lse), int(chunk_start),
              int(wstart), float(sm_scale), int(grid or 0), s)
    if timing is not None:
        timing.end(s)
    _lib.call("sbsa_prefill_combine", _lib.ptr(qmask), _lib.ptr(nvis), _lib.ptr(rev_indptr),
              _lib.ptr(qrank), _lib.ptr(part_o), _lib.ptr(part_lse), _lib.ptr(local_o),
              local_o.stride(0), local_o.stride(1), _lib.ptr(local_lse), _lib.ptr(out),
              out.stride(0), out.stride(1), None, qn, hq, hkv, d, c,
              _lib.ptr(queue[QUEUE_OVERFLOW:]) if capped else None, s)
    if capped:
        # a run again reads the run starts as this chunk's plan saw them: a token-order
        # session may lay the runs out again (into its other store) before the flag is read
        indptr_seen = bucket_indptr.clone() if guard is not None else bucket_indptr

        def rerun():
            exact = int(plan.nnz_d.item())
            if guard is not None:
                guard.cap_entries = max(guard.cap_entries, exact + exact // 4)
            kv_outer_execute(q, packed_kv, plan, exact, indptr_seen,
                             sm_scale=sm_scale, local_kv=local_kv, chunk_start=chunk_start,
                             wstart=wstart, out=out, grid=grid, timing=timing)
        if guard is not None:
            guard.watch(queue, rerun, arrived)
        elif int(queue[QUEUE_OVERFLOW].item()):
            rerun()
    stats = {"partials": nnz}
    if want_stats:
        stats["charged"] = int((counts.to(torch.int64) * nvis.to(torch.int64)).sum())
        stats["kv_read"] = int(nvis.to(torch.int64).sum())
    return out, stats


_ZEROS: dict = {}


def _zero_counts(n: int, dev) -> torch.Tensor:
    """A zero int32 buffer of at least ``n`` entries on ``dev``, made once: the dense
    chunks' work list reads it as empty cluster counts and never writes it."""
    key = torch.device(dev)
    z = _ZEROS.get(key)
    if z is None or z.numel() < n:
        z = torch.zeros(max(n, 1024), dtype=torch.int32, device=dev)
        # once: the fill has landed before any stream reads the buffer
        torch.cuda.current_stream(z.device).synchronize()
        _ZEROS[key] = z
    return z


def dense_causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, sm_scale: float,
                           chunk_start: int = 0, out: torch.Tensor | None = None,
                           grid: int | None = None, timing=None) -> torch.Tensor:
    """Exact causal attention of q (positions chunk_start..) over k/v rows 0..chunk_end
    in prompt order (fused_prefill.py:155-189, the dense-prefix chunks)."""
    qn, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    dev = q.device
    _lib.require_device(q, k, v)
    if k.shape[0] < chunk_start + qn:
        raise ValueError("k/v must cover every position up to the chunk's last query")
    qt = queries_per_item(g)
    zero_counts = _zero_counts(hkv * 32, dev)
    bound = hkv * ((qn + qt - 1) // qt) + 1
    items = torch.empty(bound, ITEM_INTS, dtype=torch.int32, device=dev)
    queue = torch.empty(QUEUE_INTS, dtype=torch.int32, device=dev)
    if out is None:
        out = torch.empty_like(q)
    s = _lib.stream(dev)
    # no cluster has queries: the index arrays are never read
    _lib.call("sbsa_prefill_items", _lib.ptr(zero_counts), hkv, 32, qn, qt, 1, _lib.ptr(zero_counts),
              _lib.ptr(zero_counts), _lib.ptr(zero_counts), _lib.ptr(items), bound, 0, _lib.ptr(queue), s)
    if timing is not None:
        timing.begin(s, "dense")
    _lib.call("sbsa_prefill_attend", _lib.ptr(q), q.stride(0), q.stride(1), qn, hq, hkv, d,
              None, 0, _lib.ptr(k), _lib.ptr(v), k.stride(0), k.stride(1), None, None, 32, None,
              None, _lib.ptr(items), _lib.ptr(queue), None, None,
              _lib.ptr(out), out.stride(0), out.stride(1), None, int(chunk_start), 0,
              float(sm_scale), int(grid or 0), s)
    if timing is not None:
        timing.end(s)
    return out


class KernelTiming:
    """HIP events around each launch of the attention kernel, on the stream it runs on.

    ``begin``/``end`` bracket one launch; ``flops`` collects the algorithmic
    FLOPs of each launch as device scalars (summed once, at read-out).  With
    ``counts_flops`` false only the events are recorded: nothing but event
    records is added to the stream, so the timing can run inside a timed region."""

    def __init__(self, counts_flops: bool = True) -> None:
        self.events: list[tuple] = []
        self.kinds: list = []
        self.flops: list = []
        self.counts_flops = counts_flops

    def begin(self, stream_handle: int, kind: str | None = None) -> None:
        """``kind``: what the launch is (the attention's dense or sparse chunks), for a
        split of the totals."""
        # the kernels launch on torch's current stream (the handle passed to libsbsa)
        assert stream_handle == torch.cuda.current_stream().cuda_stream
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self.events.append([ev, None])
        self.kinds.append(kind)

    def end(self, stream_handle: int) -> None:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self.events[-1][1] = ev

    def add_flops(self, value) -> None:
        if self.counts_flops:
            self.flops.append(value)

    def launches(self) -> int:
        return len(self.events)

    def total_ms(self) -> float:
        torch.cuda.synchronize()
        return float(sum(a.elapsed_time(b) for a, b in self.events))

    def total_flops(self) -> float:
        return float(sum(float(f) for f in self.flops))

    def split(self, kind: str, steps: int = 1) -> tuple[float, int]:
        """(ms per step, launches per step) of the launches of one kind."""
        torch.cuda.synchronize()
        sel = [i for i, k in enumerate(self.kinds) if k == kind]
        ms = sum(self.events[i][0].elapsed_time(self.events[i][1]) for i in sel)
        return ms / max(steps, 1), len(sel) // max(steps, 1)

    def split_flops(self, kind: str) -> float:
        """The FLOPs of the launches of one kind (one FLOP entry per launch)."""
        return float(sum(float(f) for f, k in zip(self.flops, self.kinds) if k == kind))
