"""Token-order streamed prefill (S10): one slice of the prompt through a layer at a time.

Host side of the reference's semblo/vllm_plugin/token_outer_prefill.py, with
every array operation on the GPU through libsbsa.  In each sparse layer:

  dense   while a slice starts before the fit point, its K/V are staged in
          prompt order and it attends exactly over positions 0..p
          (token_outer_prefill.py:214-255);
  fit     at the first slice past the fit point, the clusters are fitted on
          the staged keys with the cluster count the whole prompt would get,
          and the staged keys move into a store laid out with a reservation
          per cluster sized from the observed proportions
          (token_outer_prefill.py:260-337; sbsa_relayout_runs);
  append  every later slice assigns its keys to the fixed clusters
          (sbsa_nearest_cluster), appends them behind their cluster's last key
          (sbsa_append_rows, sbsa_append_kv) and attends through the KV-outer
          body with the counts before the slice, its own keys through the exact
          window (token_outer_prefill.py:339-364);
  repack  a cluster that outgrows its reservation lays the runs out again from
          the current proportions (token_outer_prefill.py:366-392;
          sbsa_repack_runs into the other buffer of a double-buffered store);
  finish  the index and the packed store become the layer's decode state.

Slices that start after the fit but within the dense prefix (start <= x*K)
are still exact causal attention: their keys are read back in prompt order
through the inverse map (sbsa_gather_rows), as the reference's fused body
does (token_outer_prefill.py:155-159).

Host reads: one per appended slice (the overflow flags, the reference's
``bool((sizes + counts > reserve).any())``), and the cluster sizes at the
fit and at a repack, from which the reserved layout is computed on the host.
They arrive by an asynchronous copy into pinned memory.  A sparse slice reads
no row of its own slice from the store, so its attention is enqueued between
the assignment and that read: the GPU runs it while the host waits for the
flags and lays out any repack, which then follows the attention on the stream.
"""
from __future__ import annotations

import os

import numpy as np
import torch

from . import _lib
from .config import num_flat_clusters
from .kv_outer import PartialsGuard, dense_causal_attention
from .state import PACK_ALIGN, ProductPostingIndex


def reserved_layout(sizes_ref: torch.Tensor, n_ref: int, total_tokens: int, width: int,
                    align: int) -> torch.Tensor:
    """Rows reserved per cluster, [Hkv, C] int64 on the host (token_outer_prefill.py:39-63).

    Each cluster gets its share of ``total_tokens`` in the proportion it had
    among the ``n_ref`` reference keys, rounded up to whole pages of
    ``align`` rows and never below one page (an empty cluster may still
    receive keys); the pages left in ``width`` are spread in the same
    proportions.  Raises RuntimeError if the rounded shares alone exceed
    ``width``.
    """
    align = max(int(align), 1)
    # This runs between a host read and the repack it decides, while the GPU waits,
    # so it is a few whole-array operations over every KV head at once: elementwise
    # float64 in numpy (exact, like torch's), row sums in torch (its summation order).
    share_t = sizes_ref.detach().to("cpu", torch.float64) * (float(total_tokens) / float(max(int(n_ref), 1)))
    share = share_t.numpy()
    rows = np.maximum(np.ceil(share / align).astype(np.int64), 1) * align
    need = rows.sum(1)
    spare = int(width) - need
    if (spare < 0).any():
        h = int(np.flatnonzero(spare < 0)[0])
        raise RuntimeError(f"the reserved layout needs {int(need[h])} rows for KV head {h}; "
                           f"the store holds {width}")
    total = np.maximum(share_t.sum(1, keepdim=True).numpy(), 1.0)
    extra = np.floor((share / total) * (spare // align)[:, None].astype(np.float64)).astype(np.int64) * align
    rows += np.where((spare >= align)[:, None], extra, 0)
    return torch.from_numpy(rows)


def nearest_cluster(keys: torch.Tensor, codebooks: torch.Tensor, *, router_pass: bool = True,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """[n, Hkv, D] keys -> [Hkv, n] int32 cluster ids (suffix_flush.py:154-170 after the
    key router and routing_space): cosine in fp32, all-zero descriptors never chosen."""
    n, hkv, d = keys.shape
    c = int(codebooks.shape[2])
    if keys.stride(-1) != 1:
        keys = keys.contiguous()
    if out is None:
        out = torch.empty(hkv, n, dtype=torch.int32, device=keys.device)
    _lib.call("sbsa_nearest_cluster", _lib.ptr(keys), n, keys.stride(0), keys.stride(1), hkv, d,
              int(bool(router_pass)), _lib.ptr(codebooks), c, _lib.ptr(out), _lib.stream(keys.device))
    return out


def append_rows(ids: torch.Tensor, indptr: torch.Tensor, sizes: torch.Tensor,
                reserve: torch.Tensor | None = None):
    """Destination rows [Hkv, n] int32 of a slice's keys and per-cluster counts [Hkv, C]
    (token_outer_prefill.py:66-87), plus the overflow flags [Hkv] when ``reserve`` is
    given (bit 0: some cluster would outgrow its reservation)."""
    hkv, n = ids.shape
    c = int(sizes.shape[1])
    dev = ids.device
    rows = torch.empty(hkv, n, dtype=torch.int32, device=dev)
    counts = torch.empty(hkv, c, dtype=torch.int32, device=dev)
    flags = torch.zeros(hkv, dtype=torch.int32, device=dev)
    res = None if reserve is None else reserve.to(device=dev, dtype=torch.int32).contiguous()
    ids = ids.contiguous()
    _lib.call("sbsa_append_rows", _lib.ptr(ids), n, hkv, c, _lib.ptr(indptr),
              _lib.ptr(sizes), _lib.ptr(res), _lib.ptr(rows), _lib.ptr(counts), _lib.ptr(flags),
              _lib.stream(dev))
    return rows, counts, flags


def gather_rows(index: ProductPostingIndex, first: int, n: int):
    """K/V of positions first..first+n-1 in prompt order, [n, Hkv, D] each, read through
    the inverse map."""
    packed = index.packed_kv
    hkv, d = packed.shape[2], packed.shape[3]
    k = torch.empty(n, hkv, d, dtype=packed.dtype, device=packed.device)
    v = torch.empty_like(k)
    inv = index.inverse_positions()
    _lib.call("sbsa_gather_rows", _lib.ptr(packed), packed.shape[1], hkv, d, _lib.ptr(inv),
              inv.shape[1], int(first), int(n), _lib.ptr(k), _lib.ptr(v), k.stride(0), k.stride(1),
              _lib.stream(packed.device))
    return k, v


class TokenOuterSnapshot:
    """The counts the sparse body reads under this schedule (token_outer_prefill.py:90-125).

    ``sizes`` [Hkv, C] are the keys appended by earlier slices, i.e. the rows
    of every cluster visible to the slice being attended; the slice's own
    keys are in the store but not counted here and are attended through its
    exact window.
    """

    def __init__(self, index: ProductPostingIndex) -> None:
        self.length = int(index.prompt_length)
        self.sizes = torch.zeros_like(index.bucket_sizes)
        self.chunk_start = 0

    def advance(self, last_pos: int) -> torch.Tensor:
        if int(last_pos) + 1 != self.chunk_start:
            raise RuntimeError(
                f"the token-outer snapshot holds the counts before position {self.chunk_start}; "
                f"the body asked for position {last_pos}")
        return self.sizes


class TokenOuterPrefillSession:
    """One sparse layer's share of a token-order prefill (token_outer_prefill.py:127-400).

    ``slice(hidden_states, start, stop)`` is the reference's call: it projects the
    slice with the projections the model attached to the layer
    (``SembloAttention.attach_projections``) and returns the layer's output rows.
    ``slice_projected`` takes the projections of positions [start, stop) instead --
    q_post [n, Hq, D], q_pre [n, Hq, D], k_pre, k_post, v [n, Hkv, D].  Slices must
    come in order and cover the prompt.
    """

    def __init__(self, layer, tokens: int, chunk: int, *, fit_tokens: int | None = None,
                 rope_positions: torch.Tensor | None = None) -> None:
        cfg = layer.runtime_config
        self.layer = layer
        self.tokens = int(tokens)
        # the rotary positions [T] or [3, T] the reference's session slices for its
        # projections; None: 0 .. T-1 on the hidden states' device
        self.rope_positions = rope_positions
        self.chunk = int(chunk)
        if self.chunk > int(cfg.query_chunk_size):
            raise RuntimeError(
                f"SEMBLO_PREFILL_CHUNK={self.chunk} must not exceed the query chunk "
                f"({cfg.query_chunk_size}): a slice's keys are appended once, before its queries")
        self.target = cfg.budget(self.tokens)
        self.cap = int(cfg.dense_prefix_x) * self.target
        if fit_tokens is None:
            fit_tokens = int(os.environ.get("SEMBLO_TOKEN_OUTER_FIT_TOKENS", "65536"))
        fit_tokens = min(int(fit_tokens), self.cap) if int(fit_tokens) > 0 else self.cap
        self.fit_at = min(self.tokens, ((fit_tokens // self.chunk) + 1) * self.chunk)
        self.stage_k = self.stage_v = self.stage_kpre = None
        self.index: ProductPostingIndex | None = None
        self.snapshot: TokenOuterSnapshot | None = None
        self.reserve: torch.Tensor | None = None
        self._reserve_dev: torch.Tensor | None = None
        self.repacks = 0
        self.repacks_with_slice = 0                 # repacks whose layout counts the slice's keys
        self.guard = PartialsGuard()                # sparse slices whose partial rows were capped
        self.next_start = 0
        self._spare: torch.Tensor | None = None     # the other buffer of the store, after a repack
        self._host: torch.Tensor | None = None      # pinned: the append's flags, counts and sizes
        self.verbose = os.environ.get("SEMBLO_VERBOSE", "0") == "1"
        layer.target_tokens = self.target

    def _set_reserve(self, reserve: torch.Tensor, device) -> None:
        """The reservation [Hkv, C] on the host (for the layout) and on the device (for
        the overflow test), the latter by an asynchronous copy from pinned memory, so
        that setting it never waits for the GPU."""
        self.reserve = reserve
        staged = reserve.to(torch.int32).pin_memory()
        self._reserve_dev = staged.to(device, non_blocking=True)

    # -- per slice ------------------------------------------------------------------
    def slice(self, hidden_states: torch.Tensor, start: int, stop: int) -> torch.Tensor:
        """The layer's output rows for positions [start, stop): the slice projected with
        the layer's projections, its keys appended, its queries attended, then gated and
        projected out (token_outer_prefill.py:173-196)."""
        layer = self.layer
        n = int(stop) - int(start)
        if int(hidden_states.shape[0]) != n:
            raise ValueError(f"{hidden_states.shape[0]} hidden rows for the slice [{start}, {stop})")
        if self.rope_positions is None:
            rope = torch.arange(int(start), int(stop), device=hidden_states.device)
        else:
            rope = layer._slice_positions(self.rope_positions, int(start), int(stop))
        q_post, k_post, v, q_pre, k_pre, gate = layer._project_qkv(rope, hidden_states)
        if k_post is None or v is None or k_pre is None:
            raise RuntimeError("the token-outer prefill needs a layer with its own K/V")
        attn = self.slice_projected(q_post, q_pre, k_pre, k_post, v, start, stop)
        return layer._finish_output(attn.view(n, -1), gate)

    def slice_projected(self, q_post, q_pre, k_pre, k_post, v, start: int, stop: int,
                        out: torch.Tensor | None = None, timing=None, store_timing=None) -> torch.Tensor:
        """Attention of positions [start, stop) into ``out`` [n, Hq, D].  ``timing``
        brackets the attention launches, ``store_timing`` the store kernels of an
        append (assignment, rows, K/V writes), each with HIP events."""
        if int(start) != self.next_start or not start < stop <= self.tokens:
            raise RuntimeError(f"slice [{start}, {stop}) out of order (next start {self.next_start}, "
                               f"{self.tokens} tokens)")
        layer = self.layer
        hq, hkv, d = layer.num_heads, layer.num_kv_heads, layer.head_dim
        n = stop - start
        q = q_post.reshape(n, hq, d)
        qp = q_pre.reshape(n, hq, d)
        kp = k_pre.reshape(n, hkv, d)
        kk = k_post.reshape(n, hkv, d)
        vv = v.reshape(n, hkv, d)
        _lib.require_device(q, qp, kp, kk, vv)
        if out is None:
            out = torch.empty_like(q)
        if self.index is None and start >= self.fit_at:
            self._fit_and_pack()
        if self.index is None:
            self._stage(kp, kk, vv, start, stop)
            self._count_dense(timing, start, n, hq, d)
            dense_causal_attention(q, self.stage_k[:stop], self.stage_v[:stop], sm_scale=layer.scaling,
                                   chunk_start=start, out=out, timing=timing)
        elif start <= self.cap:
            # a dense-prefix slice reads its own keys back from the store: append first
            self._append_commit(self._append_assign(kp, start, stop, store_timing), kk, vv, store_timing)
            self._attend(q, qp, kk, vv, start, stop, out, timing)
        else:
            # A sparse slice reads only rows of earlier positions (the counts before it);
            # its own keys come through the exact window.  Its attention is therefore
            # enqueued before the append's host read, and the GPU runs it while the host
            # waits for the flags and lays out any repack.
            pending = self._append_assign(kp, start, stop, store_timing)
            self.snapshot.sizes.copy_(self.index.bucket_sizes)
            self.snapshot.chunk_start = start
            pending["guard_mark"] = self.guard.mark()
            self._attend(q, qp, kk, vv, start, stop, out, timing)
            self._append_commit(pending, kk, vv, store_timing)
        self.next_start = stop
        return out

    def finish(self) -> ProductPostingIndex:
        if self.next_start != self.tokens:
            raise RuntimeError(f"the prefill stopped at {self.next_start} of {self.tokens} tokens")
        if self.index is None:
            # the prompt ended before the fit point: fit on all of it
            self.fit_at = self.tokens
            self._fit_and_pack()
        self.guard.finish()
        self._spare = None
        self.layer.adopt_index(self.index)
        return self.index

    # -- dense start ------------------------------------------------------------------
    def _stage(self, kp, kk, vv, start, stop) -> None:
        if self.stage_k is None:
            shape = (self.fit_at,) + tuple(kk.shape[1:])
            self.stage_k = kk.new_empty(shape)
            self.stage_v = vv.new_empty(shape)
            self.stage_kpre = kp.new_empty(shape)
        self.stage_k[start:stop] = kk
        self.stage_v[start:stop] = vv
        self.stage_kpre[start:stop] = kp

    @staticmethod
    def _count_dense(timing, start, n, hq, d) -> None:
        if timing is not None:
            timing.add_flops(4.0 * d * hq * (n * (start + 1) + n * (n - 1) // 2))

    # -- fit ----------------------------------------------------------------------------
    def _fit_and_pack(self) -> None:
        layer = self.layer
        cfg = layer.runtime_config
        p = self.fit_at
        unit = int(os.environ.get("SEMBLO_FLAT_UNIT_TOKENS", cfg.flat_unit_tokens))
        min_log2 = max(3, int(os.environ.get("SEMBLO_FLAT_MIN_CLUSTERS_LOG2", cfg.flat_min_clusters_log2)))
        clusters = num_flat_clusters(self.tokens, unit, min_log2)   # the count the whole prompt gets
        dev = self.stage_k.device
        index = ProductPostingIndex.build(
            self.stage_kpre[:p], torch.arange(p, device=dev), kmeans_sample_size=cfg.kmeans_sample_size,
            codebook_seed=cfg.codebook_seed + cfg.layer_idx, flat_unit_tokens=unit,
            flat_min_clusters_log2=min_log2, page_align=cfg.page_align, router_pass=True,
            num_clusters=clusters)
        hkv, d = self.stage_k.shape[1], self.stage_k.shape[2]
        align = max(int(index.page_align), 1)
        c = index.num_buckets
        width = self.tokens + c * align
        width += (-width) % PACK_ALIGN
        self._set_reserve(reserved_layout(index.bucket_sizes, p, self.tokens, width, align), dev)
        indptr_h = torch.zeros(hkv, c + 1, dtype=torch.int32)
        indptr_h[:, 1:] = torch.cumsum(self.reserve, 1).to(torch.int32)
        indptr = indptr_h.to(dev)
        packed = torch.zeros(2, width, hkv, d, dtype=self.stage_k.dtype, device=dev)
        posting = torch.zeros(hkv, width, dtype=torch.int32, device=dev)
        inverse = torch.zeros(hkv, self.tokens, dtype=torch.int32, device=dev)
        old_rows = index.inverse_positions()                          # [Hkv, p] rows of the fitted layout
        _lib.call("sbsa_relayout_runs", _lib.ptr(self.stage_k), _lib.ptr(self.stage_v),
                  self.stage_k.stride(0), self.stage_k.stride(1), p, hkv, d, _lib.ptr(old_rows),
                  old_rows.stride(0), _lib.ptr(index.bucket_indptr), _lib.ptr(indptr), c,
                  _lib.ptr(packed), width, _lib.ptr(posting), width, _lib.ptr(inverse), self.tokens,
                  _lib.stream(dev))
        index.packed_kv = packed
        index.posting_positions = posting
        index.bucket_indptr = indptr
        index._inverse_positions = inverse
        index.prompt_length = self.tokens
        index.max_position = self.tokens - 1
        index.extras["reserve"] = self.reserve
        self.index = index
        self.snapshot = TokenOuterSnapshot(index)
        self.stage_k = self.stage_v = self.stage_kpre = None

    # -- append ---------------------------------------------------------------------------
    def _append_assign(self, kp, start, stop, store_timing=None):
        """Enqueue the slice's assignment and the copy of what the host decides on:
        overflow flags, the slice's counts and the sizes so far, into pinned memory."""
        index = self.index
        hkv = kp.shape[1]
        c = index.num_buckets
        s = _lib.stream(kp.device)
        if store_timing is not None:
            store_timing.begin(s)
        ids = nearest_cluster(kp, index.codebooks, router_pass=True)
        rows, counts, flags = append_rows(ids, index.bucket_indptr, index.bucket_sizes, self._reserve_dev)
        if store_timing is not None:
            store_timing.end(s)
        words = hkv + 2 * hkv * c
        if self._host is None or self._host.numel() != words:
            self._host = torch.empty(words, dtype=torch.int32, pin_memory=True)
        self._host.copy_(torch.cat([flags, counts.flatten(), index.bucket_sizes.flatten()]),
                         non_blocking=True)
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(kp.device))
        return dict(ids=ids, rows=rows, counts=counts, ready=ready, start=int(start), stop=int(stop))

    def _append_commit(self, pending, kk, vv, store_timing=None) -> None:
        """The append's one host read per slice, any repack it decides, and the K/V
        writes (token_outer_prefill.py:339-364)."""
        index = self.index
        hkv, d = kk.shape[1], kk.shape[2]
        c = index.num_buckets
        start, stop = pending["start"], pending["stop"]
        n = stop - start
        s = _lib.stream(kk.device)
        ids, rows, counts = pending["ids"], pending["rows"], pending["counts"]
        pending["ready"].synchronize()
        # Capped chunks of earlier slices: their attention preceded this slice's assignment
        # on the stream, so their flags are in and nothing waits.  One that overflowed runs
        # again here, before this slice's repack: it reads the store its plan saw, which a
        # repack since then has left in the session's other buffer until this one.
        self.guard.poll(wait_below=pending.get("guard_mark", 0))
        host = self._host
        flags_h = host[:hkv]
        if bool((flags_h & 2).any()):
            raise RuntimeError("a key was assigned outside the cluster range")
        if bool((flags_h & 1).any()):
            counts_h = host[hkv:hkv + hkv * c].view(hkv, c).to(torch.int64)
            sizes_h = host[hkv + hkv * c:].view(hkv, c).to(torch.int64)
            width = index.packed_kv.shape[1]
            align = max(int(index.page_align), 1)
            reserve = reserved_layout(sizes_h, start, self.tokens, width, align)
            if bool((sizes_h + counts_h > reserve).any()):
                # The reference's layout, from the counts before the slice, still leaves a
                # cluster short (a burst of keys into a cluster that was small so far): the
                # reference appends anyway and those keys run into the next cluster's rows.
                # Here the runs are laid out with the slice's own keys counted, which
                # always fits; the reference's intermediate layout is skipped.
                reserve = reserved_layout(sizes_h + counts_h, start + n, self.tokens, width, align)
                self.repacks_with_slice += 1
            self._repack(start, reserve)
            rows, counts, _ = append_rows(ids, index.bucket_indptr, index.bucket_sizes, None)
        if kk.stride() != vv.stride() or kk.stride(-1) != 1:
            kk, vv = kk.contiguous(), vv.contiguous()
        packed, posting, inverse = index.packed_kv, index.posting_positions, index._inverse_positions
        if store_timing is not None:
            store_timing.begin(s)
        # the body sees the counts before this slice (snapshot.sizes); sizes advance past it
        _lib.call("sbsa_append_kv", _lib.ptr(kk), _lib.ptr(vv), kk.stride(0), kk.stride(1), n, hkv, d,
                  _lib.ptr(rows), int(start), _lib.ptr(packed), packed.shape[1], _lib.ptr(posting),
                  posting.shape[1], _lib.ptr(inverse), inverse.shape[1], _lib.ptr(index.bucket_sizes),
                  _lib.ptr(counts), c, _lib.ptr(self.snapshot.sizes), s)
        if store_timing is not None:
            store_timing.end(s)
            # algorithmic bytes: the slice's pre-RoPE keys and the descriptors read by the
            # assignment; K and V read and written once; ids, rows, posting and inverse entries
            store_timing.add_flops(float(n * hkv * d * 2 + hkv * c * d * 2 + 4 * n * hkv * d * 2
                                         + 4 * 5 * n * hkv))
        self.snapshot.chunk_start = start

    def _repack(self, n_so_far: int, reserve: torch.Tensor) -> None:
        """Lay the runs out again as ``reserve`` [Hkv, C] says (token_outer_prefill.py:366-392).

        The store is double-buffered: the keys of positions < ``n_so_far`` move in
        one pass from their rows in the current buffer to their rows in the other
        (sbsa_repack_runs), which then becomes the store."""
        index = self.index
        packed = index.packed_kv
        hkv, width, d = packed.shape[2], packed.shape[1], packed.shape[3]
        c = index.num_buckets
        new_ip = torch.zeros(hkv, c + 1, dtype=torch.int32, pin_memory=True)
        new_ip[:, 1:] = torch.cumsum(reserve, 1).to(torch.int32)
        new_ip = new_ip.to(packed.device, non_blocking=True)
        if self._spare is None:
            self._spare = torch.zeros_like(packed)
        dst = self._spare
        old_rows = index._inverse_positions[:, :n_so_far].clone()
        _lib.call("sbsa_repack_runs", _lib.ptr(packed), _lib.ptr(dst), width, hkv, d, n_so_far,
                  _lib.ptr(old_rows), old_rows.stride(0), _lib.ptr(index.bucket_indptr), _lib.ptr(new_ip),
                  c, _lib.ptr(index.posting_positions), index.posting_positions.shape[1],
                  _lib.ptr(index._inverse_positions), index._inverse_positions.shape[1],
                  _lib.stream(packed.device))
        index.packed_kv, self._spare = dst, packed
        index.bucket_indptr.copy_(new_ip)                             # same address as before
        self._set_reserve(reserve, packed.device)
        index.extras["reserve"] = reserve
        self.repacks += 1
        if self.verbose:
            print(f"[semblo_amd] token-order prefill layer {self.layer.layer_idx}: a cluster outgrew "
                  f"its reservation at position {n_so_far:,}; the store was laid out again "
                  f"(repack {self.repacks})", flush=True)

    # -- attention of an appended slice ---------------------------------------------------
    def _attend(self, q, qp, kk, vv, start, stop, out, timing) -> None:
        from .fused_prefill import fused_chunk_attention
        layer = self.layer
        cfg = layer.runtime_config
        n = stop - start
        if start <= self.cap:
            # within the dense prefix: exact causal attention over the store read in prompt order
            k_all, v_all = gather_rows(self.index, 0, stop)
            self._count_dense(timing, start, n, q.shape[1], q.shape[2])
            dense_causal_attention(q, k_all, v_all, sm_scale=layer.scaling, chunk_start=start, out=out,
                                   timing=timing)
            return
        qs = layer._query_state(qp)
        fused_chunk_attention(q, qs, self.index, None, self.snapshot, start, stop - 1,
                              temperature=cfg.selection_temperature, beta=cfg.bucket_size_penalty,
                              target_tokens=self.target, sm_scale=layer.scaling, iters=cfg.iters,
                              dense_prefix_x=cfg.dense_prefix_x, out=out, timing=timing,
                              window_kv=(kk, vv), plan_log=layer.plan_log, guard=self.guard)
