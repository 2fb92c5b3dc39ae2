"""The per-prompt index: flat spherical k-means block build and the packed K/V.

Host side of the reference's ``ProductPostingIndex`` on the flat paper path
(semblo/vllm_plugin/state.py:477-1012), with every array op on the GPU
through libsbsa:

  key_space        router + routing space            (routing_map.py:35-64, flat_index.py:144-166)
  kmeans_*         fit_flat_codebook                  (flat_index.py:193-289)
  kmeans_assign    assign_flat_buckets                (flat_index.py:376-383)
  bucket_layout    argsort/bincount + page alignment  (state.py:850-866, 44-84)
  pack_kv          pack_prompt_kv                     (state.py:950-997)

The random draws (the fit sample, the initial centroids and the restart rows
of empty clusters) come from a CPU ``torch.Generator`` seeded with
``codebook_seed``, in the reference's call order.  The reference draws on the
keys' device; drawing on the CPU makes the partition independent of the
device's RNG, and identical to the reference's own CPU build.  The
reference reads the cluster counts every k-means iteration (its
``empty.any()`` test).  Here the first RESTARTS_AHEAD restart draws of a head
are made ahead and applied on the GPU at the first iterations that leave a
cluster empty, the iterations run ahead, and one read of the counts tells
how many draws were used: the generator's state is set back before the first
unused one, and a later empty iteration is redone from there with its draw
made then.  The draws and the result are the reference's, with one host read
per head.

With an attention sink (SEMBLO_SINK_TOKENS=S, state.py:757-782) positions
0..S-1 form cluster 0, whose descriptor is zero, and the other positions are
fitted into clusters 1..C-1 by the same k-means over C-1 centroids.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

import torch

from . import _lib
from .config import check_sink_partition, fitted_sink_tokens, num_flat_clusters

PACK_ALIGN = 256
# restart draws of the k-means fit made ahead per KV head (the GPU applies them)
RESTARTS_AHEAD = 2


class _DrawBuffers:
    """Host buffers of the build's random draws, kept across builds of the same
    shape: the permutations are drawn into them (no fresh host pages per draw)
    and the sample and initial rows go to the device from pinned memory."""

    def __init__(self, length: int, fit_n: int, c: int):
        self.sub = torch.empty(fit_n, dtype=torch.int64)        # a host-side restart's draw
        # a head's draws (sample permutation, init rows, restart rows drawn ahead), in
        # two sets: the next head's are drawn ahead into the set the current head is not using
        self.sets = [_HeadDraws(length, fit_n) for _ in range(2)]
        self.pinned = torch.empty(fit_n + (1 + RESTARTS_AHEAD) * c, dtype=torch.int32,
                                  pin_memory=True)
        self.uploaded = None            # event after the last upload from `pinned`
        self.last_empties = 0           # empty k-means iterations of the last head fitted
        self.head_empties: dict = {}    # and of each KV head in the last build of this shape
        self.counts = None              # pinned [iterations, C] cluster counts

    def counts_host(self, iters: int, c: int) -> torch.Tensor:
        """Pinned host copy of the iterations' cluster counts (read after a stream
        synchronisation, so one buffer serves every build of this shape)."""
        if self.counts is None or self.counts.shape[0] < iters:
            self.counts = torch.empty(iters, c, dtype=torch.int32, pin_memory=True)
        return self.counts[:iters]


class _HeadDraws:
    """One KV head's permutations on the host."""

    def __init__(self, length: int, fit_n: int):
        self.perm = torch.empty(length, dtype=torch.int64)
        self.init = torch.empty(fit_n, dtype=torch.int64)
        self.restarts = torch.empty(RESTARTS_AHEAD, fit_n, dtype=torch.int64)


_DRAW_BUFFERS: dict = {}
_DRAW_AHEAD = None          # the worker thread that draws the next KV head's permutations ahead
DRAW_AHEAD = True           # False: every head's draws on the host thread, after its counts
DRAW_AHEAD_STATS = {"used": 0, "discarded": 0}


_DRAW_AHEAD_LAST = None     # the last draw submitted to it


def _draw_ahead_submit(fn, *args):
    global _DRAW_AHEAD, _DRAW_AHEAD_LAST
    if _DRAW_AHEAD is None:
        from concurrent.futures import ThreadPoolExecutor
        _DRAW_AHEAD = ThreadPoolExecutor(max_workers=1, thread_name_prefix="sbsa-draws")
    _DRAW_AHEAD_LAST = _DRAW_AHEAD.submit(fn, *args)
    return _DRAW_AHEAD_LAST


def _draw_ahead_settle() -> None:
    """Wait for a draw a build left running (one that raised before taking it): the
    next build of the same shape draws into the same host buffers."""
    fut = _DRAW_AHEAD_LAST
    if fut is not None and not fut.done():
        try:
            fut.result()
        except Exception:
            pass


def _draw_buffers(length: int, fit_n: int, c: int) -> _DrawBuffers:
    key = (length, fit_n, c)
    buf = _DRAW_BUFFERS.get(key)
    if buf is None:
        if len(_DRAW_BUFFERS) >= 4:
            _DRAW_BUFFERS.clear()
        buf = _DRAW_BUFFERS[key] = _DrawBuffers(length, fit_n, c)
    return buf


@dataclass
class ProductPostingIndex:
    """Flat-partition index of one layer's prompt (state.py:372-475 fields)."""

    codebooks: torch.Tensor            # [Hkv, 2, C, I/2] descriptors (key dtype)
    posting_positions: torch.Tensor    # [Hkv, W] int32 packed row -> position
    bucket_indptr: torch.Tensor        # [Hkv, C+1] int32 (page-aligned run starts)
    bucket_sizes: torch.Tensor         # [Hkv, C] int32
    prompt_length: int
    max_position: int
    flat_clusters: int
    page_align: int
    _inverse_positions: torch.Tensor   # [Hkv, L] int32 position -> packed row
    packed_kv: torch.Tensor | None = None
    original_kv: tuple | None = None   # prompt-order (k, v) [L, Hkv, D] while prefill runs
    extras: dict = field(default_factory=dict)

    @property
    def num_kv_heads(self) -> int:
        return int(self.codebooks.shape[0])

    @property
    def num_buckets(self) -> int:
        return int(self.flat_clusters)

    @property
    def num_centroids(self) -> int:
        return int(self.codebooks.shape[2])

    @property
    def is_flat(self) -> bool:
        return True

    @classmethod
    def build(cls, product_keys: torch.Tensor, positions: torch.Tensor, *, num_centroids: int = 128,
              kmeans_iters: int = 4, kmeans_sample_size: int = 8192,
              codebook_seed: int | None = 0, quantizer: str = "product",
              kmeans_init: str = "random", centroid_refiner=None, kmeans_preprocess: str = "none",
              flat_unit_tokens: int = 2048, flat_min_clusters_log2: int = 7, page_align: int = 16,
              descriptor_weight=None, descriptor_bias=None, descriptor_activation: str = "softplus",
              layer_idx: int | None = None, router_pass: bool = False,
              fit_iters: int | None = None, num_clusters: int | None = None,
              fit_trace: list | None = None, sink_tokens: int | None = None) -> "ProductPostingIndex":
        """Fit the flat codebook and the posting lists (state.py:477-542 contract).

        ``product_keys`` [L, Hkv, I] bf16 are the key router's output (or, with
        ``router_pass=True``, the pre-RoPE keys, normalised here first).
        ``positions`` must be 0..L-1.  ``num_centroids``, ``kmeans_iters``,
        ``quantizer`` and ``kmeans_init`` are accepted for signature parity;
        the flat path uses ``SEMBLO_FLAT_FIT_ITERS`` (default 8) iterations and
        32 sample points per centroid, as the reference does.

        ``fit_trace``, if given, receives one dict per KV head with the fit's
        intermediate states (the key space, the sample rows, and per iteration
        the centroids it starts from, its assignment, sums and counts; then the
        final centroids and assignment of every key, and the sample rows drawn to
        restart the clusters an iteration left empty), for parity checks of each
        k-means step.  The iterations then run one call at a time.  With a sink the
        fit covers positions S.. only, and so do the trace's rows, sample and final
        assignment (cluster ids 0..C-2 of that fit).

        ``sink_tokens``: S (None reads SEMBLO_SINK_TOKENS); 0 is the plain partition.
        """
        if product_keys.ndim != 3:
            raise ValueError("product_keys must have shape [L,Hkv,I]")
        length, hkv, index_dim = product_keys.shape
        if positions.shape != (length,):
            raise ValueError("positions must have shape [L]")
        if length == 0:
            raise ValueError("cannot build an index for an empty prompt")
        _lib.require_device(product_keys)
        if descriptor_weight is not None:
            raise NotImplementedError("cluster descriptors are not part of the flat paper path")
        unit = int(os.environ.get("SEMBLO_FLAT_UNIT_TOKENS", flat_unit_tokens))
        if unit <= 0:
            raise ValueError("the index needs the flat partition: set SEMBLO_FLAT_UNIT_TOKENS "
                             "or semblo_flat_unit_tokens to the mean block size")
        min_log2 = int(os.environ.get("SEMBLO_FLAT_MIN_CLUSTERS_LOG2", flat_min_clusters_log2))
        c = num_clusters or int(os.environ.get("SEMBLO_FLAT_CLUSTERS", "0")) \
            or num_flat_clusters(length, unit, min_log2)
        iters = fit_iters if fit_iters is not None else int(os.environ.get("SEMBLO_FLAT_FIT_ITERS", "8"))
        per_c = int(os.environ.get("SEMBLO_FLAT_FIT_PER_C", "32"))
        align = int(os.environ.get("SEMBLO_FA3_ALIGN", page_align))
        sink = fitted_sink_tokens() if sink_tokens is None else int(sink_tokens)
        if sink:
            check_sink_partition(sink, length, length, c)
        # the k-means runs over rows sink.. with cf centroids (ids 1.. of the partition
        # when a sink holds cluster 0)
        n_fit = length - sink
        cf = c - 1 if sink else c
        fit_n = min(n_fit, max(int(kmeans_sample_size), per_c * c))
        if fit_n < cf:
            raise ValueError("sample must be at least as large as num_clusters")
        if c % 64 or c > 1024:
            raise ValueError(f"{c} clusters: the kernels take a multiple of 64 up to 1024")
        dev = product_keys.device
        gen = torch.Generator()
        gen.manual_seed(int(codebook_seed or 0))
        s = _lib.stream(dev)
        pk = product_keys if product_keys.stride(-1) == 1 else product_keys.contiguous()
        if pk.dtype != torch.bfloat16:
            raise ValueError("product_keys must be bfloat16")

        space_f32 = torch.empty(length, index_dim, dtype=torch.float32, device=dev)
        space_bf = torch.empty(length, index_dim, dtype=torch.bfloat16, device=dev)
        cent_f32 = torch.empty(cf, index_dim, dtype=torch.float32, device=dev)
        cent_bf = torch.empty(cf, index_dim, dtype=torch.bfloat16, device=dev)
        n_it = max(iters, 1)
        sums_hist = torch.empty(n_it, cf, index_dim, dtype=torch.float32, device=dev)
        counts_hist = torch.empty(n_it, cf, dtype=torch.int32, device=dev)
        no_restart = torch.full((cf,), -1, dtype=torch.int32, device=dev)
        restart_flags = torch.zeros(n_it + 1, dtype=torch.int32, device=dev)   # [0] stays 0
        assign_s = torch.empty(fit_n, dtype=torch.int32, device=dev)
        assign_all = torch.empty(length, dtype=torch.int32, device=dev)
        cap = length + c * (max(align, 1) - 1)
        posting_full = torch.empty(hkv, cap, dtype=torch.int32, device=dev)
        inverse = torch.empty(hkv, length, dtype=torch.int32, device=dev)
        sizes = torch.empty(hkv, c, dtype=torch.int32, device=dev)
        indptr = torch.empty(hkv, c + 1, dtype=torch.int32, device=dev)
        totals = torch.empty(hkv, dtype=torch.int32, device=dev)
        codebooks = torch.empty(hkv, 2, c, index_dim // 2, dtype=product_keys.dtype, device=dev)
        desc_fit = torch.empty(2, cf, index_dim // 2, dtype=product_keys.dtype, device=dev) if sink else None
        # the rows the k-means sees: positions sink..
        fit_f32, fit_bf = space_f32[sink:], space_bf[sink:]
        bits_bytes = _lib.query("sbsa_kmeans_member_bits_bytes", fit_n, cf)
        member_bits = torch.empty(bits_bytes // 4, dtype=torch.int32, device=dev)
        ws_bytes = _lib.query("sbsa_bucket_layout_workspace_bytes", length, c)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

        _draw_ahead_settle()
        host = _draw_buffers(n_fit, fit_n, cf)
        counts_host = host.counts_host(n_it, cf)

        k_ahead = RESTARTS_AHEAD

        def draws(g, hd):
            """fit_flat_codebook's first two draws (flat_index.py:237-262), then the
            draws of the first k_ahead restarts (flat_index.py:277-283) made ahead: the
            GPU applies the k-th at the k-th iteration that leaves a cluster empty.
            Returns the generator's state before each restart draw, to take back the
            draws no iteration needs."""
            torch.randperm(n_fit, generator=g, out=hd.perm)
            torch.randperm(fit_n, generator=g, out=hd.init)
            before = []
            for k in range(k_ahead):
                before.append(g.get_state())
                torch.randperm(fit_n, generator=g, out=hd.restarts[k])
            return before

        def upload(hd, before):
            """The draws to the device from pinned memory."""
            if host.uploaded is not None:
                host.uploaded.synchronize()     # the previous upload has left `pinned`
            total = fit_n + (1 + k_ahead) * cf
            host.pinned[:fit_n].copy_(hd.perm[:fit_n])
            host.pinned[fit_n:fit_n + cf].copy_(hd.init[:cf])
            host.pinned[fit_n + cf:total].view(k_ahead, cf).copy_(hd.restarts[:, :cf])
            both = torch.empty(total, dtype=torch.int32, device=dev)
            both.copy_(host.pinned[:total], non_blocking=True)
            host.uploaded = torch.cuda.Event()
            host.uploaded.record()
            return both[:fit_n], both[fit_n:fit_n + cf], both[fit_n + cf:], before

        cur = 0                                 # the draw set of the head being fitted

        def draw():
            return upload(host.sets[cur], draws(gen, host.sets[cur]))

        steps: dict = {}

        def iterate(start, sample_idx, restart_rows=None):
            # k-means steps start.. in one call.  With restart_rows the first k_ahead
            # iterations that leave clusters empty restart them on the GPU; an iteration
            # that left a cluster empty without a restart is found afterwards from
            # counts_hist and redone
            def call(i0, i1):
                _lib.call("sbsa_kmeans_iterate", _lib.ptr(fit_bf), _lib.ptr(fit_f32), index_dim,
                          _lib.ptr(sample_idx), fit_n, cf, index_dim, _lib.ptr(assign_s),
                          _lib.ptr(sums_hist), _lib.ptr(counts_hist), _lib.ptr(no_restart),
                          _lib.ptr(restart_rows), k_ahead, _lib.ptr(restart_flags), _lib.ptr(cent_f32),
                          _lib.ptr(cent_bf), _lib.ptr(member_bits), bits_bytes, i0, i1, s)
            if fit_trace is not None:
                for i in range(start, iters):
                    entry = cent_bf.clone()
                    call(i, i + 1)
                    steps[i] = (entry, assign_s.clone())
                return
            if start < iters:
                call(start, iters)

        def read_counts(it0):
            """Copy the counts of iterations it0.. to the host; the event marks their arrival."""
            counts_host[it0:iters].copy_(counts_hist[it0:iters], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            return ev

        def empty_iterations(it0):
            """The iterations >= it0 that left a cluster empty (the counts are on the host)."""
            hit = torch.nonzero((counts_host[it0:iters] == 0).any(dim=1)).flatten()
            return [it0 + int(i) for i in hit]

        def finalize(h):
            """Assign every key, lay the runs out, write the descriptor."""
            _lib.call("sbsa_kmeans_assign", _lib.ptr(fit_bf), index_dim, None, n_fit,
                      _lib.ptr(cent_bf), cf, index_dim, _lib.ptr(assign_all[sink:]), s)
            fit_assign = None
            if sink:
                fit_assign = assign_all[sink:].clone() if fit_trace is not None else None
                assign_all[sink:] += 1          # clusters 1..C-1
                assign_all[:sink] = 0           # the sink
            _lib.call("sbsa_bucket_layout", _lib.ptr(assign_all), length, c, max(align, 1),
                      _lib.ptr(sizes[h]), _lib.ptr(indptr[h]), _lib.ptr(posting_full[h]), cap,
                      _lib.ptr(inverse[h]), _lib.ptr(totals[h:h + 1]), _lib.ptr(ws), ws_bytes, s)
            if sink:
                # cluster 0's descriptor is zero: no score lands there, no key joins it later
                _lib.call("sbsa_kmeans_centroids", 2, _lib.ptr(cent_f32), None, None, None, 0, None,
                          cf, index_dim, None, _lib.ptr(desc_fit), s)
                codebooks[h, :, 1:].copy_(desc_fit)
                codebooks[h, :, 0].zero_()
            else:
                _lib.call("sbsa_kmeans_centroids", 2, _lib.ptr(cent_f32), None, None, None, 0, None,
                          c, index_dim, None, _lib.ptr(codebooks[h]), s)
            return fit_assign

        sample_idx, init, restart_rows, before_restart = draw()
        for h in range(hkv):
            kh = pk[:, h]
            _lib.call("sbsa_key_space", _lib.ptr(kh), length, kh.stride(0), index_dim,
                      int(bool(router_pass)), _lib.ptr(space_f32), _lib.ptr(space_bf), s)
            _lib.call("sbsa_kmeans_centroids", 0, None, None, _lib.ptr(init), _lib.ptr(fit_f32),
                      index_dim, _lib.ptr(sample_idx), cf, index_dim, _lib.ptr(cent_f32),
                      _lib.ptr(cent_bf), s)
            iterate(0, sample_idx, restart_rows)
            counted = read_counts(0) if iters > 0 else None
            # the final steps are enqueued now, and again if an empty iteration past
            # those restarted on the GPU is redone below
            fit_assign = finalize(h)
            # The next head's draws follow the restart draws this head takes, which its
            # counts decide.  While the host waits for them, a worker draws the next head's
            # permutations into the other draw set for a guessed number of empty iterations
            # of this head (its number in the last build of this shape, else the last
            # head's), from where the generator then stands: before the restart draw of that
            # number, or after all k_ahead.  They are used if the guess holds and dropped
            # otherwise, so the sequence of draws is the reference's either way.
            ahead = None
            guess = host.head_empties.get(h, host.last_empties)
            # past k_ahead empty iterations the host draws more restarts after the counts,
            # which no draw made ahead can follow: then nothing is drawn ahead
            if (DRAW_AHEAD and h + 1 < hkv and fit_trace is None and iters > 0 and k_ahead > 0
                    and guess <= k_ahead):
                g_ahead = torch.Generator()
                g_ahead.set_state(before_restart[guess] if guess < k_ahead else gen.get_state())
                ahead = (guess, g_ahead, _draw_ahead_submit(draws, g_ahead, host.sets[1 - cur]))
            if counted is not None:
                counted.synchronize()
            empties = empty_iterations(0) if iters > 0 else []
            if len(empties) < k_ahead:
                gen.set_state(before_restart[len(empties)])   # take back the unused draws
            if fit_trace is not None:
                # the sample rows each restarted iteration drew, for its empty clusters in
                # ascending order (the GPU applied the first k_ahead of them)
                drawn = {it: host.sets[cur].restarts[k][:int((counts_host[it] == 0).sum())].clone().long()
                         for k, it in enumerate(empties[:k_ahead])}
            host.last_empties = host.head_empties[h] = len(empties)
            # the GPU restarted the first k_ahead empty iterations; the next is restarted here
            it = empties[k_ahead] if len(empties) > k_ahead else -1
            while it >= 0:
                # the reference's restart of the empty clusters at iteration it
                # (flat_index.py:277-283), then the later iterations again
                empty = counts_host[it] == 0
                src = torch.full((cf,), -1, dtype=torch.int32)
                torch.randperm(fit_n, generator=gen, out=host.sub)
                src[empty] = host.sub[:int(empty.sum())].to(torch.int32)
                if fit_trace is not None:
                    drawn[it] = host.sub[:int(empty.sum())].clone().long()
                src_d = src.to(dev)
                _lib.call("sbsa_kmeans_centroids", 1, _lib.ptr(sums_hist[it]), _lib.ptr(counts_hist[it]),
                          _lib.ptr(src_d), _lib.ptr(fit_f32), index_dim, _lib.ptr(sample_idx),
                          cf, index_dim, _lib.ptr(cent_f32), _lib.ptr(cent_bf), s)
                iterate(it + 1, sample_idx)
                if it + 1 < iters:
                    read_counts(it + 1).synchronize()
                    later = empty_iterations(it + 1)
                    it = later[0] if later else -1
                else:
                    it = -1
                if it < 0:
                    fit_assign = finalize(h)
            if fit_trace is not None:
                # copies (a tensor already on the host would otherwise be the reused buffer)
                fit_trace.append(dict(
                    space_f32=fit_f32.to('cpu', copy=True), space_bf16=fit_bf.to('cpu', copy=True), sink=sink,
                    sample=sample_idx.to('cpu', copy=True).long(),
                    entry_centroids=[steps[i][0].to('cpu', copy=True) for i in range(iters)],
                    assign=[steps[i][1].to('cpu', copy=True).long() for i in range(iters)],
                    sums=sums_hist[:iters].to('cpu', copy=True), counts=counts_hist[:iters].to('cpu', copy=True),
                    final_centroids_f32=cent_f32.to('cpu', copy=True), final_centroids=cent_bf.to('cpu', copy=True),
                    final_assign=(fit_assign if sink else assign_all).to('cpu', copy=True).long(),
                    restarts={it: d for it, d in drawn.items() if it < iters},
                    partition=assign_all.to('cpu', copy=True).long()))
                steps.clear()
            if h + 1 < hkv:
                if ahead is not None:
                    guess, g_ahead, fut = ahead
                    before_next = fut.result()
                    if len(empties) == guess:
                        # the guess held (no restart drawn on the host either): the next
                        # head's draws are the worker's, and the generator goes on from where
                        # the worker's copy stopped
                        gen.set_state(g_ahead.get_state())
                        cur = 1 - cur
                        sample_idx, init, restart_rows, before_restart = upload(host.sets[cur],
                                                                                before_next)
                        DRAW_AHEAD_STATS["used"] += 1
                        continue
                    DRAW_AHEAD_STATS["discarded"] += 1
                sample_idx, init, restart_rows, before_restart = draw()
        width = int(totals.max().item())
        posting = posting_full[:, :width].contiguous()
        return cls(codebooks=codebooks, posting_positions=posting, bucket_indptr=indptr,
                   bucket_sizes=sizes, prompt_length=length, max_position=length - 1,
                   flat_clusters=c, page_align=align if align > 1 else 0,
                   _inverse_positions=inverse)

    def pack_prompt_kv(self, key: torch.Tensor, value: torch.Tensor, *, pool=None) -> torch.Tensor:
        """K/V in bucket order, [2, W padded to 256, Hkv, D] (state.py:950-997)."""
        if key.shape != value.shape:
            raise ValueError("key and value must have the same shape")
        if key.ndim != 3 or key.shape[0] != self.prompt_length:
            raise ValueError("key and value must have shape [L,Hkv,D]")
        if key.shape[1] != self.num_kv_heads:
            raise ValueError("key and value KV-head count differs from the index")
        if key.stride() != value.stride() or key.stride(-1) != 1:
            raise ValueError("key and value must share a row-major layout")
        width = int(self.posting_positions.shape[1])
        packed_len = width + (-width) % PACK_ALIGN
        hkv, d = key.shape[1], key.shape[2]
        shape = (2, packed_len, hkv, d)
        packed = pool(shape, key.dtype, key.device) if pool is not None else \
            torch.empty(shape, dtype=key.dtype, device=key.device)
        _lib.call("sbsa_pack_kv", _lib.ptr(key), _lib.ptr(value), key.stride(0), key.stride(1),
                  hkv, d, _lib.ptr(self.posting_positions), width, packed_len, _lib.ptr(packed),
                  _lib.stream(key.device))
        self.packed_kv = packed
        return packed

    def inverse_positions(self) -> torch.Tensor:
        """[Hkv, L] int32: position -> packed row (state.py:999-1012)."""
        return self._inverse_positions

    def causal_sizes(self, pos_limit: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """[Hkv, C] keys of each cluster at positions < pos_limit."""
        hkv, c = self.bucket_sizes.shape
        if out is None:
            out = torch.empty(hkv, c, dtype=torch.int32, device=self.bucket_sizes.device)
        _lib.call("sbsa_causal_sizes", _lib.ptr(self.posting_positions),
                  self.posting_positions.shape[1], _lib.ptr(self.bucket_indptr),
                  _lib.ptr(self.bucket_sizes), hkv, c, int(pos_limit), _lib.ptr(out),
                  _lib.stream(out.device))
        return out
