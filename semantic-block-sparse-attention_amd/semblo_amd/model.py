"""The sparse attention layer behind ``semblo::attention`` (host orchestration).

Mirrors the reference's SembloAttention paths that the operator reaches
(semblo/vllm_plugin/model.py):

  attention_forward        prefill of the whole prompt, or one decode step  (model.py:1169-1269)
  _ingest_prompt_kv        index build, packed K/V                            (model.py:1301-1382)
  _run_product_attention   the query-chunk loop                               (model.py:856-1008)
  _full_graph_decode_step  the decode step over the arena                     (model.py:708-783)
  begin_token_outer_prefill  a token-order prefill session   (token_outer_prefill.py:127-212)
  begin_streamed_prefill     a layer-major streamed prefill session   (model.py:1271-1279)

The projections around the attention (Q/K/V with RoPE and the output gate and
projection) belong to the model, which is not part of this build.  A model that
drives the streamed sessions with hidden states, as the reference's streamer
does, attaches them with ``attach_projections``.

vLLM's metadata, paged cache and profiling branch are not part of this
build: the layer keeps its own per-request state, and a call with more than
one token starts a new request.
"""
from __future__ import annotations

import os

import torch

from . import suffix_flush
from .arena import DecodeArena
from .attention_op import register_layer
from .config import SembloRuntimeConfig
from .fused_decode import fused_decode_step
from .fused_prefill import CausalSnapshot, fused_chunk_execute, fused_chunk_plan
from .kv_outer import PartialsGuard
from .kv_outer import dense_causal_attention
from .state import ProductPostingIndex
from .trivial_router import trivial_router_vectors


class SembloQueryState:
    """Routing vectors [1, Q, Hq, 1, I] and mixture weights [1, Q, Hq, 1] (model.py:432-489)."""

    def __init__(self, vectors: torch.Tensor, mixture_weights: torch.Tensor):
        self.vectors = vectors
        self.mixture_weights = mixture_weights
        self.descriptor_vectors = None
        self.descriptor_gamma = None


class SembloAttention:
    """One full-attention layer's sparse core."""

    def __init__(self, config: SembloRuntimeConfig, layer_name: str | None = None) -> None:
        self.runtime_config = config
        self.num_heads = config.num_q_heads
        self.num_kv_heads = config.num_kv_heads
        self.head_dim = config.head_dim
        self.scaling = config.scale
        self.layer_idx = config.layer_idx
        self.layer_name = layer_name or f"semblo.layer.{config.layer_idx}"
        self.index: ProductPostingIndex | None = None
        self.arena: DecodeArena | None = None
        self.target_tokens = 0
        # test hook: a list here receives every sparse chunk's selection (ChunkPlan.record)
        self.plan_log: list | None = None
        self._projections = None
        self._capacity_arena: DecodeArena | None = None
        register_layer(self.layer_name, self)

    # -- the model's projections (attached by the caller) -------------------------
    def attach_projections(self, project_qkv, finish_output, project_kv=None) -> None:
        """The model's side of the layer, for the sessions driven by hidden states.

        ``project_qkv(rope_positions, hidden_states)`` returns (q_post, k_post, v,
        q_pre, k_pre, gate): Q and K after and before the rotary embedding, V, and
        the output gate or None (the reference's model ``_project_qkv``,
        qwen3_5_model.py:135, nemotron_h_model.py:149).  ``finish_output(attn, gate)``
        takes the attention [n, Hq*D] to the layer's output (``_finish_output``,
        qwen3_5_model.py:225-235).  ``project_kv`` returns (k_post, v, k_pre) alone; by
        default the full projection runs and Q is dropped (model.py:356-368)."""
        self._projections = (project_qkv, finish_output, project_kv)

    def _require_projections(self):
        if self._projections is None:
            raise RuntimeError(f"layer {self.layer_name!r} has no projections: a session driven by "
                               "hidden states needs attach_projections(project_qkv, finish_output)")
        return self._projections

    def _project_qkv(self, rope_positions, hidden_states):
        return self._require_projections()[0](rope_positions, hidden_states)

    def _project_kv(self, rope_positions, hidden_states):
        project_qkv, _, project_kv = self._require_projections()
        if project_kv is not None:
            return project_kv(rope_positions, hidden_states)
        _q, k_post, v, _qp, k_pre, _g = project_qkv(rope_positions, hidden_states)
        return k_post, v, k_pre

    def _finish_output(self, attn: torch.Tensor, gate):
        return self._require_projections()[1](attn, gate)

    @staticmethod
    def _positions_for_runtime(positions: torch.Tensor):
        """(rotary positions, flat positions): an M-RoPE grid [3, T] keeps its first row
        as the flat one (qwen3_5_model.py:124-133)."""
        if positions.ndim == 2:
            return positions, positions[0]
        return positions, positions

    @staticmethod
    def _slice_positions(rope_positions: torch.Tensor, start: int, stop: int) -> torch.Tensor:
        """Rows [start, stop) of the rotary positions, [T] or [3, T] (model.py:1290-1299)."""
        if rope_positions.ndim == 2:
            return rope_positions[:, start:stop]
        return rope_positions[start:stop]

    def _prompt_positions(self, tokens_or_positions):
        """(tokens, rotary positions or None) of a new prompt given as a length or as its
        positions, which must be 0 .. T-1: the index holds one prompt from position 0."""
        if not isinstance(tokens_or_positions, torch.Tensor):
            return int(tokens_or_positions), None
        rope, flat = self._positions_for_runtime(tokens_or_positions)
        tokens = int(flat.numel())
        if not torch.equal(flat.reshape(-1).to("cpu", torch.int64), torch.arange(tokens)):
            raise ValueError("a prompt's positions must run 0 .. T-1 (one prompt, from its start)")
        return tokens, rope

    # -- routing (S0) ---------------------------------------------------------
    def _query_state(self, q_pre: torch.Tensor) -> SembloQueryState:
        vec = trivial_router_vectors(q_pre, 1)
        q, h, d = vec.shape
        ones = torch.ones(1, q, h, 1, dtype=torch.float32, device=vec.device)
        return SembloQueryState(vec.view(1, q, h, 1, d), ones)

    # -- prefill ----------------------------------------------------------------
    def _ingest_prompt_kv(self, k_pre: torch.Tensor, k_post: torch.Tensor,
                          v: torch.Tensor) -> ProductPostingIndex:
        cfg = self.runtime_config
        length = k_pre.shape[0]
        if length < 128:
            raise ValueError("sparse prefill requires at least 128 prompt tokens")
        positions = torch.arange(length, device=k_pre.device)
        index = ProductPostingIndex.build(
            k_pre, positions, kmeans_sample_size=cfg.kmeans_sample_size,
            codebook_seed=cfg.codebook_seed + cfg.layer_idx, flat_unit_tokens=cfg.flat_unit_tokens,
            flat_min_clusters_log2=cfg.flat_min_clusters_log2, page_align=cfg.page_align,
            router_pass=True)
        index.pack_prompt_kv(k_post, v)
        index.original_kv = (k_post, v)
        return index

    def _build_stream(self, device) -> torch.cuda.Stream:
        """The stream the index is built on while the dense chunks run (default priority)."""
        st = getattr(self, "_side_stream", None)
        if st is None or st.device != torch.device(device):
            st = torch.cuda.Stream(device=device)
            self._side_stream = st
        return st

    def begin_token_outer_prefill(self, tokens, chunk: int, **kw):
        """A token-order prefill session of a prompt (its length, or its positions as
        the reference passes them) in slices of ``chunk`` (the reference's
        layer.begin_token_outer_prefill, model.py:1281, streamed_prefill.py:563-564)."""
        from .token_outer_prefill import TokenOuterPrefillSession
        tokens, rope = self._prompt_positions(tokens)
        self.index = None
        self.arena = None
        return TokenOuterPrefillSession(self, tokens, chunk, rope_positions=rope, **kw)

    def begin_streamed_prefill(self, tokens):
        """This layer's share of a layer-major streamed prefill of a prompt (its length,
        or its positions as the reference passes them): ``keys`` for every slice, then
        ``ingest``, then ``queries`` for every slice (the reference's
        layer.begin_streamed_prefill, model.py:1271-1279)."""
        from .streamed_prefill import StreamedPrefillSession
        tokens, _rope = self._prompt_positions(tokens)
        return StreamedPrefillSession(self, tokens)

    def prefill_streamed(self, q_post, q_pre, k_pre, k_post, v, output, slice_tokens: int,
                         timing=None) -> torch.Tensor:
        """The whole prompt through this layer in slices of ``slice_tokens``, keys pass then
        queries pass (streamed_prefill.py:496-545, 710-736 for one layer)."""
        length = q_post.shape[0]
        hq, hkv, d = self.num_heads, self.num_kv_heads, self.head_dim
        spans = [(s, min(length, s + slice_tokens)) for s in range(0, length, slice_tokens)]
        session = self.begin_streamed_prefill(length)
        for st, en in spans:
            session.stage_keys(k_pre.view(length, hkv, d)[st:en], k_post.view(length, hkv, d)[st:en],
                               v.view(length, hkv, d)[st:en], st, en)
        session.ingest()
        out = output.view(length, hq, d)
        for st, en in spans:
            session.attend(q_post.view(length, hq, d)[st:en], q_pre.view(length, hq, d)[st:en], st,
                           out=out[st:en], timing=timing)
        session.finish()
        return output

    def capacity_arena(self, device) -> DecodeArena:
        """The layer's fixed-address decode arena for prompts of up to
        ``decode_capacity`` positions, made on first use (before any request, for a
        caller that captures the decode step at warm-up); its cluster count is the rule's
        at the capacity (arena.py:43-48)."""
        cfg = self.runtime_config
        if cfg.decode_capacity <= 0:
            raise RuntimeError("the layer has no decode capacity (decode_capacity = 0)")
        if self._capacity_arena is None:
            from .config import num_flat_clusters
            self._capacity_arena = DecodeArena.with_capacity(
                capacity=cfg.decode_capacity, num_kv_heads=self.num_kv_heads, head_dim=self.head_dim,
                num_clusters=num_flat_clusters(cfg.decode_capacity, cfg.flat_unit_tokens,
                                               cfg.flat_min_clusters_log2),
                page_align=cfg.page_align, reserve=cfg.suffix_reserve, suffix_block=cfg.suffix_block,
                suffix_splits=cfg.decode_suffix_splits, device=device)
        return self._capacity_arena

    def decode_budget(self) -> int:
        """The selection budget of a decode step, chosen per step (model.py:847-854):
        ``decode_target_tokens`` when set, else with a capacity arena the budget at the
        capacity (the one a step captured before the request was made with), else the
        last prefill's budget.  A later prefill sets its own again."""
        cfg = self.runtime_config
        if cfg.decode_target_tokens > 0:
            return int(cfg.decode_target_tokens)
        if cfg.decode_capacity > 0:
            return cfg.budget(cfg.decode_capacity)
        return int(self.target_tokens)

    def adopt_index(self, index: ProductPostingIndex) -> None:
        """Make a finished prompt index the layer's decode state."""
        cfg = self.runtime_config
        index.original_kv = None
        self.index = index
        if cfg.decode_capacity > 0:
            if suffix_flush.flush_every() > 0:
                raise RuntimeError("the suffix flush does not run on a fixed-capacity decode arena "
                                   "(decode_capacity > 0)")
            arena = self.capacity_arena(index.packed_kv.device)
            arena.adopt(index)
            self.arena = arena
            return
        shuffle = None if cfg.suffix_shuffle_seed is None else \
            torch.Generator().manual_seed(int(cfg.suffix_shuffle_seed))
        every = suffix_flush.flush_every()
        if every > 0 and suffix_flush.keep_exact() + every > cfg.suffix_reserve - 2 * cfg.suffix_block:
            raise RuntimeError(
                f"SEMBLO_SUFFIX_KEEP_EXACT + SEMBLO_SUFFIX_FLUSH_EVERY = "
                f"{suffix_flush.keep_exact() + every} exact tokens do not fit the suffix store of "
                f"{cfg.suffix_reserve} positions (suffix_reserve) less two blocks")
        self.arena = DecodeArena(index, reserve=cfg.suffix_reserve, suffix_block=cfg.suffix_block,
                                 suffix_splits=cfg.decode_suffix_splits, shuffle_blocks=shuffle,
                                 flush_room=suffix_flush.flush_room() if every > 0 else 0)

    def prefill_token_order(self, q_post, q_pre, k_pre, k_post, v, output, chunk: int,
                            timing=None, store_timing=None, **kw) -> torch.Tensor:
        """The whole prompt in token order, one ``chunk``-position slice after another
        (streamed_prefill.py:547-593 for one layer)."""
        length = q_post.shape[0]
        hq, hkv, d = self.num_heads, self.num_kv_heads, self.head_dim
        session = self.begin_token_outer_prefill(length, chunk, **kw)
        out = output.view(length, hq, d)
        for start in range(0, length, chunk):
            stop = min(length, start + chunk)
            session.slice_projected(q_post.view(length, hq, d)[start:stop],
                                    q_pre.view(length, hq, d)[start:stop],
                                    k_pre.view(length, hkv, d)[start:stop],
                                    k_post.view(length, hkv, d)[start:stop],
                                    v.view(length, hkv, d)[start:stop], start, stop, out=out[start:stop],
                                    timing=timing, store_timing=store_timing)
        self.last_session = session
        session.finish()
        return output

    def prefill(self, q_post, q_pre, k_pre, k_post, v, output, timing=None) -> torch.Tensor:
        cfg = self.runtime_config
        length = q_post.shape[0]
        if os.environ.get("SEMBLO_PREFILL_ORDER", "layer") == "token":
            chunk = int(os.environ.get("SEMBLO_PREFILL_CHUNK", "0") or 0) or cfg.query_chunk_size
            return self.prefill_token_order(q_post, q_pre, k_pre, k_post, v, output, chunk, timing=timing)
        stream = int(os.environ.get("SEMBLO_PREFILL_CHUNK", "0") or 0)
        if 0 < stream <= length:
            # a long prefill streamed in slices, layer-major (PrefillStreamer.wants/run)
            return self.prefill_streamed(q_post, q_pre, k_pre, k_post, v, output, stream, timing=timing)
        q = q_post.view(length, self.num_heads, self.head_dim)
        qp = q_pre.view(length, self.num_heads, self.head_dim)
        kp = k_pre.view(length, self.num_kv_heads, self.head_dim)
        kk = k_post.view(length, self.num_kv_heads, self.head_dim)
        vv = v.view(length, self.num_kv_heads, self.head_dim)
        out = output.view(length, self.num_heads, self.head_dim)
        self.target_tokens = cfg.budget(length)
        step = cfg.query_chunk_size
        cap = cfg.dense_prefix_x * self.target_tokens
        # The dense-prefix chunks read only the prompt-order K/V, not the index:
        # they are enqueued first on this stream, and the index is built on a
        # second stream (default priority) that waits only for the inputs, so
        # the build's host work (its random draws and host reads) overlaps the
        # dense attention.  The sparse chunks wait for the build.  The outputs
        # do not depend on the order.
        main = torch.cuda.current_stream(q.device)
        inputs_ready = torch.cuda.Event()
        inputs_ready.record(main)
        for start in range(0, min(length, cap + 1), step):
            end = min(length, start + step)
            if timing is not None:
                n = end - start
                timing.add_flops(4.0 * self.head_dim * self.num_heads * (n * (start + 1) + n * (n - 1) // 2))
            dense_causal_attention(q[start:end], kk, vv, sm_scale=self.scaling, chunk_start=start,
                                   out=out[start:end], timing=timing)
        side = self._build_stream(q.device)
        side.wait_event(inputs_ready)
        sparse = [(st, min(length, st + step)) for st in range(0, length, step) if st > cap]
        # every sparse chunk's selection and reverse index on the build stream,
        # each followed by an event; a chunk's attention waits for its own plan
        # on the GPU only.  Its partial rows are sized by the capacity bound
        # (kv_outer.partials_capacity), so the host reads nothing and every
        # chunk is enqueued at once.
        plans, ready = [], []
        with torch.cuda.stream(side):
            index = self._ingest_prompt_kv(kp, kk, vv)
            snapshot = CausalSnapshot(index)

        def enqueue_plan(i):
            st, en = sparse[i]
            with torch.cuda.stream(side):
                pl = fused_chunk_plan(q[st:en], self._query_state(qp[st:en]), index, snapshot, st,
                                      en - 1, temperature=cfg.selection_temperature,
                                      beta=cfg.bucket_size_penalty, target_tokens=self.target_tokens,
                                      iters=cfg.iters, dense_prefix_x=cfg.dense_prefix_x,
                                      keep_theta=self.plan_log is not None)
                pl.record(self.plan_log)
                # the chunk's work list too, here rather than on the main stream
                # between two chunks' attention
                pl.kv.prepare_work(q[st:en], index.num_kv_heads, index.bucket_indptr, guard)
                ev = torch.cuda.Event()
                ev.record(side)
            plans.append(pl)
            ready.append(ev)

        self.index = index
        # chunks whose partial rows were capped (kv_outer.partials_cap_bytes) are checked
        # once, after the last chunk is enqueued, and any that overflowed is run again;
        # each flag comes from the chunk's plan (copied when its work list is built), so
        # the check waits for the plans, not for the chunks' attention
        guard = PartialsGuard()
        for i in range(len(sparse)):
            enqueue_plan(i)
        for i, (st, en) in enumerate(sparse):
            pl = plans[i]
            main.wait_event(ready[i])
            if i == 0:
                for t in (index.codebooks, index.posting_positions, index.bucket_indptr,
                          index.bucket_sizes, index._inverse_positions, index.packed_kv):
                    t.record_stream(main)
            for t in pl.tensors():
                t.record_stream(main)
            fused_chunk_execute(pl, q[st:en], index, None,
                                sm_scale=self.scaling, out=out[st:en], timing=timing, guard=guard)
        guard.finish()
        self.partials_reruns = guard.reruns
        built = torch.cuda.Event()
        built.record(side)
        # the decode state uses the index on this stream
        main.wait_event(built)
        if not sparse:
            for t in (index.codebooks, index.posting_positions, index.bucket_indptr,
                      index.bucket_sizes, index._inverse_positions, index.packed_kv):
                t.record_stream(main)
        self.adopt_index(index)
        return output

    # -- decode -----------------------------------------------------------------
    def decode(self, positions, q_post, q_pre, k_post, v, output, k_pre=None) -> torch.Tensor:
        """One decode step.  ``k_pre`` (the token's pre-RoPE key) is kept for the suffix
        flush, which routes the moved tokens; without the flush it is not read."""
        if self.arena is None:
            raise RuntimeError("decode before any prefill: the layer has no index")
        cfg = self.runtime_config
        arena = self.arena
        if arena.flush_room:
            # the suffix flush (SEMBLO_SUFFIX_FLUSH_EVERY), on the host before the step, as
            # the reference's hook around execute_model (suffix_flush.py:264-302)
            suffix_flush.maybe_flush(arena)
        # The suffix store holds `reserve` generated positions past the prompt length (the
        # reference sizes it to the model's room for generated tokens, arena.py:50-63); a
        # step past it would neither store nor read its token, so it is refused here,
        # counted on the host.
        if arena.first_prompt_length + arena.steps - arena.prompt_length >= arena.reserve:
            raise RuntimeError(f"the decode suffix holds {arena.reserve} generated positions "
                               f"(suffix_reserve); raise it to the generation length")
        arena.steps += 1
        fused_decode_step(self, self.arena, q_post=q_post, q_pre=q_pre, positions=positions,
                          k_post=k_post, v_states=v, k_pre=k_pre, output=output,
                          temperature=cfg.selection_temperature, beta=cfg.bucket_size_penalty,
                          target_tokens=self.decode_budget(), sm_scale=self.scaling,
                          num_splits=cfg.decode_num_splits, iters=cfg.iters,
                          suffix_splits=cfg.decode_suffix_splits)
        return output

    def attention_forward(self, positions, hidden_states, q_post, k_post, v_states, q_pre, k_pre,
                          output) -> None:
        """The operator's body (model.py:1169-1269): a prompt of T > 1 tokens starting at
        position 0 is a prefill; a single token after the prompt is a decode step."""
        t = q_post.shape[0]
        if t > 1 or self.arena is None:
            if k_post is None or v_states is None or k_pre is None:
                raise RuntimeError("a prefill needs the layer's K/V and pre-RoPE keys")
            self.prefill(q_post, q_pre, k_pre, k_post, v_states, output)
        else:
            pos = positions.reshape(-1)[:1]
            if pos.dtype != torch.int32:
                pos = pos.to(torch.int32)
            self.decode(pos, q_post, q_pre, k_post, v_states, output, k_pre=k_pre)
