"""Layer-major streamed prefill: one sparse layer's share of a prompt walked twice.

Host side of the reference's ``StreamedPrefillSession`` (semblo/vllm_plugin/
model.py:1431-1531), which its ``PrefillStreamer`` drives slice by slice
(streamed_prefill.py:496-545, 710-736):

  keys     every slice's K/V (and pre-RoPE keys) are staged in prompt order;
  ingest   the barrier: the index is fitted on the whole prompt's keys and the
           K/V packed in cluster order (the same build as the whole-prompt
           path, so the same clusters); the prompt-order staging is dropped;
  queries  every slice's queries run as query chunks of the layer's chunk size,
           counted from the slice's first position (model.py:856-1000 with
           ``query_offset``): dense-prefix chunks exactly over every earlier key,
           sparse chunks through selection and the KV-outer body.  The keys a
           chunk reads in prompt order (the dense prefix, a sparse chunk's own
           window) come back from the packed store through the inverse map.
  finish   the index becomes the layer's decode state.

With slices that are a multiple of the chunk size the chunks are those of the
whole-prompt path, and so are the outputs, bit for bit.

``keys(rope_positions, hidden_states, start, stop)`` and ``queries(rope_positions,
positions, hidden_states, start)`` are the reference's calls: they run the
projections the model attached to the layer (``SembloAttention.attach_projections``)
and ``queries`` returns the layer's output rows.  ``stage_keys`` and ``attend`` take
the projections themselves, for a caller that has them already.
"""
from __future__ import annotations

import torch

from . import _lib
from .fused_prefill import CausalSnapshot, chunk_window_start, fused_chunk_attention
from .kv_outer import PartialsGuard, dense_causal_attention
from .token_outer_prefill import gather_rows


class StreamedPrefillSession:
    """One sparse layer's share of a layer-major streamed prefill of ``tokens``
    positions (model.py:1431-1531)."""

    def __init__(self, layer, tokens: int) -> None:
        self.layer = layer
        self.tokens = int(tokens)
        if self.tokens < 1:
            raise ValueError("a streamed prefill needs at least one position")
        self.k_pre = self.k_post = self.v = None
        self.staged = 0
        self.index = None
        self.snapshot: CausalSnapshot | None = None
        self.target = layer.runtime_config.budget(self.tokens)
        layer.target_tokens = self.target
        layer.index = None
        layer.arena = None

    # -- pass 1 -----------------------------------------------------------------
    def keys(self, rope_positions: torch.Tensor, hidden_states: torch.Tensor, start: int,
             stop: int) -> None:
        """Project positions [start, stop) with the layer's projections and stage their
        K/V and pre-RoPE keys (model.py:1463-1491)."""
        k_post, v, k_pre = self.layer._project_kv(rope_positions, hidden_states)
        if k_post is None or v is None or k_pre is None:
            raise RuntimeError("the streamed prefill needs a layer with its own K/V")
        self.stage_keys(k_pre, k_post, v, start, stop)

    def stage_keys(self, k_pre: torch.Tensor, k_post: torch.Tensor, v: torch.Tensor, start: int,
                   stop: int) -> None:
        """Stage positions [start, stop): k_pre, k_post, v [n, Hkv, D] (model.py:1481-1491)."""
        if self.index is not None:
            raise RuntimeError("keys after ingest: the index is already fitted")
        layer = self.layer
        hkv, d = layer.num_kv_heads, layer.head_dim
        n = int(stop) - int(start)
        if not 0 <= start < stop <= self.tokens:
            raise ValueError(f"slice [{start}, {stop}) outside the prompt of {self.tokens}")
        kp, kk, vv = (t.reshape(n, hkv, d) for t in (k_pre, k_post, v))
        _lib.require_device(kp, kk, vv)
        if self.k_post is None:
            shape = (self.tokens, hkv, d)
            self.k_pre = kp.new_empty(shape)
            self.k_post = kk.new_empty(shape)
            self.v = vv.new_empty(shape)
        self.k_pre[start:stop] = kp
        self.k_post[start:stop] = kk
        self.v[start:stop] = vv
        self.staged += n

    def ingest(self) -> None:
        """Fit the index on every staged key and pack the K/V; the staging is dropped
        (model.py:1493-1507)."""
        if self.k_post is None:
            raise RuntimeError("no slice was staged before the index was asked for")
        if self.staged != self.tokens:
            raise RuntimeError(f"{self.staged} of {self.tokens} positions staged before ingest")
        index = self.layer._ingest_prompt_kv(self.k_pre, self.k_post, self.v)
        index.original_kv = None            # no prompt-order views on this path
        self.index = index
        self.layer.index = index
        self.k_pre = self.k_post = self.v = None

    # -- pass 2 -----------------------------------------------------------------
    def queries(self, rope_positions: torch.Tensor, positions: torch.Tensor,
                hidden_states: torch.Tensor, start: int) -> torch.Tensor:
        """The layer's output rows for the slice at ``start``: its queries projected with
        the layer's projections, attended, then gated and projected out
        (model.py:1509-1524).  ``positions`` are the slice's flat positions (start ..
        start+n-1; only their count is checked, so that nothing waits for the GPU)."""
        layer = self.layer
        n = int(hidden_states.shape[0])
        if positions.numel() != n:
            raise ValueError(f"{positions.numel()} positions for {n} hidden rows")
        q_post, _k, _v, q_pre, _kp, gate = layer._project_qkv(rope_positions, hidden_states)
        attn = self.attend(q_post, q_pre, start)
        return layer._finish_output(attn.view(n, -1), gate)

    def attend(self, q_post: torch.Tensor, q_pre: torch.Tensor, start: int,
               out: torch.Tensor | None = None, timing=None) -> torch.Tensor:
        """The attention of positions start..start+n-1 (q_post, q_pre [n, Hq, D]) into
        ``out`` [n, Hq, D] (model.py:1509-1524, 856-1000)."""
        if self.index is None:
            raise RuntimeError("queries before ingest")
        layer = self.layer
        cfg = layer.runtime_config
        hq, d = layer.num_heads, layer.head_dim
        n = q_post.shape[0]
        start = int(start)
        if not (0 <= start and start + n <= self.tokens):
            raise ValueError(f"queries [{start}, {start + n}) outside the prompt of {self.tokens}")
        q = q_post.reshape(n, hq, d)
        qp = q_pre.reshape(n, hq, d)
        _lib.require_device(q, qp)
        if out is None:
            out = torch.empty_like(q)
        o = out.view(n, hq, d)
        # a fresh snapshot per call, as the reference's loop makes one
        snapshot = CausalSnapshot(self.index)
        # chunks whose partial rows were capped are settled once, before returning
        guard = PartialsGuard()
        step = cfg.query_chunk_size
        for a in range(0, n, step):
            b = min(n, a + step)
            cs, ce = start + a, start + b - 1
            wstart = chunk_window_start(cs, self.target, cfg.dense_prefix_x)
            if wstart == 0:
                # dense prefix: exact causal attention over positions 0..ce in prompt order
                k_all, v_all = gather_rows(self.index, 0, ce + 1)
                if timing is not None:
                    m = b - a
                    timing.add_flops(4.0 * d * hq * (m * (cs + 1) + m * (m - 1) // 2))
                dense_causal_attention(q[a:b], k_all, v_all, sm_scale=layer.scaling, chunk_start=cs,
                                       out=o[a:b], timing=timing)
                continue
            window = gather_rows(self.index, wstart, ce + 1 - wstart)
            fused_chunk_attention(q[a:b], layer._query_state(qp[a:b]), self.index, None, snapshot,
                                  cs, ce, temperature=cfg.selection_temperature,
                                  beta=cfg.bucket_size_penalty, target_tokens=self.target,
                                  sm_scale=layer.scaling, iters=cfg.iters,
                                  dense_prefix_x=cfg.dense_prefix_x, out=o[a:b], timing=timing,
                                  window_kv=window, plan_log=layer.plan_log, guard=guard)
        guard.finish()
        return out

    def finish(self):
        """The index becomes the layer's decode state (model.py:1526-1531)."""
        if self.index is None:
            raise RuntimeError("finish before ingest")
        self.layer.adopt_index(self.index)
        return self.index
