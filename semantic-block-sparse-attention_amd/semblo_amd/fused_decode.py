"""The sparse decode step (S7-S9) on HIP: one libsbsa call, three launches.

Same contract as the reference's ``fused_decode_step``
(semblo/vllm_plugin/fused_decode.py:393-521): the token's K/V go into the
arena's suffix store, the query is routed, the clusters are selected against
the full cluster sizes (bisection under the budget), the selected packed rows
and the visible suffix are attended in split-K partials, and the partials are
merged into ``output``.  Nothing is allocated and nothing is read back after
the workspace exists, so the step can be captured in a HIP graph.
"""
from __future__ import annotations

import torch

from . import _lib
from .config import fitted_sink_tokens
from .fused_prefill import PagedSparseAttentionResult


class FusedDecodeWorkspace:
    """The step's fixed buffers (fused_decode.py:365-385)."""

    def __init__(self, *, num_q_heads: int, num_kv_heads: int, head_dim: int, num_clusters: int,
                 num_splits: int, suffix_splits: int, device: torch.device) -> None:
        self.shape_key = (num_q_heads, num_kv_heads, head_dim, num_clusters, num_splits,
                          suffix_splits)
        nbytes = _lib.query("sbsa_decode_workspace_bytes", num_q_heads, num_kv_heads,
                            num_clusters, head_dim, num_splits, suffix_splits)
        self.buffer = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        self.nbytes = nbytes
        self.num_splits = num_splits
        self.suffix_splits = suffix_splits
        self.lse = torch.empty(num_q_heads, dtype=torch.float32, device=device)


def _workspace(holder, *, hq, hkv, d, c, splits, suffix_splits, device) -> FusedDecodeWorkspace:
    ws = getattr(holder, "fused_decode_ws", None)
    key = (hq, hkv, d, c, splits, suffix_splits)
    if ws is None or ws.shape_key != key:
        ws = FusedDecodeWorkspace(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, num_clusters=c,
                                  num_splits=splits, suffix_splits=suffix_splits, device=device)
        holder.fused_decode_ws = ws
    return ws


def fused_decode_step(layer, arena, *, q_post: torch.Tensor, q_pre: torch.Tensor,
                      positions: torch.Tensor, k_post: torch.Tensor | None,
                      v_states: torch.Tensor | None, k_pre: torch.Tensor | None = None,
                      output: torch.Tensor, temperature: float, beta: float, target_tokens: int,
                      sm_scale: float, num_splits: int, iters: int = 16,
                      suffix_splits: int | None = None, out_lse: torch.Tensor | None = None,
                      csr_out: torch.Tensor | None = None, no_alloc: bool = False) -> None:
    """The whole decode step of one layer into ``output`` [1, Hq*D] (fused_decode.py:393-521).

    ``positions`` [1] is the token's position as a device tensor; the arena
    (arena.DecodeArena) holds the index, the packed K/V and the suffix store.
    ``no_alloc``: run sbsa_decode_step_noalloc, whose scratch is the library's
    static per-GPU array (no workspace tensor is made); steps on one GPU must not
    overlap.
    """
    hq, hkv, d = int(layer.num_heads), int(layer.num_kv_heads), int(layer.head_dim)
    c = int(arena.num_clusters)
    ss = int(suffix_splits or arena.suffix_splits)
    ws = None if no_alloc else _workspace(arena, hq=hq, hkv=hkv, d=d, c=c, splits=int(num_splits),
                                          suffix_splits=ss, device=q_post.device)
    q = q_post.reshape(hq, d)
    qp = q_pre.reshape(hq, d)
    if q.stride(-1) != 1 or qp.stride(-1) != 1:
        raise ValueError("q_post and q_pre need unit inner strides")
    pos = positions[:1]
    if pos.dtype != torch.int32:
        raise ValueError("positions must be int32 (converting would allocate inside a capture)")
    kk = vv = kp = None
    if k_post is not None and v_states is not None:
        kk = k_post.reshape(hkv, d)
        vv = v_states.reshape(hkv, d)
        if k_pre is not None and getattr(arena, "suffix_kpre", None) is not None:
            kp = k_pre.reshape(hkv, d)
            if kp.stride(0) != kk.stride(0) or kp.stride(-1) != 1:
                raise ValueError("k_pre must share k_post's row layout (the step stores both)")
    out = output.reshape(hq, d)
    head = (_lib.ptr(q), q.stride(0), _lib.ptr(qp), qp.stride(0), 1,
            _lib.ptr(kk), _lib.ptr(vv), kk.stride(0) if kk is not None else 0, _lib.ptr(pos),
            _lib.ptr(arena.codebooks), _lib.ptr(arena.sizes), _lib.ptr(arena.indptr),
            _lib.ptr(arena.packed_kv), arena.packed_kv.shape[1], _lib.ptr(arena.suffix_kv),
            arena.suffix_kv.shape[1], arena.suffix_block, _lib.ptr(arena.suffix_table),
            arena.prompt_length, arena.max_tiles,
            _lib.ptr(arena.prompt_length_t) if arena.reads_prompt_length_on_device else None,
            _lib.ptr(kp), _lib.ptr(arena.suffix_kpre) if kp is not None else None, hq, hkv, c, d,
            1.0 / float(temperature),
            float(beta), float(target_tokens), int(iters), fitted_sink_tokens(), float(sm_scale),
            int(num_splits), ss)
    tail = (_lib.ptr(out), out.stride(0), _lib.ptr(out_lse), _lib.ptr(csr_out), _lib.stream(q.device))
    if no_alloc:
        _lib.call("sbsa_decode_step_noalloc", *head, *tail)
    else:
        _lib.call("sbsa_decode_step", *head, _lib.ptr(ws.buffer), ws.nbytes, *tail)


class _PromptOnly:
    """A suffix store that no position reaches (for the prompt-only seam)."""

    def __init__(self, index, device):
        self.num_clusters = index.num_buckets
        hkv = index.num_kv_heads
        d = index.packed_kv.shape[-1]
        self.codebooks = index.codebooks
        self.sizes = index.bucket_sizes
        self.indptr = index.bucket_indptr
        self.packed_kv = index.packed_kv
        self.suffix_kv = torch.zeros(2, 1, 256, hkv, d, dtype=index.packed_kv.dtype, device=device)
        self.suffix_block = 256
        self.suffix_table = torch.zeros(1, dtype=torch.int32, device=device)
        self.prompt_length = 1 << 40
        self.max_tiles = 0
        self.suffix_splits = 1


def decode_prompt_only(q_chunk: torch.Tensor, vectors: torch.Tensor, index, *, temperature: float,
                       beta: float, target_tokens: int, sm_scale: float, iters: int = 16,
                       num_splits: int = 64,
                       csr_out: torch.Tensor | None = None) -> PagedSparseAttentionResult:
    """fused_decode_attention's contract: [1, Hq, D] out and [1, Hq] LSE over the prompt.
    ``csr_out`` (int32, 3 Hkv C + 2 Hkv) receives the step's selected runs, as in
    fused_decode_step."""
    hq, d = q_chunk.shape[1], q_chunk.shape[2]
    hkv = index.num_kv_heads
    dev = q_chunk.device
    holder = index.extras.setdefault("prompt_only", _PromptOnly(index, dev))
    ws = _workspace(holder, hq=hq, hkv=hkv, d=d, c=index.num_buckets, splits=num_splits,
                    suffix_splits=1, device=dev)
    q = q_chunk.reshape(hq, d).contiguous()
    v = vectors.reshape(hq, d).contiguous()
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty(1, hq, d, dtype=q_chunk.dtype, device=dev)
    lse = torch.empty(1, hq, dtype=torch.float32, device=dev)
    _lib.call("sbsa_decode_step", _lib.ptr(q), d, _lib.ptr(v), d, 0, None, None, 0, _lib.ptr(pos),
              _lib.ptr(holder.codebooks), _lib.ptr(holder.sizes), _lib.ptr(holder.indptr),
              _lib.ptr(holder.packed_kv), holder.packed_kv.shape[1], _lib.ptr(holder.suffix_kv), 1,
              256, _lib.ptr(holder.suffix_table), holder.prompt_length, holder.max_tiles, None, None,
              None, hq, hkv,
              index.num_buckets, d, 1.0 / float(temperature), float(beta), float(target_tokens),
              int(iters), fitted_sink_tokens(), float(sm_scale), int(num_splits), 1,
              _lib.ptr(ws.buffer), ws.nbytes,
              _lib.ptr(out), d, _lib.ptr(lse), _lib.ptr(csr_out), _lib.stream(dev))
    return PagedSparseAttentionResult(output=out, logsumexp=lse)
