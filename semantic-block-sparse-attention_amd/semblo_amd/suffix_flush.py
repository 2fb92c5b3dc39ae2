"""Generated tokens moved from the exact suffix into the clusters (the reference's
semblo/vllm_plugin/suffix_flush.py).

With ``SEMBLO_SUFFIX_FLUSH_EVERY=F`` (> 0) the newest ``SEMBLO_SUFFIX_KEEP_EXACT=W``
generated tokens stay exact, and whenever the exact suffix reaches W + F tokens
everything older than the newest W is moved into the clusters (flush_range,
suffix_flush.py:140-152).  A moved token joins the cluster of its nearest
descriptor (cosine in the routing space, all-zero descriptors never chosen,
suffix_flush.py:154-170), the centroids stay, and the cluster-ordered store is
laid out again with every cluster's old rows followed by its newcomers in
position order, each run page-aligned (repack_plan / repack_apply,
suffix_flush.py:55-137).

Here the flush is four libsbsa calls over the arena (semblo_amd.arena), all on
the device: the assignment (sbsa_nearest_cluster, on the pre-RoPE keys the
decode step kept beside the suffix K/V), the counts (sbsa_append_rows), the old
runs moved to their new starts (sbsa_repack_runs, into the arena's spare store)
and the newcomers written after them (sbsa_append_kv).  The spare store is then
copied back, so every address a captured decode step reads stays fixed, and
``prompt_length_t`` advances on the device (suffix_flush.py:226-231).
"""
from __future__ import annotations

import os

import torch

from . import _lib
from .token_outer_prefill import append_rows, nearest_cluster


def flush_every() -> int:
    """SEMBLO_SUFFIX_FLUSH_EVERY (suffix_flush.py:28-29); 0 leaves the suffix exact."""
    return int(os.environ.get("SEMBLO_SUFFIX_FLUSH_EVERY", "0") or 0)


def keep_exact() -> int:
    """SEMBLO_SUFFIX_KEEP_EXACT (suffix_flush.py:32-33)."""
    return int(os.environ.get("SEMBLO_SUFFIX_KEEP_EXACT", "1024") or 1024)


def flush_room() -> int:
    """SEMBLO_SUFFIX_FLUSH_ROOM: generated positions the packed store has room for
    (the reference sizes its arena's packed store for every position the model holds,
    arena.py:88-96); default 65,536."""
    return int(os.environ.get("SEMBLO_SUFFIX_FLUSH_ROOM", "65536") or 65536)


def flush_range(prompt_len: int, written: int, plen_cur: int, keep: int, every: int):
    """The positions [frm, to) to move now, or None (suffix_flush.py:140-152).

    ``written`` generated tokens sit at positions [prompt_len, prompt_len + written);
    those below ``plen_cur`` were moved already.  Once the exact suffix holds keep +
    every tokens, all but the newest ``keep`` move."""
    live = prompt_len + written - plen_cur
    if every > 0 and live >= keep + every:
        return plen_cur, prompt_len + written - keep
    return None


def flush_layer(arena, frm: int, to: int) -> int:
    """Move positions [frm, to) of the arena's exact suffix into its clusters
    (flush_layer, suffix_flush.py:173-231).  Returns the widest run layout in rows."""
    n = int(to) - int(frm)
    if n <= 0:
        return 0
    if arena.suffix_kpre is None or arena.inverse is None:
        raise RuntimeError("the arena was made without the suffix flush (flush_room = 0)")
    if int(frm) != arena.prompt_length:
        raise RuntimeError(f"a flush moves the oldest exact positions: from {arena.prompt_length}, "
                           f"not {frm}")
    if int(to) > arena.first_prompt_length + arena.flush_room:
        raise RuntimeError(f"the packed store has room for {arena.flush_room} moved positions "
                           f"(SEMBLO_SUFFIX_FLUSH_ROOM); position {to - 1} does not fit")
    packed = arena.packed_kv
    dev = packed.device
    _, width, hkv, d = packed.shape
    c = arena.num_clusters
    align = arena.page_align
    s = _lib.stream(dev)
    bs = arena.suffix_block
    pos = torch.arange(int(frm), int(to), device=dev, dtype=torch.int64)
    blk = pos // bs
    phys = arena.suffix_table[blk].to(torch.int64)
    off = pos - blk * bs
    kpre = arena.suffix_kpre[phys, off]                       # [n, Hkv, D]
    k_new = arena.suffix_kv[0, phys, off]
    v_new = arena.suffix_kv[1, phys, off]
    ids = nearest_cluster(kpre, arena.codebooks, router_pass=True)      # [Hkv, n]
    # the new layout: every cluster's run grows by its newcomers, runs page-aligned
    _, counts, _ = append_rows(ids, arena.indptr, arena.sizes)
    new_sizes = arena.sizes.to(torch.int64) + counts.to(torch.int64)
    padded = (new_sizes + align - 1) // align * align
    new_indptr = torch.zeros(hkv, c + 1, dtype=torch.int64, device=dev)
    new_indptr[:, 1:] = padded.cumsum(1)
    widest = int(new_indptr[:, -1].max())                     # one host read per flush
    if widest > width:
        raise RuntimeError(f"the flushed layout needs {widest} rows; the arena holds {width}")
    new_indptr = new_indptr.to(torch.int32)
    if arena.spare is None:
        arena.spare = torch.empty_like(packed)
    dst = arena.spare
    old_rows = arena.inverse[:, :frm].clone()
    _lib.call("sbsa_repack_runs", _lib.ptr(packed), _lib.ptr(dst), width, hkv, d, int(frm),
              _lib.ptr(old_rows), old_rows.stride(0), _lib.ptr(arena.indptr), _lib.ptr(new_indptr), c,
              _lib.ptr(arena.posting), arena.posting.shape[1], _lib.ptr(arena.inverse),
              arena.inverse.stride(0), s)
    arena.indptr.copy_(new_indptr)                            # same address as before
    rows, counts, _ = append_rows(ids, arena.indptr, arena.sizes)
    kk, vv = k_new.contiguous(), v_new.contiguous()
    _lib.call("sbsa_append_kv", _lib.ptr(kk), _lib.ptr(vv), kk.stride(0), kk.stride(1), n, hkv, d,
              _lib.ptr(rows), int(frm), _lib.ptr(dst), width, _lib.ptr(arena.posting),
              arena.posting.shape[1], _lib.ptr(arena.inverse), arena.inverse.shape[1],
              _lib.ptr(arena.sizes), _lib.ptr(counts), c, None, s)
    packed[:, :widest].copy_(dst[:, :widest])
    arena.prompt_length = int(to)
    arena.index.prompt_length = int(to)
    arena.index.max_position = int(to) - 1
    arena.prompt_length_t.fill_(int(to))
    arena.flushes += 1
    return widest


def maybe_flush(arena, keep: int | None = None, every: int | None = None):
    """Before a decode step (SuffixFlusher.before_step, suffix_flush.py:264-302): move
    the suffix's oldest positions when it has grown to keep + every.  Returns the range
    moved, or None."""
    keep = keep_exact() if keep is None else int(keep)
    every = flush_every() if every is None else int(every)
    rng = flush_range(arena.first_prompt_length, arena.steps, arena.prompt_length, keep, every)
    if rng is not None:
        flush_layer(arena, *rng)
    return rng
