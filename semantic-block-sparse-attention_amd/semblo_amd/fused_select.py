"""Centroid scoring and budget selection (S2 + S3) on HIP.

Same contract as the reference's ``theta_select_bitmask_flat``
(semblo/vllm_plugin/fused_select.py:806-919): the mixture probability of
every cluster for every (query, KV head) -- the flat form of the scorer,
s = (q0.c0 + q1.c1) / tau with bf16 operands and fp32 sums, log-softmax over
the clusters, plus logmix, exp, summed over the KV head's query heads
(fused_select.py:1097-1247) -- then the RESIDENT bisection of
``_streaming_select_kernel`` (fused_select.py:604-646).  One fused kernel:
the [Q, Hkv, C] probability is never written unless asked for.
"""
from __future__ import annotations

import torch

from . import _lib


def _vectors_3d(vectors: torch.Tensor) -> torch.Tensor:
    # [Q, Hq, R=1, I] -> [Q, Hq, I]
    if vectors.ndim == 4:
        if vectors.shape[2] != 1:
            raise NotImplementedError("the flat paper path routes one vector per head (R = 1)")
        vectors = vectors[:, :, 0]
    if vectors.stride(-1) != 1:
        vectors = vectors.contiguous()
    return vectors


def _logmix_2d(logmix: torch.Tensor | None, q: int, hq: int) -> torch.Tensor | None:
    if logmix is None:
        return None
    return logmix.reshape(q, hq).float().contiguous()


def theta_select_bitmask_flat(vectors: torch.Tensor, logmix: torch.Tensor | None,
                              codebooks: torch.Tensor, causal_sizes: torch.Tensor,
                              bitmask: torch.Tensor | None, *, temperature: float, beta: float,
                              target_tokens: int, g_union: int, tile: int = 512, iters: int = 16,
                              qmask: torch.Tensor | None = None, sink_tokens: int = 0,
                              prob_out: torch.Tensor | None = None,
                              theta_out: torch.Tensor | None = None,
                              **unused) -> tuple[torch.Tensor, torch.Tensor]:
    """Select each query's clusters under the budget; returns (counts, tokens) [Q, Hkv] int32.

    vectors [Q, Hq, 1, I] (or [Q, Hq, I]) bf16 routing vectors; logmix [Q, Hq, 1]
    fp32 (log mixture weight, all zero on the paper path); codebooks
    [Hkv, 2, C, I/2]; causal_sizes [NB, Hkv, C] int32 (NB may be 1 with a
    zero stride); bitmask [NB, Hkv, C/32] is OR-ed into (pre-zeroed by the
    caller); qmask [Q, Hkv, C/32] receives each query's own set.
    """
    if unused.get("group_desc") is not None or unused.get("cluster_descriptors") is not None:
        raise NotImplementedError("group and cluster descriptors are not on the flat paper path")
    v = _vectors_3d(vectors)
    q, hq, dim = v.shape
    hkv, two, c, df = codebooks.shape
    if two != 2 or dim != 2 * df:
        raise ValueError(f"codebooks {tuple(codebooks.shape)} and vectors {tuple(v.shape)} disagree")
    if causal_sizes.dtype != torch.int32 or causal_sizes.stride(-1) != 1:
        raise ValueError("causal_sizes must be int32 with a unit last stride")
    _lib.require_device(v, codebooks, causal_sizes)
    cb = codebooks if codebooks.is_contiguous() else codebooks.contiguous()
    lm = _logmix_2d(logmix, q, hq)
    counts = torch.empty(q, hkv, dtype=torch.int32, device=v.device)
    tokens = torch.empty_like(counts)
    s_nb = causal_sizes.stride(0) if causal_sizes.shape[0] > 1 else 0
    for t in (bitmask, qmask):
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous()):
            raise ValueError("bitmask / qmask must be contiguous int32")
    # query q belongs to block q // g_union: its sizes row (unless broadcast) and its bitmask row
    nb = (q + int(g_union) - 1) // max(int(g_union), 1)
    if causal_sizes.shape[0] > 1 and causal_sizes.shape[0] < nb:
        raise ValueError(f"causal_sizes has {causal_sizes.shape[0]} query blocks; {q} queries in "
                         f"blocks of {g_union} need {nb}")
    if bitmask is not None and (bitmask.shape[0] < nb or tuple(bitmask.shape[1:]) != (hkv, c // 32)):
        raise ValueError(f"bitmask {tuple(bitmask.shape)} must be [{nb}, {hkv}, {c // 32}] for {q} "
                         f"queries in blocks of {g_union}")
    if qmask is not None and tuple(qmask.shape) != (q, hkv, c // 32):
        raise ValueError(f"qmask {tuple(qmask.shape)} must be [{q}, {hkv}, {c // 32}]")
    _lib.call("sbsa_score_select", _lib.ptr(v), v.stride(0), v.stride(1), _lib.ptr(lm),
              _lib.ptr(cb), _lib.ptr(causal_sizes), s_nb, causal_sizes.stride(1), q, hq, hkv, c,
              dim, int(g_union), 1.0 / float(temperature), float(beta), float(target_tokens),
              int(iters), int(sink_tokens), _lib.ptr(bitmask), _lib.ptr(qmask), _lib.ptr(counts),
              _lib.ptr(tokens), _lib.ptr(prob_out), _lib.ptr(theta_out), _lib.stream(v.device))
    return counts, tokens


def flat_mixture_scores_qtiled(vectors: torch.Tensor, logmix: torch.Tensor | None,
                               codebooks: torch.Tensor, *, temperature: float,
                               **unused) -> torch.Tensor:
    """[Q, Hkv, C] fp32 mixture probability (fused_select.py:1250-1357 contract)."""
    v = _vectors_3d(vectors)
    q, hq, _ = v.shape
    hkv, _, c, _ = codebooks.shape
    prob = torch.empty(q, hkv, c, dtype=torch.float32, device=v.device)
    sizes = torch.ones(1, hkv, c, dtype=torch.int32, device=v.device)
    theta_select_bitmask_flat(v, logmix, codebooks, sizes, None, temperature=temperature, beta=0.0,
                              target_tokens=1, g_union=max(q, 1), iters=0, prob_out=prob)
    return prob
