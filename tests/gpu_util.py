"""Shared helpers of the GPU parity tests (selection near-tie accounting, fp64 references)."""
from __future__ import annotations

import math

import torch

from oracle import reference_cpu as ref

# Tolerances of the attention outputs (bf16), from the build's contract.
ATOL = 2e-2
RTOL = 1e-2
# A selection difference is a near-tie when the cluster's score lies within this
# relative margin of the cut (theta) of either run.
NEAR_TIE_REL = 1e-4


def assert_close_bf16(got: torch.Tensor, want: torch.Tensor, what: str = "") -> float:
    g = got.double().cpu()
    w = want.double().cpu()
    err = (g - w).abs()
    bad = err > ATOL + RTOL * w.abs()
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {bad.numel()} values off by more than "
        f"{ATOL} + {RTOL}*|ref| (max err {float(err.max()):.4g})")
    return float(err.max())


def compare_selection(sel_gpu: torch.Tensor, sel_ref: torch.Tensor, score: torch.Tensor,
                      theta_ref: torch.Tensor, theta_gpu: torch.Tensor | None = None) -> dict:
    """sel_* [Q, Hkv, C] bool, score [Q, Hkv, C] (oracle scores), theta [Q, Hkv].

    Every differing cluster must be a near-tie: its score within NEAR_TIE_REL
    (relative) of theta, plus the bisection's resolution (range * 2^-16).
    Returns counts for the report.
    """
    sel_gpu = sel_gpu.cpu()
    sel_ref = sel_ref.cpu()
    diff = sel_gpu != sel_ref
    n_diff = int(diff.sum())
    if n_diff == 0:
        return {"differ": 0, "near_ties": 0, "pairs": int(sel_ref.shape[0] * sel_ref.shape[1])}
    live = score > -1e38
    big = torch.full_like(score, 1e38)
    rng = score.max(-1).values - torch.where(live, score, big).min(-1).values
    slack = rng.clamp_min(0) * 2.0 ** -16
    thetas = [theta_ref.cpu()]
    if theta_gpu is not None:
        thetas.append(theta_gpu.cpu())
    ok = torch.zeros_like(diff)
    for th in thetas:
        tol = NEAR_TIE_REL * th.abs().clamp_min(1.0) + slack
        ok |= (score - th[..., None]).abs() <= tol[..., None]
    bad = diff & ~ok
    assert not bool(bad.any()), (
        f"{int(bad.sum())} selection differences are not near-ties, e.g. "
        f"{torch.nonzero(bad)[:5].tolist()}")
    return {"differ": n_diff, "near_ties": n_diff, "pairs": int(sel_ref.shape[0] * sel_ref.shape[1])}


def attention_reference(q: torch.Tensor, keys_pos: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        sm_scale: float) -> torch.Tensor:
    """fp64 softmax attention. q [Q, Hq, D]; keys_pos bool [Q, Hkv, L] (the key set of every
    query and KV head); k/v [L, Hkv, D] in prompt order."""
    qd = q.double()
    kd = k.double()
    vd = v.double()
    qn, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = torch.zeros(qn, hq, d, dtype=torch.float64)
    for h in range(hkv):
        s = torch.einsum("qgd,ld->qgl", qd[:, h * g:(h + 1) * g], kd[:, h]) * sm_scale
        m = keys_pos[:, h][:, None, :]
        s = s.masked_fill(~m, -math.inf)
        p = torch.softmax(s, dim=-1)
        out[:, h * g:(h + 1) * g] = torch.einsum("qgl,ld->qgd", p, vd[:, h])
    return out


def cluster_position_mask(posting: torch.Tensor, indptr: torch.Tensor, counts: torch.Tensor,
                          length: int) -> torch.Tensor:
    """[Hkv, C, L] bool: the positions of the first counts[h, c] rows of cluster c's run."""
    hkv, c = counts.shape
    m = torch.zeros(hkv, c, length, dtype=torch.bool)
    for h in range(hkv):
        for cl in range(c):
            s = int(indptr[h, cl])
            n = int(counts[h, cl])
            if n:
                m[h, cl, posting[h, s:s + n].long()] = True
    return m


def oracle_select(vectors, codebooks, sizes, *, temperature, beta, target, g_union=None):
    """The oracle's scores and bisection; one size snapshot ([1, Hkv, C]) serves every query."""
    prob = ref.mixture_probs(vectors.cpu(), None, codebooks.cpu(), temperature)
    if g_union is None:
        g_union = prob.shape[0] if sizes.shape[0] == 1 else 1
    return ref.theta_select(prob, sizes.cpu(), beta=beta, target_tokens=target, g_union=max(g_union, 1))


def membership_near_ties(product: torch.Tensor, codebooks: torch.Tensor, got: torch.Tensor,
                         want: torch.Tensor) -> tuple[int, float]:
    """Keys whose cluster differs between two builds: check each is a near-tie of the bf16
    similarity argmax under the reference build's centroids.  The similarities are bf16
    values, so a tie is resolved at bf16 resolution: the two clusters' fp32 similarities must
    lie within two bf16 ulps (2^-7 relative) of each other.  Returns (moved, worst gap / ulp).
    """
    moved = torch.nonzero(got != want)
    if moved.numel() == 0:
        return 0, 0.0
    space = torch.nn.functional.normalize(product.float(), dim=-1)
    worst = 0.0
    for h, pos in moved.tolist():
        cent = torch.cat([codebooks[h, 0], codebooks[h, 1]], dim=-1).float()
        x = space[pos, h].to(torch.bfloat16).double()
        s_want = float(x @ cent[want[h, pos]].double())
        s_got = float(x @ cent[got[h, pos]].double())
        ulp = 2.0 ** -8 * max(abs(s_want), abs(s_got), 1e-6)
        worst = max(worst, abs(s_want - s_got) / ulp)
    assert worst <= 2.0, f"a moved key is not a near-tie: similarity gap {worst:.2f} bf16 ulps"
    return int(moved.shape[0]), worst
