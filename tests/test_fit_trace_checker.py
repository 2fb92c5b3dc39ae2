"""The k-means step checker of the GPU build tests (gpu_util.check_fit_trace), run on the
CPU against a trace made from the oracle itself: an exact trace passes with no flips, and
plausible faults (a last-index tie-break, an off-by-one cluster, a dropped row in the sums)
fail."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gpu_util import assignment_near_ties, bf16_midpoint_gap, check_fit_trace
from oracle import reference_cpu as ref


def _oracle_trace(length=2048, d=64, seed=3):
    gen = torch.Generator().manual_seed(seed)
    centres = torch.randn(16, d, generator=gen)
    k = centres[torch.randint(0, 16, (length,), generator=gen)] + 0.3 * torch.randn(length, d, generator=gen)
    product = ref.routing_normalize_keys(k[:, None].to(torch.bfloat16))
    steps, draws = [], []
    ref.build_flat_index(product, codebook_seed=1, fit_steps=steps, traces=draws)
    st = steps[0]
    space = F.normalize(ref.routing_space(product[:, 0]).float(), dim=-1)
    sample = [x[1] for x in draws[0] if x[0] == "sample"][0]
    iters = len(st["steps"])
    tr = dict(space_f32=space, space_bf16=space.to(torch.bfloat16), sample=sample,
              entry_centroids=[s["entry"].to(torch.bfloat16) for s in st["steps"]],
              assign=[s["assign"] for s in st["steps"]],
              sums=torch.stack([s["sums"] for s in st["steps"]]),
              counts=torch.stack([s["counts"].to(torch.int32) for s in st["steps"]]),
              final_centroids_f32=st["final_centroids"],
              final_centroids=st["final_centroids"].to(torch.bfloat16),
              final_assign=st["final_assign"].clone())
    assert iters == 8
    return product[:, 0], tr, st


def test_exact_trace_passes_with_no_flips():
    product, tr, st = _oracle_trace()
    rep = check_fit_trace(product, tr, st["steps"], st["final_assign"], st["final_centroids"])
    assert rep["moved"] == 0 and rep["origin_flips"] == 0 and rep["first_departure"] == -1


def test_off_by_one_cluster_fails():
    product, tr, st = _oracle_trace()
    a = tr["final_assign"]
    a[17] = (a[17] + 1) % tr["final_centroids"].shape[0]
    with pytest.raises(AssertionError):
        check_fit_trace(product, tr, st["steps"], st["final_assign"], st["final_centroids"])


def test_dropped_row_in_the_sums_fails():
    product, tr, st = _oracle_trace()
    i = 3
    a = tr["assign"][i]
    tr["sums"] = tr["sums"].clone()
    tr["sums"][i, a[0]] -= tr["space_f32"][tr["sample"][0]]
    with pytest.raises(AssertionError):
        check_fit_trace(product, tr, st["steps"], st["final_assign"], st["final_centroids"])


def test_last_index_tie_break_fails():
    # two identical centroids: every row that prefers them ties exactly, far from any
    # rounding midpoint in general; taking the last index is not a near-tie
    gen = torch.Generator().manual_seed(0)
    x = F.normalize(torch.randn(256, 32, generator=gen), dim=-1).to(torch.bfloat16)
    cent = F.normalize(torch.randn(8, 32, generator=gen), dim=-1)
    cent[5] = cent[2]
    cb = cent.to(torch.bfloat16)
    first = ref.argmax_sim_chunked(x.float(), cb.float(), 1024)
    last = first.clone()
    last[first == 2] = 5
    assert int((first == 2).sum()) > 0
    gaps = bf16_midpoint_gap((x.double() @ cb.double().T)[first == 2, 2])
    if bool((gaps > 1e-4).any()):
        with pytest.raises(AssertionError):
            assignment_near_ties(x, cb, last, first)


def _router_space(r: torch.Tensor):
    """The GPU build's key space of a bf16 router output r: two fp32 normalisations."""
    s = F.normalize(F.normalize(r.float(), dim=-1), dim=-1)
    return s, s.to(torch.bfloat16)


def _reordered_router(k: torch.Tensor) -> torch.Tensor:
    """A key router that sums the squares in another order than torch's (pairwise halves,
    then the halves reversed), as a GPU wave reduction does."""
    x = k.float()
    ss = x.pow(2)
    while ss.shape[-1] > 1:
        h = ss.shape[-1] // 2
        ss = ss[..., h:] + ss[..., :h]
    n = ss.sqrt().clamp_min(1e-12)
    return (x / n).to(torch.bfloat16)


def test_key_router_check_accepts_a_reordered_router():
    from gpu_util import check_key_router
    gen = torch.Generator().manual_seed(5)
    k = (torch.randn(4096, 256, generator=gen) * 3).to(torch.bfloat16)
    r = _reordered_router(k)
    s32, s16 = _router_space(r)
    rep = check_key_router(k, s32, s16, "reordered")
    assert rep["router_elements"] == int((r != ref.routing_normalize_keys(k)).sum())


def test_key_router_check_rejects_a_flip_that_is_not_a_near_tie():
    """One element one bf16 step off, in a row that also holds a true rounding near-tie
    elsewhere: the element itself must be the near-tie, so the check fails."""
    from gpu_util import check_key_router, router_flip_margin
    gen = torch.Generator().manual_seed(6)
    k = (torch.randn(512, 128, generator=gen)).to(torch.bfloat16)
    r = ref.routing_normalize_keys(k).clone()
    exact = F.normalize(k.double(), dim=-1)
    gap = bf16_midpoint_gap(exact) / exact.abs().clamp_min(1e-30)
    row = int(torch.nonzero((gap < router_flip_margin(128)).any(-1))[0]) if bool(
        (gap < router_flip_margin(128)).any()) else 0
    col = int(gap[row].argmax())                        # the element farthest from a midpoint
    bits = r.view(torch.int16)
    bits[row, col] += 1
    s32, s16 = _router_space(r)
    with pytest.raises(AssertionError, match="without a rounding near-tie"):
        check_key_router(k, s32, s16, "corrupt")


def test_key_router_check_rejects_a_space_that_no_router_output_gives():
    from gpu_util import check_key_router
    gen = torch.Generator().manual_seed(7)
    k = torch.randn(256, 64, generator=gen).to(torch.bfloat16)
    s32, s16 = _router_space(ref.routing_normalize_keys(k))
    s32 = s32.clone()
    s32[9, 3] += 1e-5
    with pytest.raises(AssertionError, match="not the routing space"):
        check_key_router(k, s32, s16, "space")


def test_restarted_cluster_must_take_its_drawn_row():
    """An iteration that leaves a cluster empty restarts it on the drawn sample row; a
    trace whose next centroid for it is another row fails."""
    gen = torch.Generator().manual_seed(23)
    length, d = 1024, 64
    dirs = torch.randn(5, d, generator=gen)
    k = dirs[torch.randint(0, 5, (length,), generator=gen)] + 1e-3 * torch.randn(length, d, generator=gen)
    product = ref.routing_normalize_keys(k[:, None].to(torch.bfloat16))
    steps, draws = [], []
    ref.build_flat_index(product, codebook_seed=5, fit_steps=steps, traces=draws)
    st = steps[0]
    space = F.normalize(ref.routing_space(product[:, 0]).float(), dim=-1)
    sample = [x[1] for x in draws[0] if x[0] == "sample"][0]
    empties = [x[1] for x in draws[0] if x[0] == "empty"]
    restarts = {i: e for i, e in enumerate(empties) if e.numel()}
    assert restarts, "the fit must leave a cluster empty"
    tr = dict(space_f32=space, space_bf16=space.to(torch.bfloat16), sample=sample,
              entry_centroids=[s["entry"].to(torch.bfloat16) for s in st["steps"]],
              assign=[s["assign"] for s in st["steps"]],
              sums=torch.stack([s["sums"] for s in st["steps"]]),
              counts=torch.stack([s["counts"].to(torch.int32) for s in st["steps"]]),
              final_centroids_f32=st["final_centroids"],
              final_centroids=st["final_centroids"].to(torch.bfloat16),
              final_assign=st["final_assign"].clone(), restarts=restarts)
    rep = check_fit_trace(product[:, 0], tr, st["steps"], st["final_assign"], st["final_centroids"])
    assert rep["restarted"] == sum(int(e.numel()) for e in restarts.values())
    assert rep["shadow_reseeds"] == [] and rep["shadow_moved"] == 0
    it = min(restarts)
    bad = dict(tr, restarts={**restarts, it: (restarts[it] + 1) % sample.numel()})
    with pytest.raises(AssertionError):
        check_fit_trace(product[:, 0], bad, st["steps"], st["final_assign"], st["final_centroids"])
