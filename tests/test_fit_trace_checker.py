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
