"""The CPU oracle against the reference's golden vectors and against closed forms.

The golden files were written by the reference's own code (tests/golden/make_golden.py):
ProductPostingIndex.build on CPU (state.py:477-948) and, under the Triton CPU
interpreter, the flat scoring and RESIDENT selection kernels (fused_select.py).
"""
from __future__ import annotations

import math
from pathlib import Path

import pytest
import torch

from oracle import reference_cpu as ref
from synth import golden_keys, keys_checksum

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return torch.load(GOLDEN / name, weights_only=True)


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("kmeans_*.pt")))
def test_block_build_matches_the_reference_bit_for_bit(name):
    g = _load(name)
    length, hkv, d = int(g["length"]), int(g["hkv"]), int(g["d"])
    k_pre = golden_keys(length, hkv, d, int(g["seed"]), mixture=name.endswith("_mix.pt"))
    assert torch.allclose(keys_checksum(k_pre), g["keys_checksum"], rtol=0, atol=1e-6), \
        "the key generator changed"
    product = ref.routing_normalize_keys(k_pre)
    if "product" in g:
        assert torch.equal(product, g["product"])
    idx = ref.build_flat_index(product, codebook_seed=int(g["codebook_seed"]),
                               min_clusters_log2=int(g["min_log2"]),
                               sink_tokens=int(g["sink"]) if "sink" in g else 0)
    assert torch.equal(idx["sizes"], g["sizes"])
    assert torch.equal(idx["indptr"], g["indptr"])
    assert torch.equal(idx["posting"], g["posting"])
    assert torch.equal(idx["inverse"], g["inverse"])
    assert torch.equal(idx["codebooks"], g["codebooks"])


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("select_*.pt")))
def test_scores_match_the_reference_torch_form(name):
    g = _load(name)
    prob = ref.mixture_probs(g["vectors"], None, g["codebooks"], float(g["tau"]))
    # the reference's torch-form scorer, the same ops on CPU: bit-exact
    assert torch.equal(prob, g["prob"])
    want = ref.mixture_probs_fp64(g["vectors"], None, g["codebooks"], float(g["tau"]))
    assert torch.allclose(prob.double(), want, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("select_*.pt")))
def test_bisection_matches_the_reference_kernel(name):
    g = _load(name)
    out = ref.theta_select(g["prob"], g["sizes"], beta=float(g["beta"]),
                           target_tokens=float(g["target"]), g_union=int(g["g_union"]))
    assert torch.equal(out["qmask"], g["qmask"])
    assert torch.equal(out["bitmask"], g["bitmask"])
    assert torch.equal(out["counts"], g["counts"])
    assert torch.equal(out["tokens"], g["tokens"])


def test_sorted_rule_is_a_subset_of_the_bisection():
    g = _load("select_q64_c128.pt")
    out = ref.theta_select(g["prob"], g["sizes"], beta=0.25, target_tokens=512, g_union=32)
    sorted_sel = ref.sorted_select(out["score"], g["sizes"], 512, g_union=32)
    assert not (sorted_sel & ~out["sel"]).any()
    # the extra clusters sit within range * 2^-16 of the sorted cut
    extra = out["sel"] & ~sorted_sel
    rng = (out["score"].max(-1).values - torch.where(out["score"] > -1e38, out["score"],
           torch.full_like(out["score"], 1e38)).min(-1).values)
    for q, h, c in torch.nonzero(extra).tolist():
        assert out["score"][q, h, c] >= out["theta"][q, h]
        assert out["score"][q, h, c] - out["theta"][q, h] <= rng[q, h] * 2 ** -15 + 2e-5


def test_dead_clusters_are_never_selected_and_all_fit_takes_everything():
    gen = torch.Generator().manual_seed(5)
    prob = torch.rand(8, 2, 64, generator=gen)
    sizes = torch.randint(0, 30, (1, 2, 64), generator=gen, dtype=torch.int32)
    sizes[..., ::3] = 0
    out = ref.theta_select(prob, sizes, beta=0.25, target_tokens=10 ** 6, g_union=8)
    live = sizes[0] > 0
    assert torch.equal(out["sel"], live[None].expand_as(out["sel"]))
    out = ref.theta_select(prob, sizes, beta=0.25, target_tokens=100, g_union=8)
    assert not (out["sel"] & ~live[None]).any()
    have = (out["sel"] * sizes[0][None]).sum(-1)
    assert (have >= 100).all()


def test_router_closed_form():
    x = torch.randn(7, 4, 256).to(torch.bfloat16)
    v = ref.trivial_router_vectors(x, 1)
    n = v.float().norm(dim=-1)
    assert torch.allclose(n, torch.ones_like(n), atol=4e-3)
    # idempotent up to one bf16 rounding
    assert torch.allclose(ref.trivial_router_vectors(v, 1).float(), v.float(), atol=2 ** -8)


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("router_*.pt")))
def test_router_matches_the_reference_golden(name):
    """S0 bit for bit against vectors written by the reference's own router
    (trivial_router.py:55-61, the torch path), and the fixtures are strong
    enough that dropping the intermediate bf16 rounding or the eps fails."""
    g = torch.load(GOLDEN / name, weights_only=True)
    x, f = g["x"], int(g["factors"])
    assert torch.equal(ref.trivial_router_vectors(x, f), g["out"])
    q, h, d = x.shape
    halves = x.float().view(q, h, f, d // f)
    unit = halves / halves.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    no_eps = halves / halves.norm(dim=-1, keepdim=True)
    no_eps = no_eps.to(x.dtype).float()
    no_eps = (no_eps / no_eps.norm(dim=-1, keepdim=True)).to(x.dtype).view(q, h, d)
    assert not torch.equal(no_eps, g["out"])           # the zero rows turn to NaN
    if name.endswith("_d16_f2.pt"):
        no_round = (unit / unit.norm(dim=-1, keepdim=True).clamp_min(1e-12)).to(x.dtype)
        assert not torch.equal(no_round.view(q, h, d), g["out"])


def test_cluster_count_rule():
    assert ref.num_flat_clusters(131072) == 128
    assert ref.num_flat_clusters(524288) == 256
    assert ref.num_flat_clusters(32768) == 128
    assert ref.num_flat_clusters(8192) == 128
    assert ref.num_flat_clusters(512) == 128
    assert ref.num_flat_clusters(100) == 64


def test_lse_merge_closed_form():
    o = torch.randn(3, 5)
    out, lse = ref.lse_merge(o, torch.zeros(3), o, torch.zeros(3))
    assert torch.allclose(out, o.double())
    assert torch.allclose(lse, torch.full((3,), math.log(2.0), dtype=torch.float64))


def test_reverse_index_is_the_transpose():
    gen = torch.Generator().manual_seed(1)
    sel = torch.rand(50, 2, 64, generator=gen) < 0.2
    live = torch.rand(2, 64, generator=gen) < 0.9
    counts, indptr, qvals = ref.reverse_index(sel, live)
    for h in range(2):
        for c in range(64):
            e0 = int(indptr[h * 64 + c])
            n = int(counts[h, c])
            got = qvals[e0:e0 + n].tolist()
            want = torch.nonzero(sel[:, h, c] & live[h, c]).flatten().tolist()
            assert got == want


# ---- S10: token-order append ---------------------------------------------------

def test_reserved_layout_is_proportional_paged_and_fits():
    """The properties the reference's own test asserts (test_token_outer_prefill.py:14-27)
    and one case worked by hand."""
    sizes = torch.tensor([[100, 0, 300, 20], [50, 150, 0, 200]])
    width = 16 * 200
    reserve = ref.reserved_layout(sizes, n_ref=420, total_tokens=2000, width=width, align=16)
    assert reserve.shape == sizes.shape
    assert bool((reserve % 16 == 0).all()) and bool((reserve >= 16).all())
    assert bool((reserve.sum(dim=1) <= width).all())
    assert bool((reserve.double() >= sizes.double() * (2000 / 420)).all())
    assert 2.5 < reserve[0, 2].item() / reserve[0, 0].item() < 3.5
    # head 0 by hand: shares 476.19, 0, 1428.57, 95.24 -> pages 30, 1, 90, 6 (2032 rows);
    # the 73 spare pages split 0.238 / 0 / 0.714 / 0.048 -> 17, 0, 52, 3 more pages
    assert reserve[0].tolist() == [752, 16, 2272, 144]


def test_reserved_layout_refuses_a_store_too_small():
    with pytest.raises(RuntimeError):
        ref.reserved_layout(torch.tensor([[10, 10]]), n_ref=20, total_tokens=1000, width=512,
                            align=16)


def test_append_rows_known_answers():
    """test_token_outer_prefill.py:30-38 of the reference."""
    indptr = torch.tensor([[0, 32, 64, 96]], dtype=torch.int32)
    sizes = torch.tensor([[5, 0, 30]], dtype=torch.int32)
    rows, counts = ref.append_rows(torch.tensor([[2, 0, 2, 1, 0]]), indptr, sizes)
    assert counts.tolist() == [[2, 1, 2]]
    assert rows.tolist() == [[94, 5, 95, 32, 6]]


def test_append_rows_matches_a_stable_sort():
    """The scan against the rank of each key in a stable sort of the ids."""
    gen = torch.Generator().manual_seed(5)
    c, n = 64, 3000
    ids = torch.randint(0, c, (2, n), generator=gen)
    sizes = torch.randint(0, 50, (2, c), generator=gen)
    indptr = torch.zeros(2, c + 1, dtype=torch.int64)
    indptr[:, 1:] = torch.cumsum(sizes + 200, 1)
    rows, counts = ref.append_rows(ids, indptr, sizes)
    for h in range(2):
        order = torch.argsort(ids[h], stable=True)
        cnt = torch.bincount(ids[h], minlength=c)
        first = torch.cumsum(cnt, 0) - cnt
        rank = torch.empty(n, dtype=torch.int64)
        rank[order] = torch.arange(n) - first[ids[h][order]]
        assert torch.equal(rows[h], indptr[h, ids[h]] + sizes[h, ids[h]] + rank)
        assert torch.equal(counts[h], cnt)


def test_nearest_cluster_is_the_fp64_argmax_and_skips_dead_descriptors():
    gen = torch.Generator().manual_seed(6)
    n, c, d = 400, 128, 64
    keys = torch.randn(n, d, generator=gen).to(torch.bfloat16)
    cents = torch.nn.functional.normalize(torch.randn(c, d, generator=gen), dim=-1)
    cents[7] = 0
    cents[90] = 0
    cb = torch.stack(list(cents.chunk(2, dim=-1))).to(torch.bfloat16)      # [2, C, d/2]
    ids, sim = ref.nearest_cluster(keys, cb, return_sim=True)
    # fp64 restatement of the same chain
    unit = keys.double() / keys.double().norm(dim=-1, keepdim=True)
    unit = unit.to(torch.bfloat16).double()
    unit = unit / unit.norm(dim=-1, keepdim=True)
    c64 = torch.cat([cb[0], cb[1]], dim=-1).double()
    s64 = unit @ c64.t()
    s64[:, [7, 90]] = -math.inf
    top2 = s64.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 1e-5
    assert int(clear.sum()) > n * 0.9
    assert torch.equal(ids[clear], s64.argmax(-1)[clear])
    assert not bool(((ids == 7) | (ids == 90)).any())
    # equal maxima: the first index
    dup = torch.cat([cb, cb], dim=1)                                          # clusters c..2c-1 repeat
    assert bool((ref.nearest_cluster(keys, dup) < c).all())


def test_relayout_keeps_each_key_at_its_offset_in_the_new_run():
    sizes = torch.tensor([[3, 0, 5]])
    old_ip = torch.tensor([[0, 16, 16, 32]])
    new_ip = torch.tensor([[0, 48, 64, 112]])
    old_rows = torch.tensor([[0, 16, 1, 17, 18, 2, 19, 20]])   # positions 0..7
    new = ref.relayout_rows(old_rows, old_ip, new_ip)
    assert new.tolist() == [[0, 64, 1, 65, 66, 2, 67, 68]]
    assert int(sizes.sum()) == new.shape[1]


def test_sink_partition_properties():
    """The reference's own sink tests (tests/test_fitted_sink.py:62-82) on the oracle:
    positions < S are exactly cluster 0, in order, and nothing else is; cluster 0's
    descriptor is zero and every used cluster's is not."""
    sink = 32
    k = torch.randn(512, 2, 16, generator=torch.Generator().manual_seed(0))
    product = ref.routing_normalize_keys(k.to(torch.bfloat16))
    idx = ref.build_flat_index(product, unit_tokens=16, min_clusters_log2=3, sample_size=256,
                               fit_iters=2, sink_tokens=sink)
    for h in range(2):
        ip, sz, post = idx["indptr"][h], idx["sizes"][h], idx["posting"][h]
        assert torch.equal(post[int(ip[0]):int(ip[0]) + int(sz[0])], torch.arange(sink, dtype=torch.int32))
        for c in range(1, sz.numel()):
            assert bool((post[int(ip[c]):int(ip[c]) + int(sz[c])] >= sink).all())
        assert int(sz.sum()) == 512
    cb = idx["codebooks"].float()
    assert torch.count_nonzero(cb[:, :, 0]) == 0
    used = idx["sizes"][:, 1:] > 0
    assert bool((cb[:, :, 1:].norm(dim=-1).sum(1)[used] > 0).all())


@pytest.mark.parametrize("sink, length, match", [(24, 512, "multiple of 16"), (512, 512, "too few keys"),
                                                 (496, 512, "too few keys")])
def test_sink_settings_that_do_not_compose_are_refused(sink, length, match):
    """state.py:26-34 (the refusals of tests/test_fitted_sink.py:85-97 that apply here)."""
    k = torch.randn(length, 1, 16, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match=match):
        ref.build_flat_index(ref.routing_normalize_keys(k), unit_tokens=16, min_clusters_log2=3,
                             sample_size=256, fit_iters=2, sink_tokens=sink)


def test_sink_hold_out_and_forced_bit_known_answers():
    """tests/test_fitted_sink.py:100-117 of the reference: the selector's view hides
    cluster 0, the budget shrinks by S, the caller's sizes are untouched, and the forced
    bit is bit 0 of word 0 (other bits untouched)."""
    sizes = torch.tensor([[[32, 10, 0, 7]], [[32, 3, 5, 0]]], dtype=torch.int32)
    held, target = ref.hold_out_sink(sizes, 100, 32)
    assert target == 68
    assert (held[..., 0] == 0).all() and torch.equal(held[..., 1:], sizes[..., 1:])
    assert int(sizes[0, 0, 0]) == 32
    qmask = torch.zeros(3, 2, 2, dtype=torch.int32)
    qmask[1, 0, 1] = 5
    ref.force_sink_bit(qmask, None)
    got = ref.unpack_bits(qmask, 64)
    assert got[..., 0].all()
    assert int(got[..., 1:].sum()) == 2


def test_flush_range_keeps_the_exact_suffix_between_keep_and_keep_plus_every():
    """suffix_flush.py:140-152: simulated over a long generation, the moved ranges are
    contiguous from the prompt's end, and after each step's flush decision the exact
    suffix holds fewer than keep + every tokens, at least keep once it first reached
    keep + every, and exactly keep right after a move."""
    prompt, keep, every = 1000, 48, 32
    plen, moved = prompt, []
    for written in range(400):
        rng = ref.flush_range(prompt, written, plen, keep, every)
        live = prompt + written - plen
        if rng is not None:
            frm, to = rng
            assert frm == plen and to - frm >= every and live >= keep + every
            moved.append(rng)
            plen = to
        live = prompt + written - plen
        assert live < keep + every
        if moved:
            assert keep <= live
            assert live == keep or rng is None
    assert moved[0] == (prompt, prompt + every)
    assert len(moved) == (399 - (keep + every)) // every + 1
    assert all(a[1] == b[0] for a, b in zip(moved, moved[1:]))


def test_flush_store_known_answer_and_invariants():
    """The layout after a flush (suffix_flush.py:55-137) on a hand-worked case:
    sizes [2, 0, 3] at align 4 with newcomers to clusters [2, 0, 2] -> sizes [3, 0, 5],
    runs at rows 0, 4, 4 (the padded runs 4 + 0 + 8), each cluster's old rows then its
    newcomers in position order; and, on random stores, no position lost or doubled."""
    posting = torch.tensor([[7, 3, -1, -1, 1, 0, 9, -1]])
    indptr = torch.tensor([[0, 4, 4, 8]])
    sizes = torch.tensor([[2, 0, 3]])
    ids = torch.tensor([[2, 0, 2]])
    runs, new_sizes, new_indptr = ref.flush_store(posting, indptr, sizes, ids, 20, 4)
    assert runs[0] == [[7, 3, 21], [], [1, 0, 9, 20, 22]]
    assert new_sizes.tolist() == [[3, 0, 5]] and new_indptr.tolist() == [[0, 4, 4, 12]]
    gen = torch.Generator().manual_seed(3)
    for trial in range(20):
        hkv, c, align = 2, 16, 16
        n_old = int(torch.randint(1, 300, (1,), generator=gen))
        n_new = int(torch.randint(0, 60, (1,), generator=gen))
        post, ip, sz = [], [], []
        for h in range(hkv):
            assign = torch.randint(0, c, (n_old,), generator=gen)
            perm = torch.randperm(n_old, generator=gen)
            counts = torch.bincount(assign, minlength=c)
            pad = (counts + align - 1) // align * align
            ptr = torch.zeros(c + 1, dtype=torch.int64)
            ptr[1:] = pad.cumsum(0)
            row = torch.full((int(ptr[-1]) + 1,), -1, dtype=torch.int64)
            fill = ptr[:-1].clone()
            for p in perm.tolist():
                row[fill[assign[p]]] = p
                fill[assign[p]] += 1
            post.append(row)
            ip.append(ptr)
            sz.append(counts)
        width = max(int(x.numel()) for x in post)
        posting = torch.stack([torch.cat([x, x.new_full((width - x.numel(),), -1)]) for x in post])
        ids = torch.randint(0, c, (hkv, n_new), generator=gen)
        runs, new_sizes, new_indptr = ref.flush_store(posting, torch.stack(ip), torch.stack(sz), ids,
                                                      n_old, align)
        for h in range(hkv):
            flat = sorted(p for lst in runs[h] for p in lst)
            assert flat == list(range(n_old + n_new))
            assert (new_indptr[h] % align == 0).all()
            assert (new_indptr[h, 1:] - new_indptr[h, :-1] >= new_sizes[h]).all()
            for b in range(c):
                old = posting[h, int(ip[h][b]):int(ip[h][b]) + int(sz[h][b])].tolist()
                newc = [n_old + i for i in range(n_new) if int(ids[h, i]) == b]
                assert runs[h][b] == old + newc
