"""S1/S1b on the GPU: the flat k-means block build against the oracle (itself pinned
bit-exact to the reference's ProductPostingIndex.build) and the reference's
golden vectors.

Both sides draw the same random rows (a CPU generator seeded alike), so the
partition must match; a key may change cluster only as a near-tie of the bf16
similarity argmax, which is counted and printed.
"""
from __future__ import annotations

from pathlib import Path

import pytest
import torch

from gpu_util import check_fit_trace
from oracle import reference_cpu as ref
from synth import golden_keys

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
DEV = "cuda"


def _build_gpu(product, **kw):
    from semblo_amd.state import ProductPostingIndex
    length = product.shape[0]
    idx = ProductPostingIndex.build(product.to(DEV), torch.arange(length, device=DEV), **kw)
    torch.cuda.synchronize()
    return idx


def _membership(posting, indptr, sizes):
    """position -> cluster, [Hkv, L]."""
    hkv, c = sizes.shape
    length = int(sizes[0].sum())
    out = torch.full((hkv, length), -1, dtype=torch.int64)
    for h in range(hkv):
        for cl in range(c):
            s, n = int(indptr[h, cl]), int(sizes[h, cl])
            out[h, posting[h, s:s + n].long()] = cl
    return out


def _check_index_invariants(idx, length):
    sizes = idx.bucket_sizes.cpu()
    indptr = idx.bucket_indptr.cpu()
    posting = idx.posting_positions.cpu()
    inverse = idx.inverse_positions().cpu()
    hkv, c = sizes.shape
    assert (sizes.sum(-1) == length).all()
    assert ((indptr[:, 1:] - indptr[:, :-1]) % 16 == 0).all()
    assert ((indptr[:, 1:] - indptr[:, :-1]) >= sizes).all()
    for h in range(hkv):
        seen = torch.zeros(length, dtype=torch.int64)
        for cl in range(c):
            s, n = int(indptr[h, cl]), int(sizes[h, cl])
            run = posting[h, s:s + n].long()
            assert (run[1:] > run[:-1]).all(), "a run is not in position order"
            seen[run] += 1
            assert torch.equal(inverse[h, run], torch.arange(s, s + n, dtype=torch.int32))
        assert (seen == 1).all(), "every position in exactly one cluster"


def _traced_builds(product, codebook_seed, sink=0, **kw):
    """The GPU build with its fit trace, and the oracle's build with its steps."""
    trace = []
    idx = _build_gpu(product, codebook_seed=codebook_seed, fit_trace=trace, sink_tokens=sink, **kw)
    steps = []
    want = ref.build_flat_index(product, codebook_seed=codebook_seed, fit_steps=steps,
                               sink_tokens=sink,
                               **({"min_clusters_log2": kw["flat_min_clusters_log2"]}
                                  if "flat_min_clusters_log2" in kw else {}))
    return idx, trace, want, steps


def _check_trace(product, idx, trace, want, steps, tag):
    """Every k-means step against the oracle (near-ties counted); the layout is exactly the
    oracle's layout of the GPU's own final assignment.  Returns the per-head reports."""
    reps = []
    posting_gpu = idx.posting_positions.cpu()
    for h, (tr, st) in enumerate(zip(trace, steps)):
        sink = int(tr.get("sink", 0))
        # with a sink the fit (and its trace) covers positions sink.. only
        rep = check_fit_trace(product[sink:, h], tr, st["steps"], st["final_assign"],
                              st["final_centroids"], tag=f"{tag} head {h}")
        reps.append(rep)
        # the bucket layout of the GPU's assignment is the oracle's layout of it, bit for bit
        a = tr["partition"]
        if sink:
            assert torch.equal(a[:sink], torch.zeros(sink, dtype=a.dtype))
            assert torch.equal(a[sink:], tr["final_assign"] + 1)
        order = torch.argsort(a, stable=True)
        counts = torch.bincount(a, minlength=idx.num_buckets).to(torch.int32)
        length = a.numel()
        new_order, indptr, inverse = ref.page_align_order(order, counts, torch.arange(length), 16)
        assert torch.equal(idx.bucket_sizes[h].cpu(), counts)
        assert torch.equal(idx.bucket_indptr[h].cpu(), indptr)
        assert torch.equal(posting_gpu[h, :new_order.numel()], new_order.to(torch.int32))
        assert torch.equal(idx.inverse_positions()[h].cpu(), inverse)
    print(f"{tag}: " + "; ".join(f"head {h} {r}" for h, r in enumerate(reps)))
    return reps


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("kmeans_*.pt")))
def test_build_matches_the_reference_golden(name):
    """Against the reference's own build.  The oracle reproduces the goldens bit for bit
    (test_oracle.py), so every GPU step is checked against the oracle fed the GPU's own
    inputs; a key may sit in another cluster than the reference's only downstream of a
    counted near-tie."""
    g = torch.load(GOLDEN / name, weights_only=True)
    length, hkv, d = int(g["length"]), int(g["hkv"]), int(g["d"])
    k_pre = golden_keys(length, hkv, d, int(g["seed"]), mixture=name.endswith("_mix.pt"))
    product = ref.routing_normalize_keys(k_pre)
    sink = int(g["sink"]) if "sink" in g else 0
    idx, trace, want, steps = _traced_builds(product, int(g["codebook_seed"]), sink=sink,
                                             flat_min_clusters_log2=int(g["min_log2"]))
    if sink:
        # cluster 0 holds positions 0..S-1 and nothing else; its descriptor is zero
        assert (idx.bucket_sizes[:, 0].cpu() == sink).all()
        assert torch.count_nonzero(idx.codebooks[:, :, 0].cpu()) == 0
    _check_index_invariants(idx, length)
    assert torch.equal(want["posting"], g["posting"])       # the oracle is the reference here
    reps = _check_trace(product, idx, trace, want, steps, name)
    got = _membership(idx.posting_positions.cpu(), idx.bucket_indptr.cpu(), idx.bucket_sizes.cpu())
    ref_m = _membership(g["posting"], g["indptr"], g["sizes"])
    moved = int((got != ref_m).sum())
    print(f"{name}: {moved} of {got.numel()} keys in another cluster than the reference's")
    if sum(r["origin_flips"] for r in reps) == 0:
        assert moved == sum(r["final_flips"] for r in reps)
    if moved == 0:
        assert torch.equal(idx.posting_positions.cpu(), g["posting"])
        assert torch.equal(idx.bucket_indptr.cpu(), g["indptr"])
        assert torch.equal(idx.inverse_positions().cpu(), g["inverse"])
        cb = (idx.codebooks.cpu().float() - g["codebooks"].float()).abs()
        assert float(cb.max()) <= 2 ** -8


@pytest.mark.parametrize("length,hkv,d,c", [(8192, 2, 128, None), (16384, 4, 256, None),
                                           (32768, 1, 256, 256)])
def test_build_matches_the_oracle_on_mixture_keys(length, hkv, d, c):
    """Mixture keys (the benchmark's key model): every k-means step of every head against
    the oracle, and the final membership against the oracle's own build, with each
    difference traced to a counted near-tie."""
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(length, hkv * 4, hkv, d, mixtures=64, seg=(32, 256), seed=length)
    product = ref.routing_normalize_keys(inp.k)
    kw = {"num_clusters": c} if c else {}
    trace = []
    idx = _build_gpu(product, codebook_seed=5, fit_trace=trace, **kw)
    steps = []
    want = ref.build_flat_index(product, codebook_seed=5, fit_steps=steps, **kw)
    _check_index_invariants(idx, length)
    _check_trace(product, idx, trace, want, steps, f"L={length} Hkv={hkv} D={d}")
    got_m = _membership(idx.posting_positions.cpu(), idx.bucket_indptr.cpu(), idx.bucket_sizes.cpu())
    want_m = _membership(want["posting"], want["indptr"], want["sizes"])
    print(f"L={length} Hkv={hkv} D={d}: {int((got_m != want_m).sum())} of {got_m.numel()} keys "
          f"moved against the oracle's build")


def test_router_pass_equals_building_from_router_output():
    """The product path's build (router_pass: the GPU normalises the pre-RoPE keys itself)
    against the oracle built from the oracle's router output: every router element that
    differs is itself a counted rounding near-tie (check_key_router), every k-means step
    is checked, and the membership equals the build from the CPU router's output unless a
    near-tie was counted."""
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(4096, 8, 2, 128, mixtures=32, seed=9)
    product = ref.routing_normalize_keys(inp.k)
    a = _build_gpu(product, codebook_seed=1)
    trace = []
    b = _build_gpu(inp.k, codebook_seed=1, router_pass=True, fit_trace=trace)
    steps = []
    ref.build_flat_index(product, codebook_seed=1, fit_steps=steps)
    reps = [check_fit_trace(product[:, h], trace[h], steps[h]["steps"], steps[h]["final_assign"],
                            steps[h]["final_centroids"], tag=f"router_pass head {h}", k_pre_h=inp.k[:, h])
            for h in range(2)]
    print("router_pass:", reps)
    ma = _membership(a.posting_positions.cpu(), a.bucket_indptr.cpu(), a.bucket_sizes.cpu())
    mb = _membership(b.posting_positions.cpu(), b.bucket_indptr.cpu(), b.bucket_sizes.cpu())
    for h, r in enumerate(reps):
        if r["origin_flips"] == 0:
            assert int((ma[h] != mb[h]).sum()) <= r["final_flips"] + r["router_rows"], r


@pytest.mark.parametrize("length,d", [(131072, 256), (524288, 256), (8192, 128)])
def test_key_router_matches_the_oracle_element_by_element(length, d):
    """sbsa_key_space with the router pass, at the benchmarks' prompt lengths, against
    the oracle's router (routing_map.py:52-59) and routing space (flat_index.py:165-166):
    each router element that differs is a rounding near-tie of its own exact quotient."""
    from semblo_amd import _lib
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(length, 4, 1, d, mixtures=64, seg=(32, 256), sinks=4, seed=length + d,
                        num_queries=1)
    k = inp.k[:, 0]
    kd = k.to(DEV).contiguous()
    s32 = torch.empty(length, d, dtype=torch.float32, device=DEV)
    s16 = torch.empty(length, d, dtype=torch.bfloat16, device=DEV)
    _lib.call("sbsa_key_space", _lib.ptr(kd), length, kd.stride(0), d, 1, _lib.ptr(s32),
              _lib.ptr(s16), _lib.stream(kd.device))
    torch.cuda.synchronize()
    from gpu_util import check_key_router
    rep = check_key_router(k, s32, s16, f"L={length} D={d}")
    print(f"key router L={length} D={d}: {rep} of {k.numel()} elements")


def test_pack_gathers_through_the_posting_list():
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(2048, 8, 2, 128, mixtures=16, seed=4)
    idx = _build_gpu(ref.routing_normalize_keys(inp.k), codebook_seed=0)
    k, v = inp.k.to(DEV), inp.v.to(DEV)
    packed = idx.pack_prompt_kv(k, v).cpu()
    want = ref.pack_prompt_kv(idx.posting_positions.cpu(), inp.k, inp.v)
    assert torch.equal(packed, want)


def test_causal_sizes_match_the_snapshot_rule():
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(4096, 8, 2, 128, mixtures=16, seed=2)
    idx = _build_gpu(ref.routing_normalize_keys(inp.k), codebook_seed=0)
    for limit in (0, 1, 777, 2048, 4095, 4096):
        got = idx.causal_sizes(limit).cpu()
        want = ref.causal_sizes_at(idx.posting_positions.cpu(), idx.bucket_indptr.cpu(),
                                   idx.bucket_sizes.cpu(), limit)
        assert torch.equal(got, want)


def test_build_with_empty_clusters_matches_the_oracle():
    """Heads 0 and 2 draw their keys from a few directions, so k-means leaves
    clusters empty and restarts them on sample rows drawn from the generator;
    head 1 is ordinary.  The restart draws, and the draws of every later head,
    must follow the reference's order (flat_index.py:277-283)."""
    gen = torch.Generator().manual_seed(23)
    length, d = 2048, 128
    k = torch.randn(length, 3, d, generator=gen)
    for h in (0, 2):
        dirs = torch.randn(6, d, generator=gen)
        k[:, h] = dirs[torch.randint(0, 6, (length,), generator=gen)] \
            + 1e-3 * torch.randn(length, d, generator=gen)
    product = ref.routing_normalize_keys(k.to(torch.bfloat16))
    traces, steps, trace = [], [], []
    want = ref.build_flat_index(product, codebook_seed=5, traces=traces, fit_steps=steps)
    empties = [sum(len(x[1]) for x in tr if x[0] == "empty") for tr in traces]
    assert empties[0] > 0 and empties[1] == 0 and empties[2] > 0, empties
    # more empty iterations than the GPU restarts ahead (RESTARTS_AHEAD = 2): the
    # iterations past those are restarted on the host and redone
    from semblo_amd.state import RESTARTS_AHEAD
    empty_iters = [sum(1 for x in tr if x[0] == "empty" and len(x[1]) > 0) for tr in traces]
    assert empty_iters[0] > RESTARTS_AHEAD and empty_iters[2] > RESTARTS_AHEAD, empty_iters
    idx = _build_gpu(product, codebook_seed=5, fit_trace=trace)
    _check_index_invariants(idx, length)
    reps = _check_trace(product, idx, trace, want, steps, "restarts")
    gpu_empties = [int((tr["counts"] == 0).sum()) for tr in trace]
    print(f"restart draws per head {empties}, GPU empty clusters per head {gpu_empties}")
    if all(r["origin_flips"] == 0 for r in reps):
        assert gpu_empties == empties
        assert torch.equal(idx.posting_positions.cpu(), want["posting"])


@pytest.mark.parametrize("dim", [256, 320])
def test_update_sums_and_counts_each_cluster(dim):
    """The centroid sums through the C-ABI on a skewed assignment: cluster 0 holds
    most rows (more than the kernel lists at once, so it is summed in windows),
    cluster 5 none, the row count is ragged and the rows are read through a row map.
    Counts exact; each sum within fp32 summation-order error of the fp64 sum of its
    rows (the bound the fit's trace check uses); a second call on stale scratch gives
    the same bits."""
    from semblo_amd import _lib
    gen = torch.Generator().manual_seed(11)
    # ragged (not a multiple of 512 rows), two segments of 32768 rows, cluster 0 past the
    # kernel's 8192-entry member list within one segment
    rows, n, c = 48000, 40000 + 37, 64
    x = torch.randn(rows, dim, generator=gen)
    row_index = torch.randperm(rows, generator=gen)[:n].to(torch.int32)
    assign = torch.randint(1, c, (n,), generator=gen, dtype=torch.int32)
    assign[torch.rand(n, generator=gen) < 0.7] = 0
    assign[assign == 5] = 6
    xd, rd, ad = x.to(DEV), row_index.to(DEV), assign.to(DEV)
    sums = torch.full((c, dim), float("nan"), device=DEV)
    counts = torch.full((c,), -1, dtype=torch.int32, device=DEV)
    nbytes = _lib.query("sbsa_kmeans_member_bits_bytes", n, c)
    bits = torch.full((nbytes // 4,), -1, dtype=torch.int32, device=DEV)    # stale contents
    _lib.call("sbsa_kmeans_update", _lib.ptr(xd), dim, _lib.ptr(rd), n, _lib.ptr(ad), c, dim,
              _lib.ptr(sums), _lib.ptr(counts), _lib.ptr(bits), nbytes, _lib.stream(xd.device))
    torch.cuda.synchronize()
    first = sums.clone()
    _lib.call("sbsa_kmeans_update", _lib.ptr(xd), dim, _lib.ptr(rd), n, _lib.ptr(ad), c, dim,
              _lib.ptr(sums), _lib.ptr(counts), _lib.ptr(bits), nbytes, _lib.stream(xd.device))
    torch.cuda.synchronize()
    assert torch.equal(sums, first)
    want = torch.zeros(c, dim, dtype=torch.float64).index_add_(0, assign.long(),
                                                               x[row_index.long()].double())
    cnt = torch.bincount(assign.long(), minlength=c)
    assert int(cnt[:1]) > 2 * 8192 and int(cnt[5]) == 0
    assert torch.equal(counts.cpu(), cnt.to(torch.int32))
    scale = cnt.clamp_min(1).double()[:, None]
    assert float(((sums.cpu().double() - want).abs() / scale).max()) <= 1e-5
    assert torch.count_nonzero(sums[5]) == 0
