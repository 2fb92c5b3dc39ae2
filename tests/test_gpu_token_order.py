"""S10 on the GPU: the token-order streamed prefill's store and its attention.

The kernels are checked against the oracle (oracle/reference_cpu.py, S10):
  nearest_cluster  ids equal the oracle's except near-ties (fp32 similarity of
                   the two clusters within 1e-4 relative), counted;
  append_rows      rows and counts bit-exact, overflow flags exact;
  store            a replay of the whole session in the oracle -- reserved
                   layout, relayout of the fitted runs (the S1 build's own
                   output), every slice's append with the GPU's ids, repacks --
                   gives the same
                   indptr, sizes, posting, inverse and packed rows, bit for bit;
  attention        every slice against fp64 over its key set: exact causal
                   before the fit and within the dense prefix, otherwise the
                   selected clusters' rows appended by earlier slices plus the
                   slice's own causal window.  Tolerance 2e-2 abs + 1e-2 rel.
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import (assert_close_bf16, attention_reference, check_recorded_chunk,
                      cluster_position_mask, oracle_select)
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
NEAR_REL = 1e-4


def _ids_near_ties(keys_h, codebooks_h, got, want):
    """Every key whose GPU cluster differs must be an fp32 near-tie in the oracle."""
    _, sim = ref.nearest_cluster(keys_h, codebooks_h, return_sim=True)
    moved = torch.nonzero(got.long() != want.long()).flatten()
    for i in moved.tolist():
        a, b = float(sim[i, want[i]]), float(sim[i, got[i]])
        assert abs(a - b) <= NEAR_REL * max(abs(a), 1e-6), (i, a, b)
    return int(moved.numel())


@pytest.mark.parametrize("cfg", [dict(n=3001, hkv=2, d=128, c=128, seed=1),
                                 dict(n=8192, hkv=4, d=256, c=256, seed=2),
                                 dict(n=37, hkv=4, d=256, c=1024, seed=3)])
def test_nearest_cluster_matches_the_oracle(cfg):
    from semblo_amd.state import ProductPostingIndex
    from semblo_amd.synthetic import mixture_layer
    from semblo_amd.token_outer_prefill import nearest_cluster
    n, hkv, d, c = cfg["n"], cfg["hkv"], cfg["d"], cfg["c"]
    inp = mixture_layer(max(n, 2 * c) + 512, 2 * hkv, hkv, d, mixtures=48, seed=cfg["seed"])
    head = inp.k[:2 * c + 512].to(DEV)
    idx = ProductPostingIndex.build(head, torch.arange(head.shape[0], device=DEV), router_pass=True,
                                    num_clusters=c, codebook_seed=cfg["seed"])
    cb = idx.codebooks.clone()
    cb[:, :, 5] = 0                                        # a dead cluster on every head
    keys = inp.k[-n:]
    ids = nearest_cluster(keys.to(DEV), cb).cpu()
    moved = 0
    for h in range(hkv):
        want = ref.nearest_cluster(keys[:, h], cb[h].cpu())
        moved += _ids_near_ties(keys[:, h], cb[h].cpu(), ids[h], want)
        assert not bool((ids[h] == 5).any())
    print(f"{cfg}: {moved} near-tie assignments of {n * hkv}")


@pytest.mark.parametrize("n,c", [(8192, 256), (1, 128), (63, 64), (5000, 1024), (0, 128)])
def test_append_rows_bit_exact(n, c):
    from semblo_amd.token_outer_prefill import append_rows
    gen = torch.Generator().manual_seed(n + c)
    hkv = 3
    # runs of equal ids, as segments of a prompt produce
    ids = torch.randint(0, c, (hkv, max(n, 1)), generator=gen)[:, :n]
    if n > 8:
        ids[:, n // 3:n // 2] = 7
    sizes = torch.randint(0, 40, (hkv, c), generator=gen, dtype=torch.int32)
    reserve = (sizes + torch.randint(0, 40, (hkv, c), generator=gen, dtype=torch.int32)).to(torch.int64)
    reserve = (reserve + 15) // 16 * 16
    indptr = torch.zeros(hkv, c + 1, dtype=torch.int32)
    indptr[:, 1:] = torch.cumsum(reserve, 1).to(torch.int32)
    rows, counts, flags = append_rows(ids.to(torch.int32).to(DEV), indptr.to(DEV), sizes.to(DEV),
                                      reserve.to(DEV))
    want_rows, want_counts = ref.append_rows(ids, indptr, sizes)
    assert torch.equal(rows.cpu().long(), want_rows)
    assert torch.equal(counts.cpu().long(), want_counts)
    want_flag = (sizes.long() + want_counts > reserve).any(1).to(torch.int32)
    assert torch.equal(flags.cpu(), want_flag)


def test_append_rows_flags_an_id_out_of_range():
    from semblo_amd.token_outer_prefill import append_rows
    ids = torch.tensor([[0, 1, 64, 1]], dtype=torch.int32, device=DEV)
    indptr = torch.arange(0, 65 * 16, 16, dtype=torch.int32, device=DEV)[None]
    sizes = torch.zeros(1, 64, dtype=torch.int32, device=DEV)
    rows, counts, flags = append_rows(ids, indptr, sizes)
    assert int(flags[0]) & 2
    assert rows.cpu().tolist() == [[0, 16, -1, 17]]


def _oracle_store(inp, tokens, chunk, fit_at, c, seed, ids_by_slice, align=16):
    """The session replayed on the CPU: reserved layout, relayout, appends, repacks.

    The fit itself is the S1 build, pinned against the oracle (up to bf16
    near-ties of the membership) by test_gpu_kmeans.py; the replay starts from
    the GPU build of the same staged keys, which is deterministic."""
    from semblo_amd.state import ProductPostingIndex
    k = inp.k
    hkv, d = k.shape[1], k.shape[2]
    gb = ProductPostingIndex.build(k[:fit_at].to(DEV), torch.arange(fit_at, device=DEV),
                                   codebook_seed=seed, router_pass=True, num_clusters=c,
                                   page_align=align)
    built = dict(codebooks=gb.codebooks.cpu(), sizes=gb.bucket_sizes.cpu(),
                 inverse=gb.inverse_positions().cpu(), indptr=gb.bucket_indptr.cpu())
    width = tokens + c * align
    width += (-width) % 256
    reserve = ref.reserved_layout(built["sizes"], fit_at, tokens, width, align)
    indptr = torch.zeros(hkv, c + 1, dtype=torch.int64)
    indptr[:, 1:] = torch.cumsum(reserve, 1)
    rows = ref.relayout_rows(built["inverse"], built["indptr"], indptr)      # [Hkv, fit_at]
    inverse = torch.zeros(hkv, tokens, dtype=torch.int64)
    inverse[:, :fit_at] = rows
    inverse_fit = inverse.clone()
    sizes = built["sizes"].to(torch.int64).clone()
    before, repacks, trail, with_slice = [], 0, [], 0
    for start in range(fit_at, tokens, chunk):
        stop = min(tokens, start + chunk)
        ids = ids_by_slice[start].long()
        r, counts = ref.append_rows(ids, indptr, sizes)
        if bool((sizes + counts > reserve).any()):
            # the reference's layout from the counts before the slice; if the slice would
            # still not fit, the layout with its keys counted instead
            reserve = ref.reserved_layout(sizes, start, tokens, width, align)
            if bool((sizes + counts > reserve).any()):
                reserve = ref.reserved_layout(sizes + counts, stop, tokens, width, align)
                with_slice += 1
            new_ip = torch.zeros_like(indptr)
            new_ip[:, 1:] = torch.cumsum(reserve, 1)
            inverse[:, :start] = ref.relayout_rows(inverse[:, :start], indptr, new_ip)
            indptr = new_ip
            repacks += 1
            r, counts = ref.append_rows(ids, indptr, sizes)
            assert not bool((sizes + counts > reserve).any())
        inverse[:, start:stop] = r
        trail.append(inverse.clone())
        before.append(sizes.clone())
        sizes = sizes + counts
    return dict(codebooks=built["codebooks"], indptr=indptr, sizes=sizes, inverse=inverse,
                before=before, repacks=repacks, with_slice=with_slice, width=width, trail=trail,
                fitted=inverse_fit)


def _first_divergence(trail, exp, fit_at, chunk):
    """Name the first appended slice after which the GPU's inverse map differs from the replay."""
    for i, (got, want) in enumerate(zip(trail, exp["trail"])):
        if not torch.equal(got, want):
            bad = torch.nonzero(got != want)
            h, p = bad[0].tolist()
            fit_bad = int((got[:, :fit_at] != exp["fitted"][:, :fit_at]).sum()) if i == 0 else -1
            raise AssertionError(
                f"inverse differs after the slice at {fit_at + i * chunk}: {bad.shape[0]} entries, "
                f"first (head {h}, position {p}) got {int(got[h, p])} want {int(want[h, p])}; "
                f"positions {bad[:, 1].min().item()}..{bad[:, 1].max().item()}; fitted part off: {fit_bad}")


def _run_session(cfg, k_override=None):
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    from semblo_amd.synthetic import mixture_layer
    from semblo_amd.token_outer_prefill import nearest_cluster
    tokens, hq, hkv, d, chunk = cfg["tokens"], cfg["hq"], cfg["hkv"], cfg["d"], cfg["chunk"]
    rc = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=chunk,
                             codebook_seed=cfg["seed"], layer_idx=0)
    layer = SembloAttention(rc, layer_name=f"test.token_order.{cfg['seed']}")
    layer.plan_log = []
    inp = mixture_layer(tokens, hq, hkv, d, mixtures=32, seg=(32, 256), seed=cfg["seed"])
    if k_override is not None:
        k_override(inp)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    session = layer.begin_token_outer_prefill(tokens, chunk, fit_tokens=cfg["fit_tokens"])
    out = torch.empty(tokens, hq, d, dtype=torch.bfloat16, device=DEV)
    ids_by_slice, before, dense = {}, {}, {}
    trail = []
    for start in range(0, tokens, chunk):
        stop = min(tokens, start + chunk)
        appended = session.index is not None or start >= session.fit_at
        session.slice_projected(q[start:stop], q[start:stop], k[start:stop], k[start:stop], v[start:stop],
                                start, stop, out=out[start:stop])
        if appended:
            # the ids the session appended with (same kernel, same input)
            ids_by_slice[start] = nearest_cluster(k[start:stop], session.index.codebooks).cpu()
            before[start] = session.snapshot.sizes.cpu().clone()
            trail.append(session.index.inverse_positions().cpu().long().clone())
        dense[start] = session.index is None or start <= session.cap
    index = session.finish()
    torch.cuda.synchronize()
    _run_session.trail = trail
    return layer, session, index, inp, out.cpu(), ids_by_slice, before, dense


@pytest.mark.parametrize("cfg", [
    dict(tokens=4096, hq=8, hkv=2, d=128, chunk=512, fit_tokens=512, seed=11),
    dict(tokens=6000, hq=16, hkv=4, d=256, chunk=1024, fit_tokens=1024, seed=12),   # ragged end
])
def test_token_order_session_store_and_attention(cfg):
    layer, session, index, inp, out, ids_by_slice, before, dense = _run_session(cfg)
    tokens, hkv, d = cfg["tokens"], cfg["hkv"], cfg["d"]
    c = index.num_buckets
    fit_at = session.fit_at
    # the ids the session used against the oracle's assignment
    moved = 0
    for start, ids in ids_by_slice.items():
        stop = min(tokens, start + cfg["chunk"])
        for h in range(hkv):
            want = ref.nearest_cluster(inp.k[start:stop, h], index.codebooks[h].cpu())
            moved += _ids_near_ties(inp.k[start:stop, h], index.codebooks[h].cpu(), ids[h], want)
    exp = _oracle_store(inp, tokens, cfg["chunk"], fit_at, c, cfg["seed"], ids_by_slice)
    assert torch.equal(index.codebooks.cpu(), exp["codebooks"])
    assert torch.equal(index.bucket_indptr.cpu().long(), exp["indptr"])
    assert torch.equal(index.bucket_sizes.cpu().long(), exp["sizes"])
    inv = index.inverse_positions().cpu().long()
    _first_divergence(_run_session.trail, exp, fit_at, cfg["chunk"])
    assert torch.equal(inv, exp["inverse"])
    assert session.repacks == exp["repacks"]
    assert session.repacks_with_slice == exp["with_slice"]
    for i, start in enumerate(sorted(before)):
        assert torch.equal(before[start].long(), exp["before"][i])
    posting = index.posting_positions.cpu().long()
    packed = index.packed_kv.cpu()
    for h in range(hkv):
        assert torch.equal(posting[h, inv[h]], torch.arange(tokens))
        assert torch.equal(packed[0, inv[h], h], inp.k[:, h])
        assert torch.equal(packed[1, inv[h], h], inp.v[:, h])
        # every key lies inside its cluster's run, runs in position order
        for cl in range(c):
            s, n = int(index.bucket_indptr[h, cl]), int(index.bucket_sizes[h, cl])
            assert n <= int(index.bucket_indptr[h, cl + 1]) - s
            assert bool((posting[h, s + 1:s + n] > posting[h, s:s + n - 1]).all())
    # attention, slice by slice
    target = session.target
    sm = d ** -0.5
    recs = {r["chunk_start"]: r for r in layer.plan_log}
    near_ties = 0
    for start in range(0, tokens, cfg["chunk"]):
        stop = min(tokens, start + cfg["chunk"])
        p = torch.arange(start, stop)
        if dense[start]:
            keys = (torch.arange(tokens)[None, :] <= p[:, None])[:, None, :].expand(-1, hkv, -1)
            want = attention_reference(inp.q[start:stop], keys, inp.k, inp.v, sm)
            assert_close_bf16(out[start:stop], want, f"dense slice {start}")
            continue
        rec = recs[start]
        assert torch.equal(rec["causal_sizes"].cpu(), before[start])
        rep = check_recorded_chunk(rec, inp.q, inp.q, inp.k, inp.v, index, out, target=target,
                                   tag="token order")
        near_ties += rep["near_ties"]
    print(f"{cfg}: fit at {fit_at}, {len(ids_by_slice)} appended slices, {moved} near-tie ids, "
          f"{session.repacks} repacks ({session.repacks_with_slice} counting the slice), {near_ties} near-tie selection "
          f"differences against the oracle")
    assert layer.arena is not None and layer.arena.prompt_length == tokens


def test_token_order_repacks_when_a_cluster_outgrows_its_reservation():
    cfg = dict(tokens=4096, hq=8, hkv=2, d=128, chunk=512, fit_tokens=512, seed=21)

    def crowd(inp):
        # after the fit point every key lies near one key of the head: one cluster takes them all
        gen = torch.Generator().manual_seed(3)
        base = inp.k[100].float()
        tail = base[None] + 0.05 * torch.randn(4096 - 1024, *base.shape, generator=gen)
        inp.k[1024:] = tail.to(inp.k.dtype)

    layer, session, index, inp, out, ids_by_slice, before, dense = _run_session(cfg, crowd)
    assert session.repacks >= 1
    c = index.num_buckets
    exp = _oracle_store(inp, cfg["tokens"], cfg["chunk"], session.fit_at, c, cfg["seed"], ids_by_slice)
    assert session.repacks == exp["repacks"]
    assert session.repacks_with_slice == exp["with_slice"]
    assert torch.equal(index.bucket_indptr.cpu().long(), exp["indptr"])
    inv = index.inverse_positions().cpu().long()
    assert torch.equal(inv, exp["inverse"])
    packed = index.packed_kv.cpu()
    posting = index.posting_positions.cpu().long()
    for h in range(cfg["hkv"]):
        assert torch.equal(packed[0, inv[h], h], inp.k[:, h])
        assert torch.equal(packed[1, inv[h], h], inp.v[:, h])
        assert torch.equal(posting[h, inv[h]], torch.arange(cfg["tokens"]))
    print(f"repacks: {session.repacks} ({session.repacks_with_slice} counting the slice)")


def test_decode_after_a_token_order_prefill():
    """The finished store serves the decode step: steps against fp64 over the GPU's
    selected clusters' rows (the layout has gaps between runs) plus the suffix, and the
    GPU's selection against the oracle's up to near-ties."""
    from gpu_util import compare_selection
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.synthetic import decode_queries
    from test_gpu_decode import _csr_to_sel
    cfg = dict(tokens=4096, hq=8, hkv=2, d=128, chunk=512, fit_tokens=512, seed=31)
    layer, session, index, inp, out, *_ = _run_session(cfg)
    qs, kn, vn = decode_queries(inp, 3, cfg["hq"], seed=5)
    hq, hkv, d = cfg["hq"], cfg["hkv"], cfg["d"]
    c = index.num_buckets
    res = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    csr = torch.empty(3 * hkv * c + 2 * hkv, dtype=torch.int32, device=DEV)
    packed = index.packed_kv.cpu()
    rc = layer.runtime_config
    for t in range(3):
        pos = torch.tensor([cfg["tokens"] + t], dtype=torch.int32, device=DEV)
        q = qs[t:t + 1].to(DEV)
        fused_decode_step(layer, layer.arena, q_post=q, q_pre=q, positions=pos,
                          k_post=kn[t:t + 1].to(DEV), v_states=vn[t:t + 1].to(DEV), output=res,
                          temperature=rc.selection_temperature, beta=rc.bucket_size_penalty,
                          target_tokens=session.target, sm_scale=d ** -0.5,
                          num_splits=rc.decode_num_splits, iters=rc.iters, csr_out=csr)
        torch.cuda.synchronize()
        sel = _csr_to_sel(csr.cpu(), index)
        vec = ref.trivial_router_vectors(q.cpu(), 1)
        exp = oracle_select(vec, index.codebooks.cpu(), index.bucket_sizes.cpu()[None],
                            temperature=0.1, beta=0.25, target=session.target)
        compare_selection(sel[None], exp["sel"], exp["score"], exp["theta"])
        want = ref.decode_reference(q[0].cpu(), packed, index.bucket_indptr.cpu(),
                                    index.bucket_sizes.cpu(), sel, kn[:t + 1].cpu(), vn[:t + 1].cpu(),
                                    d ** -0.5)
        assert_close_bf16(res.view(hq, d).cpu(), want, f"decode step {t}")
