"""S3c/S4/S5/S6 on the GPU: the KV-outer sparse prefill and the dense-prefix chunks.

The attention is checked against an fp64 softmax over exactly the key set the
reference defines for a query at position p in KV group h
(kv_outer.py:482-816): the first causal_sizes[h, c] rows of every cluster c
the query selected, plus positions wstart..p -- with the GPU's own selection,
which is itself checked against the oracle's up to near-ties.  Tolerance:
2e-2 abs + 1e-2 rel (bf16).
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import (assert_close_bf16, attention_reference, check_recorded_chunk,
                      cluster_position_mask, compare_selection, oracle_select)
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(length, hq, hkv, d, seed, mixtures=32):
    from semblo_amd.state import ProductPostingIndex
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(length, hq, hkv, d, mixtures=mixtures, seg=(32, 256), seed=seed)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    idx = ProductPostingIndex.build(k, torch.arange(length, device=DEV), codebook_seed=seed,
                                    router_pass=True)
    idx.pack_prompt_kv(k, v)
    idx.original_kv = (k, v)
    return inp, q, k, v, idx


def _run_sparse_chunk(idx, q, k, v, cs, ce, target, *, tau=0.1, beta=0.25):
    from semblo_amd.kv_outer import kv_outer_attention
    from semblo_amd.fused_select import theta_select_bitmask_flat
    from semblo_amd.trivial_router import trivial_router_vectors
    hkv, c = idx.bucket_sizes.shape
    qc = q[cs:ce + 1]
    qn, hq, d = qc.shape
    sizes = idx.causal_sizes(cs)
    vec = trivial_router_vectors(qc, 1)
    qmask = torch.empty(qn, hkv, c // 32, dtype=torch.int32, device=DEV)
    theta = torch.empty(qn, hkv, dtype=torch.float32, device=DEV)
    theta_select_bitmask_flat(vec.view(qn, hq, 1, d), None, idx.codebooks, sizes[None], None,
                              temperature=tau, beta=beta, target_tokens=target, g_union=32,
                              qmask=qmask, theta_out=theta)
    out, stats = kv_outer_attention(qc, idx.packed_kv, qmask, sizes, idx.bucket_indptr,
                                    sm_scale=d ** -0.5, local_kv=(k[cs:ce + 1], v[cs:ce + 1]),
                                    chunk_start=cs, wstart=cs)
    torch.cuda.synchronize()
    return out.cpu(), qmask.cpu(), sizes.cpu(), vec.cpu(), theta.cpu()


def _reference_sparse(idx, q, k, v, cs, ce, qmask, sizes):
    hkv, c = sizes.shape
    length = k.shape[0]
    sel = ref.unpack_bits(qmask, c)                                   # [Qc, Hkv, C]
    pos = cluster_position_mask(idx.posting_positions.cpu(), idx.bucket_indptr.cpu(), sizes, length)
    keys = torch.einsum("qhc,hcl->qhl", sel.double(), pos.double()) > 0
    p = torch.arange(cs, ce + 1)
    win = (torch.arange(length)[None, :] >= cs) & (torch.arange(length)[None, :] <= p[:, None])
    keys |= win[:, None, :]
    return attention_reference(q[cs:ce + 1].cpu(), keys, k.cpu(), v.cpu(), q.shape[-1] ** -0.5)


@pytest.mark.parametrize("cfg", [
    dict(length=4096, hq=8, hkv=2, d=128, cs=2048, ce=3071, seed=1),
    dict(length=2048, hq=16, hkv=4, d=256, cs=1024, ce=1535, seed=2),
    dict(length=4096, hq=16, hkv=4, d=256, cs=3000, ce=3299, seed=3),     # ragged chunk
    dict(length=3000, hq=4, hkv=4, d=128, cs=1900, ce=2999, seed=4),      # G = 1, odd length
    dict(length=3072, hq=16, hkv=2, d=128, cs=2048, ce=3071, seed=5),     # G = 8
    dict(length=2048, hq=8, hkv=4, d=256, cs=1024, ce=1700, seed=6),      # G = 2, D = 256
])
def test_sparse_chunk_matches_fp64_over_the_selected_set(cfg):
    inp, q, k, v, idx = _setup(cfg["length"], cfg["hq"], cfg["hkv"], cfg["d"], cfg["seed"])
    target = cfg["length"] // 16
    cs, ce = cfg["cs"], cfg["ce"]
    out, qmask, sizes, vec, theta = _run_sparse_chunk(idx, q, k, v, cs, ce, target)
    want = _reference_sparse(idx, q, k, v, cs, ce, qmask, sizes)
    err = assert_close_bf16(out, want, f"sparse chunk {cfg}")
    # the GPU's selection against the oracle's on the same index
    exp = oracle_select(vec, idx.codebooks.cpu(), sizes[None], temperature=0.1, beta=0.25,
                        target=target)
    rep = compare_selection(ref.unpack_bits(qmask, sizes.shape[1]), exp["sel"], exp["score"],
                            exp["theta"], theta)
    print(f"{cfg}: max err {err:.3g}, selection {rep}")


@pytest.mark.parametrize("cfg", [dict(hq=16, hkv=4, d=256, grid=8), dict(hq=8, hkv=2, d=128, grid=0)])
def test_sparse_chunk_redone_when_keys_tower_over_the_first_tile(cfg):
    """Sparse chunk (the pipelined kernel form): the index is built on ordinary keys,
    the attention reads keys of which every 97th lies far along the queries' common
    direction, so items whose cluster run (or window) holds one past its first tile
    pass 2^64 and are redone with the rows' true maxima.  On a grid of 8 blocks each
    block works through many items, with the next item's query slots and Q rows
    staged during the current one.  Exact attention over the selected set."""
    from semblo_amd.kv_outer import kv_outer_attention
    from semblo_amd.fused_select import theta_select_bitmask_flat
    from semblo_amd.state import ProductPostingIndex
    from semblo_amd.trivial_router import trivial_router_vectors
    gen = torch.Generator().manual_seed(23)
    length, hq, hkv, d = 4096, cfg["hq"], cfg["hkv"], cfg["d"]
    cs, ce = 2048, 3071
    u = torch.randn(d, generator=gen)
    q = (3 * u + torch.randn(length, hq, d, generator=gen)).to(torch.bfloat16)
    k = torch.randn(length, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(length, hkv, d, generator=gen).to(torch.bfloat16)
    k_att = k.clone()
    k_att[97::97] = (3.0 * u).to(torch.bfloat16)
    qd, kd, kad, vd = q.to(DEV), k.to(DEV), k_att.to(DEV), v.to(DEV)
    idx = ProductPostingIndex.build(kd, torch.arange(length, device=DEV), codebook_seed=5,
                                    router_pass=True)
    idx.pack_prompt_kv(kad, vd)
    c = idx.bucket_sizes.shape[1]
    qc = qd[cs:ce + 1]
    qn = qc.shape[0]
    sizes = idx.causal_sizes(cs)
    vec = trivial_router_vectors(qc, 1)
    qmask = torch.empty(qn, hkv, c // 32, dtype=torch.int32, device=DEV)
    theta_select_bitmask_flat(vec.view(qn, hq, 1, d), None, idx.codebooks, sizes[None], None,
                              temperature=0.1, beta=0.25, target_tokens=length // 16, g_union=32,
                              qmask=qmask)
    out, _ = kv_outer_attention(qc, idx.packed_kv, qmask, sizes, idx.bucket_indptr,
                                sm_scale=d ** -0.5, local_kv=(kad[cs:ce + 1], vd[cs:ce + 1]),
                                chunk_start=cs, wstart=cs, grid=cfg["grid"] or None)
    torch.cuda.synchronize()
    want = _reference_sparse(idx, q, k_att, v, cs, ce, qmask.cpu(), sizes.cpu())
    err = assert_close_bf16(out.cpu(), want, f"towering keys, sparse chunk {cfg}")
    print(f"{cfg}: max err {err:.3g}")


@pytest.mark.parametrize("cfg", [dict(length=2048, hq=8, hkv=2, d=128, cs=0, ce=1023),
                                 dict(length=2048, hq=16, hkv=4, d=256, cs=512, ce=1300),
                                 dict(length=2048, hq=8, hkv=1, d=128, cs=1024, ce=1535),   # G = 8
                                 dict(length=1536, hq=4, hkv=4, d=256, cs=700, ce=1300)])   # G = 1
def test_dense_prefix_chunk_is_exact_causal_attention(cfg):
    from semblo_amd.kv_outer import dense_causal_attention
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(cfg["length"], cfg["hq"], cfg["hkv"], cfg["d"], mixtures=8, seed=7)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    cs, ce = cfg["cs"], cfg["ce"]
    out = dense_causal_attention(q[cs:ce + 1], k, v, sm_scale=cfg["d"] ** -0.5, chunk_start=cs).cpu()
    p = torch.arange(cs, ce + 1)
    keys = (torch.arange(cfg["length"])[None, :] <= p[:, None])[:, None, :].expand(-1, cfg["hkv"], -1)
    want = attention_reference(inp.q[cs:ce + 1], keys, inp.k, inp.v, cfg["d"] ** -0.5)
    err = assert_close_bf16(out, want, f"dense chunk {cfg}")
    print(f"dense {cfg}: max err {err:.3g}")


def test_layer_prefill_chunk_loop_through_the_operator():
    """The whole-prompt path behind semblo::attention: build, pack, the chunk loop with
    dense and sparse chunks.  Dense chunks against fp64 causal attention; each sparse
    chunk against fp64 over the GPU's own key sets (recorded plans), with no query off
    tolerance, and its selection against the oracle's up to counted near-ties."""
    from semblo_amd.attention_op import sparse_attention_op
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    from semblo_amd.synthetic import mixture_layer
    length, hq, hkv, d = 4096, 8, 2, 128
    cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=512,
                              codebook_seed=3, layer_idx=0)
    layer = SembloAttention(cfg, layer_name="test.prefill.0")
    layer.plan_log = []
    inp = mixture_layer(length, hq, hkv, d, mixtures=32, seed=11)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    positions = torch.arange(length, device=DEV)
    out = torch.empty(length, hq * d, dtype=torch.bfloat16, device=DEV)
    sparse_attention_op(positions, q.view(length, -1), q.view(length, -1), k, v, q, k, out,
                        "test.prefill.0")
    torch.cuda.synchronize()
    got = out.view(length, hq, d).cpu()
    idx = layer.index
    target = length // 16
    sparse_starts = [r["chunk_start"] for r in layer.plan_log]
    assert sparse_starts == [cs for cs in range(0, length, 512) if cs > 4 * target]
    for cs in range(0, 4 * target + 1, 512):
        ce = cs + 511
        p = torch.arange(cs, ce + 1)
        keys = (torch.arange(length)[None, :] <= p[:, None])[:, None, :].expand(-1, hkv, -1)
        want = attention_reference(inp.q[cs:ce + 1], keys, inp.k, inp.v, d ** -0.5)
        assert_close_bf16(got[cs:ce + 1], want, f"dense chunk {cs}")
    for rec in layer.plan_log:
        rep = check_recorded_chunk(rec, inp.q, inp.q, inp.k, inp.v, idx, got, target=target,
                                   tag="operator")
        print(f"chunk {rec['chunk_start']}: {rep}")


@pytest.mark.parametrize("beta", [3.0, 6.0])
def test_dense_chunk_redone_when_a_key_towers_over_the_first_tile(beta):
    """A key far above every score of the first tile: probabilities against the
    first tile's maximum pass 2^64 (beta 3: about 2^90) or fp32 range (beta 6), the
    item is redone with the rows' true maxima, and the result is exact attention."""
    from semblo_amd.kv_outer import dense_causal_attention
    gen = torch.Generator().manual_seed(17)
    length, hq, hkv, d = 2048, 8, 2, 128
    cs, ce = 1024, 1535
    u = torch.randn(d, generator=gen)
    q = (3 * u + torch.randn(length, hq, d, generator=gen)).to(torch.bfloat16)
    k = torch.randn(length, hkv, d, generator=gen)
    v = torch.randn(length, hkv, d, generator=gen).to(torch.bfloat16)
    k[900] = beta * u                                      # tile 28 of the keys, every query sees it
    k = k.to(torch.bfloat16)
    out = dense_causal_attention(q[cs:ce + 1].to(DEV), k.to(DEV), v.to(DEV), sm_scale=d ** -0.5,
                                 chunk_start=cs).cpu()
    p = torch.arange(cs, ce + 1)
    keys = (torch.arange(length)[None, :] <= p[:, None])[:, None, :].expand(-1, hkv, -1)
    want = attention_reference(q[cs:ce + 1], keys, k, v, d ** -0.5)
    err = assert_close_bf16(out, want, f"towering key, beta {beta}")
    print(f"beta {beta}: max err {err:.3g}")


def test_layer_prefill_is_bit_identical_across_reruns():
    """The work items are claimed in whatever order the blocks reach the queue,
    and every item writes its own partial rows: the same prompt must give the
    same bits on every run.  A missing barrier between an item's last tile and
    the next item's loads showed up here as one wave's rows differing in about
    one run in sixteen, so the layer is run 24 times."""
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    from semblo_amd.synthetic import mixture_layer
    length, hq, hkv, d = 4096, 8, 2, 128
    inp = mixture_layer(length, hq, hkv, d, mixtures=32, seed=11)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    outs = []
    for i in range(24):
        cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=512,
                                  codebook_seed=3, layer_idx=0)
        layer = SembloAttention(cfg, layer_name=f"rerun.{i}")
        out = torch.empty(length, hq * d, dtype=torch.bfloat16, device=DEV)
        layer.prefill(q.view(length, -1), q.view(length, -1), k, k, v, out)
        outs.append(out)
    torch.cuda.synchronize()
    for i, out in enumerate(outs[1:], 1):
        rows = (out != outs[0]).any(1).nonzero().flatten()
        assert rows.numel() == 0, f"run {i}: rows {rows[:16].tolist()} differ from run 0"


def _synthetic_runs(seed, *, hkv, g, d, clusters=64, qn=48, n_local=56, page=16, empty_head=None):
    """A chunk over synthetic page-multiple cluster runs, after the reference's own
    synthetic case (tests/test_kv_outer_fused_local.py:86-106): run sizes 1-16 pages,
    visible rows anywhere from none to the whole run, random selections of which three
    queries pick nothing in KV head 1, and optionally a KV head with no cluster at all.
    The window holds n_local >= qn rows, as every query sees itself."""
    gen = torch.Generator().manual_seed(seed)
    sizes = torch.randint(1, 17, (clusters,), generator=gen) * page
    length = int(sizes.sum())
    indptr = torch.zeros(hkv, clusters + 1, dtype=torch.int32)
    indptr[:, 1:] = torch.cumsum(sizes, 0)[None].to(torch.int32)
    causal = (torch.rand(hkv, clusters, generator=gen) * (sizes[None] + 1)).floor()
    causal = torch.minimum(causal, sizes[None].float()).to(torch.int32)
    qmask = torch.randint(0, 1 << 31, (qn, hkv, clusters // 32), generator=gen, dtype=torch.int64)
    qmask = (qmask & torch.randint(0, 1 << 31, qmask.shape, generator=gen)).to(torch.int32)
    qmask[:3, 1] = 0
    if empty_head is not None:
        qmask[:, empty_head] = 0
    packed = torch.randn(2, length, hkv, d, generator=gen).to(torch.bfloat16)
    q = torch.randn(qn, hkv * g, d, generator=gen).to(torch.bfloat16)
    local = torch.randn(2, n_local, hkv, d, generator=gen).to(torch.bfloat16)
    return q, packed, qmask, causal, indptr, local


def _synthetic_reference(q, packed, qmask, causal, indptr, local, wstart, chunk_start):
    """fp64 attention of each query over its selected clusters' first causal rows and
    the window rows up to its own position."""
    qn = q.shape[0]
    hkv, c = causal.shape
    length, n_local = packed.shape[1], local.shape[1]
    sel = ref.unpack_bits(qmask, c)                                   # [Q, Hkv, C]
    run = torch.zeros(hkv, c, length, dtype=torch.bool)
    for h in range(hkv):
        for ci in range(c):
            a = int(indptr[h, ci])
            run[h, ci, a:a + int(causal[h, ci])] = True
    keys_run = torch.einsum("qhc,hcl->qhl", sel.double(), run.double()) > 0
    own = chunk_start + torch.arange(qn) - wstart                     # window row of each query
    keys_win = (torch.arange(n_local)[None, :] <= own[:, None])[:, None, :].expand(qn, hkv, n_local)
    keys = torch.cat([keys_run, keys_win], -1)
    k = torch.cat([packed[0], local[0]], 0)
    v = torch.cat([packed[1], local[1]], 0)
    return attention_reference(q, keys, k, v, q.shape[-1] ** -0.5)


@pytest.mark.parametrize("hkv,g,d,empty_head", [(2, 2, 128, None), (2, 2, 128, 0), (4, 4, 256, 2)])
def test_kv_outer_on_synthetic_runs_with_empty_selections(hkv, g, d, empty_head):
    """Cluster runs of ragged page counts, visible rows from none to all, queries and a
    whole KV head selecting nothing: every row within bf16 tolerance of fp64 over the
    defined key set, and a query that selected nothing in a head gets exactly the
    window's attention (the same bits as a run in which no query selects anything)."""
    from semblo_amd.kv_outer import kv_outer_attention
    q, packed, qmask, causal, indptr, local = _synthetic_runs(11 + hkv, hkv=hkv, g=g, d=d,
                                                              empty_head=empty_head)
    qn, n_local = q.shape[0], local.shape[1]
    wstart, chunk_start = 1000, 1000 + n_local - qn

    def run(mask):
        out, _ = kv_outer_attention(q.to(DEV), packed.to(DEV), mask.to(DEV), causal.to(DEV),
                                    indptr.to(DEV), sm_scale=d ** -0.5,
                                    local_kv=(local[0].to(DEV), local[1].to(DEV)),
                                    chunk_start=chunk_start, wstart=wstart)
        torch.cuda.synchronize()
        return out.cpu()

    got = run(qmask)
    want = _synthetic_reference(q, packed, qmask, causal, indptr, local, wstart, chunk_start)
    assert torch.isfinite(got.float()).all()
    assert_close_bf16(got, want, "synthetic runs")
    window_only = run(torch.zeros_like(qmask))
    assert_close_bf16(window_only, _synthetic_reference(q, packed, torch.zeros_like(qmask), causal,
                                                        indptr, local, wstart, chunk_start), "window")
    none = ~ref.unpack_bits(qmask, causal.shape[1]).any(-1)           # [Q, Hkv]: selected nothing
    assert bool(none[:3, 1].all())
    for h in range(hkv):
        rows = none[:, h].nonzero().flatten()
        assert torch.equal(got[rows, h * g:(h + 1) * g], window_only[rows, h * g:(h + 1) * g]), h
