"""Parity at the benchmark configurations' full sizes.

Each test runs the product path at the configuration's real shape (prompt length, heads,
head dim, cluster count, budget, query chunk) and checks a sample of its outputs against
the oracle, so that the paths only these sizes reach run under a check: cluster runs
longer than a decode split's row chunk, C = 256, thousands of work items over the eight
XCD queues, x8-norm sink keys, the decode block table past its LDS copy, and the token-
order store at 512K positions.

  * membership: every k-means step of some KV heads against the oracle fed the GPU's own
    inputs (flips counted as near-ties), the layout bit-exact;
  * prefill: sampled queries of sparse chunks against fp64 over the GPU's recorded key
    sets (no query off tolerance) and their selection against the oracle's (near-ties
    counted); sampled queries of dense chunks against fp64 causal attention;
  * decode: steps against fp64 over the GPU's own selected runs plus the suffix, and the
    selection against the oracle's.

Tolerances: attention 2e-2 abs + 1e-2 rel (bf16); near-ties within 1e-4 relative.
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import (assert_close_bf16, causal_rows_reference, check_fit_trace,
                      check_recorded_chunk, compare_selection, decode_rows_reference,
                      oracle_select)
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _log(*a):
    print("[configs]", *a, flush=True)


def _inputs(conf, seed, device=DEV):
    from semblo_amd.synthetic import mixture_layer
    return mixture_layer(conf["length"], conf["hq"], conf["hkv"], conf["d"],
                         mixtures=conf["mixtures"], seg=conf["seg"],
                         log_uniform=conf["log_uniform"], sinks=conf["sinks"], seed=seed,
                         device=device)


def _layer(conf, seed, chunk, name, reserve=1024):
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    cfg = SembloRuntimeConfig(num_q_heads=conf["hq"], num_kv_heads=conf["hkv"], head_dim=conf["d"],
                              query_chunk_size=chunk, codebook_seed=seed, suffix_reserve=reserve)
    layer = SembloAttention(cfg, layer_name=name)
    layer.plan_log = []
    return layer


def _prefill(layer, inp):
    from semblo_amd.attention_op import sparse_attention_op
    length, hq, d = inp.q.shape
    out = torch.empty(length, hq * d, dtype=torch.bfloat16, device=DEV)
    sparse_attention_op(torch.arange(length, device=DEV), inp.q.view(length, -1),
                        inp.q.view(length, -1), inp.k, inp.v, inp.q, inp.k, out, layer.layer_name)
    torch.cuda.synchronize()
    return out.view(length, hq, d)


def _membership_check(k_cpu, index, seed, heads, tag, num_clusters=None, same_sizes=True):
    """A traced GPU build (same call as the layer's, so bit-identical to it) with every
    k-means step of ``heads`` checked against the oracle."""
    from semblo_amd.state import ProductPostingIndex
    product = ref.routing_normalize_keys(k_cpu)
    kw = {"num_clusters": num_clusters} if num_clusters else {}
    trace = []
    idx = ProductPostingIndex.build(k_cpu.to(DEV), torch.arange(k_cpu.shape[0], device=DEV),
                                    codebook_seed=seed, router_pass=True, fit_trace=trace, **kw)
    torch.cuda.synchronize()
    assert torch.equal(idx.codebooks.cpu(), index.codebooks.cpu()), "the build is not deterministic"
    if same_sizes:
        assert torch.equal(idx.bucket_sizes.cpu(), index.bucket_sizes.cpu())
    steps = []
    ref.build_flat_index(product, codebook_seed=seed, fit_steps=steps, **kw)
    for h in heads:
        rep = check_fit_trace(product[:, h], trace[h], steps[h]["steps"], steps[h]["final_assign"],
                              steps[h]["final_centroids"], tag=f"{tag} head {h}",
                              k_pre_h=k_cpu[:, h])
        _log(f"{tag} membership head {h}: {rep}")


def _sparse_checks(layer, inp_cpu, out_cpu, chunk_ids, rows_per_chunk, tag, gen):
    recs = {r["chunk_start"]: r for r in layer.plan_log}
    starts = sorted(recs)
    for i in chunk_ids:
        rec = recs[starts[i]]
        n = rec["chunk_end"] + 1 - rec["chunk_start"]
        rows = torch.randperm(n, generator=gen)[:rows_per_chunk].sort().values
        rows[-1] = n - 1                                   # the chunk's last query too
        rep = check_recorded_chunk(rec, inp_cpu.q, inp_cpu.q, inp_cpu.k, inp_cpu.v, layer.index,
                                   out_cpu, target=layer.target_tokens, rows=rows, tag=tag)
        _log(f"{tag} sparse chunk {rec['chunk_start']}: {rep}")


def _dense_check(inp_cpu, out_cpu, cs, ce, nrows, tag, gen):
    n = ce + 1 - cs
    rows = torch.randperm(n, generator=gen)[:nrows].sort().values
    want = causal_rows_reference(inp_cpu.q[cs + rows], cs + rows, inp_cpu.k, inp_cpu.v,
                                 inp_cpu.q.shape[-1] ** -0.5)
    err = assert_close_bf16(out_cpu[cs + rows], want, f"{tag} dense chunk {cs}")
    _log(f"{tag} dense chunk {cs}: {nrows} rows, max err {err:.3g}")


def _decode_checks(layer, inp, steps, tag, seed=1, graph_replay=False):
    """``steps`` decode steps through fused_decode_step: each against fp64 over its own
    selected runs plus the suffix so far, its selection against the oracle's.  With
    ``graph_replay`` the same steps are then captured in one HIP graph and replayed: the
    outputs must equal the eager ones bit for bit."""
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.synthetic import decode_queries
    from test_gpu_decode import _csr_to_sel
    idx, arena = layer.index, layer.arena
    cfg = layer.runtime_config
    hq, hkv, d = layer.num_heads, layer.num_kv_heads, layer.head_dim
    c = idx.num_buckets
    length = int(arena.prompt_length)
    qs, kn, vn = decode_queries(inp, steps, hq, seed=seed)
    qs, kn, vn = qs.to(DEV), kn.to(DEV), vn.to(DEV)
    pos = torch.arange(length, length + steps, dtype=torch.int32, device=DEV)
    outs = torch.empty(steps, hq * d, dtype=torch.bfloat16, device=DEV)
    csr = torch.empty(3 * hkv * c + 2 * hkv, dtype=torch.int32, device=DEV)
    kw = dict(temperature=cfg.selection_temperature, beta=cfg.bucket_size_penalty,
              target_tokens=layer.decode_budget(), sm_scale=layer.scaling,
              num_splits=cfg.decode_num_splits, iters=cfg.iters, suffix_splits=arena.suffix_splits)
    codebooks, sizes, indptr = idx.codebooks.cpu(), idx.bucket_sizes.cpu(), idx.bucket_indptr.cpu()
    near = 0
    for t in range(steps):
        fused_decode_step(layer, arena, q_post=qs[t:t + 1], q_pre=qs[t:t + 1], positions=pos[t:t + 1],
                          k_post=kn[t:t + 1], v_states=vn[t:t + 1], output=outs[t:t + 1],
                          csr_out=csr, **kw)
        torch.cuda.synchronize()
        sel = _csr_to_sel(csr.cpu(), idx)
        q_cpu = qs[t].cpu()
        exp = oracle_select(ref.trivial_router_vectors(q_cpu[None], 1), codebooks, sizes[None],
                            temperature=cfg.selection_temperature, beta=cfg.bucket_size_penalty,
                            target=layer.decode_budget())
        near += compare_selection(sel[None], exp["sel"], exp["score"], exp["theta"])["near_ties"]
        want = decode_rows_reference(q_cpu, idx.packed_kv, indptr, sizes, sel, kn[:t + 1].cpu(),
                                     vn[:t + 1].cpu(), layer.scaling)
        assert_close_bf16(outs[t].view(hq, d).cpu(), want, f"{tag} decode step {t}")
    _log(f"{tag}: {steps} decode steps match fp64 ({near} near-tie selection differences)")
    if graph_replay:
        eager = outs.clone()
        outs.zero_()

        def body():
            for t in range(steps):
                fused_decode_step(layer, arena, q_post=qs[t:t + 1], q_pre=qs[t:t + 1],
                                  positions=pos[t:t + 1], k_post=kn[t:t + 1], v_states=vn[t:t + 1],
                                  output=outs[t:t + 1], **kw)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            body()
        for rep in range(2):
            outs.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(outs, eager), f"{tag}: graph replay {rep} differs from the eager steps"
        _log(f"{tag}: {steps} steps captured in one HIP graph replay bit-equal to eager")


@pytest.mark.parametrize("chunk", [8192, 1024])
def test_config1_prefill_and_decode(chunk):
    """Config 1 (8 / 2 / 128, L = 8192, 64 mixtures, K = 512).  At the paper's query chunk
    (8192) the single chunk is dense; at 1024 the chunks past 4K = 2048 are sparse."""
    from semblo_amd.synthetic import CONFIGS
    conf = dict(CONFIGS[1])
    _log(f"config 1, chunk {chunk}")
    inp = _inputs(conf, seed=101, device="cpu")
    inp_d = type(inp)(q=inp.q.to(torch.bfloat16).to(DEV), k=inp.k.to(torch.bfloat16).to(DEV),
                      v=inp.v.to(torch.bfloat16).to(DEV), seg_centre=inp.seg_centre,
                      centres=inp.centres.to(DEV))
    layer = _layer(conf, 101, chunk, f"test.config1.{chunk}")
    out = _prefill(layer, inp_d).cpu()
    cpu = type(inp)(q=inp_d.q.cpu(), k=inp_d.k.cpu(), v=inp_d.v.cpu(), seg_centre=None, centres=None)
    gen = torch.Generator().manual_seed(chunk)
    length = conf["length"]
    target = layer.target_tokens
    assert target == 512
    for cs in range(0, length, chunk):
        if cs <= 4 * target:
            _dense_check(cpu, out, cs, cs + chunk - 1, min(chunk, 256), "config 1", gen)
    if chunk == 1024:
        assert len(layer.plan_log) == 5
        _sparse_checks(layer, cpu, out, range(5), 128, "config 1", gen)
        _membership_check(cpu.k, layer.index, 101, [0, 1], "config 1")
    else:
        assert not layer.plan_log
    _decode_checks(layer, inp_d, 16, f"config 1 chunk {chunk}")


def test_config2_prefill_and_decode_shuffled_suffix_past_the_table():
    """Config 2 (16 / 4 / 256, L = 32768, 256 mixtures, K = 2048).  The decode arena is
    re-made with a suffix of 70,000 tokens in shuffled block order, so the block table is
    past what a step stages in LDS (tb_n > 256) and the step reads it from memory."""
    from semblo_amd.arena import DecodeArena
    from semblo_amd.synthetic import CONFIGS
    conf = dict(CONFIGS[2])
    _log("config 2")
    inp = _inputs(conf, seed=202)
    layer = _layer(conf, 202, 8192, "test.config2")
    out = _prefill(layer, inp).cpu()
    cpu = type(inp)(q=inp.q.cpu(), k=inp.k.cpu(), v=inp.v.cpu(), seg_centre=None, centres=None)
    gen = torch.Generator().manual_seed(2)
    assert [r["chunk_start"] for r in layer.plan_log] == [16384, 24576]
    _dense_check(cpu, out, 8192, 16383, 64, "config 2", gen)
    _sparse_checks(layer, cpu, out, range(2), 96, "config 2", gen)
    _membership_check(cpu.k, layer.index, 202, range(4), "config 2")
    layer.arena = DecodeArena(layer.index, reserve=70000,
                              shuffle_blocks=torch.Generator().manual_seed(5))
    base = conf["length"] // layer.arena.suffix_block
    table = layer.arena.suffix_table[base:].cpu()
    assert table.numel() > 256 and not torch.equal(table, torch.arange(table.numel(), dtype=table.dtype))
    _decode_checks(layer, inp, 64, "config 2 (shuffled suffix, table in memory)")


def test_config3_headline_prefill_and_decode():
    """Config 3 (16 / 4 / 256, L = 131072, 1024 mixtures, log-uniform segments, 4 sink
    keys at 8x norm, C = 128, K = 8192): 5 dense-prefix and 11 sparse chunks."""
    from semblo_amd.synthetic import CONFIGS
    conf = dict(CONFIGS[3])
    _log("config 3")
    inp = _inputs(conf, seed=303)
    layer = _layer(conf, 303, 8192, "test.config3")
    out = _prefill(layer, inp).cpu()
    cpu = type(inp)(q=inp.q.cpu(), k=inp.k.cpu(), v=inp.v.cpu(), seg_centre=None, centres=None)
    gen = torch.Generator().manual_seed(3)
    assert layer.index.num_buckets == 128 and layer.target_tokens == 8192
    assert len(layer.plan_log) == 11
    _dense_check(cpu, out, 0, 8191, 16, "config 3", gen)          # every query sees the sinks
    _dense_check(cpu, out, 32768, 40959, 32, "config 3", gen)
    _sparse_checks(layer, cpu, out, [0, 5, 10], 48, "config 3", gen)
    _membership_check(cpu.k, layer.index, 303, [0, 3], "config 3")
    _decode_checks(layer, inp, 16, "config 3", graph_replay=True)


def test_config4_token_order_store_and_attention():
    """Config 4 (16 / 4 / 256, L = 524288, C = 256, K = 32768): the token-order prefill in
    8192-position slices, blocks fitted on the first 73,728 positions, later keys assigned
    into them.  Checked: the fit (every k-means step of one head), the store (each position
    once, runs in position order, rows equal to the prompt's K/V), the nearest-cluster ids
    of two slices against the oracle, sampled queries of three sparse slices and of a dense
    slice, and decode steps over the reserved-gap layout plus the suffix."""
    from semblo_amd.synthetic import CONFIGS
    from semblo_amd.token_outer_prefill import nearest_cluster
    from test_gpu_token_order import _ids_near_ties
    conf = dict(CONFIGS[4])
    _log("config 4")
    inp = _inputs(conf, seed=404)
    length, hq, hkv, d = conf["length"], conf["hq"], conf["hkv"], conf["d"]
    layer = _layer(conf, 404, 8192, "test.config4")
    out = torch.empty(length, hq * d, dtype=torch.bfloat16, device=DEV)
    layer.prefill_token_order(inp.q, inp.q, inp.k, inp.k, inp.v, out, 8192,
                              fit_tokens=conf["fit_tokens"])
    torch.cuda.synchronize()
    session = layer.last_session
    idx = layer.index
    c = idx.num_buckets
    assert c == 256 and session.target == 32768 and session.fit_at == 73728
    _log(f"config 4: {session.repacks} repacks, {len(layer.plan_log)} sparse slices")
    # the store, on the device
    inv = idx.inverse_positions().long()
    post = idx.posting_positions.long()
    ar = torch.arange(length, device=DEV)
    for h in range(hkv):
        assert torch.equal(post[h, inv[h]], ar)
        assert torch.equal(idx.packed_kv[0, inv[h], h], inp.k[:, h])
        assert torch.equal(idx.packed_kv[1, inv[h], h], inp.v[:, h])
        cl = torch.searchsorted(idx.bucket_indptr[h].long(), inv[h], right=True) - 1
        # runs in position order: within a cluster, rows increase with position
        order = torch.argsort(cl * length + ar)
        assert bool((inv[h][order][1:] > inv[h][order][:-1]).all())
        assert torch.equal(torch.bincount(cl, minlength=c).to(torch.int32), idx.bucket_sizes[h])
    cpu = type(inp)(q=inp.q.cpu(), k=inp.k.cpu(), v=inp.v.cpu(), seg_centre=None, centres=None)
    # the fit on the staged prefix
    _membership_check(cpu.k[:session.fit_at], idx, 404, [1], "config 4 fit", num_clusters=256,
                      same_sizes=False)
    # nearest-cluster ids of two appended slices: the store's clusters of those positions
    for start in (81920, 516096):
        ids = nearest_cluster(inp.k[start:start + 8192], idx.codebooks).cpu()
        for h in range(hkv):
            rows = inv[h, start:start + 8192]
            cl = (torch.searchsorted(idx.bucket_indptr[h].long(), rows, right=True) - 1).cpu()
            assert torch.equal(cl, ids[h].long())
            want = ref.nearest_cluster(cpu.k[start:start + 8192, h], idx.codebooks[h].cpu())
            flips = _ids_near_ties(cpu.k[start:start + 8192, h], idx.codebooks[h].cpu(), ids[h], want)
            _log(f"config 4 slice {start} head {h}: {flips} near-tie ids")
    out_cpu = out.view(length, hq, d).cpu()
    gen = torch.Generator().manual_seed(4)
    _dense_check(cpu, out_cpu, 98304, 106495, 16, "config 4", gen)
    _sparse_checks(layer, cpu, out_cpu, [0, 20, len(layer.plan_log) - 1], 24, "config 4", gen)
    _decode_checks(layer, inp, 8, "config 4")
