"""The attention sink on the GPU (SEMBLO_SINK_TOKENS=S; off by default in the reference).

Positions 0..S-1 form cluster 0, whose descriptor is zero, and the other positions are
fitted into clusters 1..C-1 (state.py:757-782).  Every selection hides cluster 0 from its
search, shares the budget less S among the other clusters, and then reads cluster 0 for
every query: the prefill through _hold_out_sink / _force_sink_bit (fused_prefill.py:
202-216, 382-405), the decode step inside its selection (fused_decode.py:164-187).

Checked: the partition (cluster 0 exactly, zero descriptor), every sparse chunk's
attention against fp64 over the GPU's own key sets with no query off tolerance, its
selection against the oracle's sink rule up to counted near-ties, and decode steps the
same way.  The build itself against the reference's own sink build is
test_gpu_kmeans.py's golden test (kmeans_sink*.pt).
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import (assert_close_bf16, attention_reference, check_recorded_chunk,
                      compare_selection, oracle_select)
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
SINK = 32


def _csr_to_sel(csr, idx):
    hkv, c = idx.bucket_sizes.shape
    n = hkv * c
    rstart = csr[:n].view(hkv, c)
    rcount = csr[3 * n:3 * n + hkv]
    indptr = idx.bucket_indptr.cpu()
    sizes = idx.bucket_sizes.cpu()
    sel = torch.zeros(hkv, c, dtype=torch.bool)
    for h in range(hkv):
        for p in range(int(rcount[h])):
            st = int(rstart[h, p])
            cand = torch.nonzero((indptr[h, :-1] == st) & (sizes[h] > 0)).flatten()
            assert cand.numel() == 1
            sel[h, cand[0]] = True
    return sel


def test_layer_prefill_and_decode_with_a_sink(monkeypatch):
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    from semblo_amd.synthetic import decode_queries, mixture_layer
    monkeypatch.setenv("SEMBLO_SINK_TOKENS", str(SINK))
    length, hq, hkv, d = 4096, 8, 2, 128
    cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=512,
                              codebook_seed=7, layer_idx=0, suffix_reserve=64)
    layer = SembloAttention(cfg, layer_name="test.sink.0")
    layer.plan_log = []
    inp = mixture_layer(length, hq, hkv, d, mixtures=32, seg=(32, 256), seed=7)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    out = torch.empty(length, hq * d, dtype=torch.bfloat16, device=DEV)
    layer.prefill(q, q, k, k, v, out)
    torch.cuda.synchronize()
    got = out.view(length, hq, d).cpu()
    idx = layer.index
    sizes, indptr = idx.bucket_sizes.cpu(), idx.bucket_indptr.cpu()
    posting = idx.posting_positions.cpu()
    # the partition: cluster 0 is positions 0..S-1 on every head, and only they
    for h in range(hkv):
        assert int(sizes[h, 0]) == SINK
        assert torch.equal(posting[h, int(indptr[h, 0]):int(indptr[h, 0]) + SINK],
                           torch.arange(SINK, dtype=torch.int32))
    assert torch.count_nonzero(idx.codebooks[:, :, 0].cpu()) == 0
    target = length // 16
    assert layer.plan_log, "no sparse chunk ran"
    near = 0
    for rec in layer.plan_log:
        assert bool((rec["qmask"].cpu()[..., 0] & 1).all()), "the sink is not read by every query"
        rep = check_recorded_chunk(rec, inp.q, inp.q, inp.k, inp.v, idx, got, target=target,
                                   tag="sink", sink=SINK)
        near += rep["near_ties"]
    # decode steps: the same rule inside the step's own selection
    steps = 8
    qs, kn, vn = decode_queries(inp, steps, hq, seed=7)
    c = idx.num_buckets
    csr = torch.empty(3 * hkv * c + 2 * hkv, dtype=torch.int32, device=DEV)
    dec = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    packed = idx.packed_kv.cpu()
    from semblo_amd.fused_decode import fused_decode_step
    for t in range(steps):
        pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
        qd = qs[t:t + 1].to(DEV)
        fused_decode_step(layer, layer.arena, q_post=qd, q_pre=qd, positions=pos,
                          k_post=kn[t:t + 1].to(DEV), v_states=vn[t:t + 1].to(DEV), output=dec,
                          temperature=cfg.selection_temperature, beta=cfg.bucket_size_penalty,
                          target_tokens=target, sm_scale=d ** -0.5, num_splits=16, iters=16,
                          csr_out=csr)
        torch.cuda.synchronize()
        sel = _csr_to_sel(csr.cpu(), idx)
        assert bool(sel[:, 0].all()), "the decode step did not read the sink"
        want = ref.decode_reference(qd[0].cpu(), packed, indptr, sizes, sel, kn[:t + 1].cpu(),
                                    vn[:t + 1].cpu(), d ** -0.5)
        assert_close_bf16(dec.view(hq, d).cpu(), want, f"sink decode step {t}")
        vec = ref.trivial_router_vectors(qd.cpu(), 1)
        exp = oracle_select(vec, idx.codebooks.cpu(), sizes[None], temperature=0.1, beta=0.25,
                            target=target, sink=SINK)
        near += compare_selection(sel[None], exp["sel"], exp["score"], exp["theta"])["near_ties"]
    print(f"sink {SINK}: {len(layer.plan_log)} sparse chunks, {steps} decode steps, "
          f"{near} near-tie selection differences")
