"""The capped partial buffer of the sparse chunks (kv_outer.partials_cap_bytes).

A chunk enqueued without a host read sizes its partial rows by the bound every
query selecting every cluster, capped at SEMBLO_KV_OUTER_PARTIALS_CAP_MB.  A
chunk with more entries than the cap runs nothing (empty work list, combine
skipped) and is run again at its exact count once its overflow flag is read
(the reference reads the count in the first place, kv_outer.py:592-613).  The
outputs must not depend on the cap: bit-equal to the uncapped run, on the
layer-major, token-order and streamed paths."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(name, chunk, seed=3, hq=8, hkv=2, d=128):
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=chunk,
                              codebook_seed=seed, layer_idx=0)
    return SembloAttention(cfg, layer_name=name)


def _inputs(length, hq=8, hkv=2, d=128, seed=11):
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(length, hq, hkv, d, mixtures=32, seed=seed)
    return inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)


def _layer_major(cap_mb, monkeypatch, length=4096):
    if cap_mb is None:
        monkeypatch.delenv("SEMBLO_KV_OUTER_PARTIALS_CAP_MB", raising=False)
    else:
        monkeypatch.setenv("SEMBLO_KV_OUTER_PARTIALS_CAP_MB", str(cap_mb))
    q, k, v = _inputs(length)
    layer = _layer(f"cap.{cap_mb}", 512)
    out = torch.empty(length, 8 * 128, dtype=torch.bfloat16, device=DEV)
    layer.prefill(q.view(length, -1), q.view(length, -1), k, k, v, out)
    torch.cuda.synchronize()
    return out.cpu(), layer.partials_reruns


def test_layer_major_prefill_is_the_same_under_any_cap(monkeypatch):
    from semblo_amd.kv_outer import partials_capacity
    # 4096 tokens, chunk 512, 8/2/128: 3 dense-prefix chunks (K = 256, starts up to 4 K = 1024), 5 sparse
    full_mb = partials_capacity(512, 2, 128) * (4 * 128 * 2 + 4 * 4) / (1 << 20)
    base, reruns0 = _layer_major(None, monkeypatch)
    assert reruns0 == 0                              # the bound fits under the default cap
    tiny, reruns_t = _layer_major(0.01, monkeypatch)   # every sparse chunk overflows
    assert reruns_t == 5, reruns_t
    half, reruns_h = _layer_major(full_mb / 2, monkeypatch)   # capped, no chunk overflows
    assert reruns_h == 0, reruns_h
    assert torch.equal(tiny, base)
    assert torch.equal(half, base)


def test_token_order_prefill_is_the_same_under_a_tiny_cap(monkeypatch):
    tokens, chunk = 4096, 512
    q, k, v = _inputs(tokens, seed=12)
    outs, reruns = [], []
    for cap in (None, 0.01):
        if cap is None:
            monkeypatch.delenv("SEMBLO_KV_OUTER_PARTIALS_CAP_MB", raising=False)
        else:
            monkeypatch.setenv("SEMBLO_KV_OUTER_PARTIALS_CAP_MB", str(cap))
        layer = _layer(f"cap.token.{cap}", chunk, seed=12)
        session = layer.begin_token_outer_prefill(tokens, chunk, fit_tokens=512)
        out = torch.empty(tokens, 8, 128, dtype=torch.bfloat16, device=DEV)
        for start in range(0, tokens, chunk):
            stop = min(tokens, start + chunk)
            session.slice_projected(q[start:stop], q[start:stop], k[start:stop], k[start:stop], v[start:stop],
                                    start, stop, out=out[start:stop])
        session.finish()
        torch.cuda.synchronize()
        outs.append(out.cpu())
        reruns.append(session.guard.reruns)
    assert reruns[0] == 0 and reruns[1] > 0, reruns
    assert torch.equal(outs[0], outs[1])


def test_streamed_queries_are_the_same_under_a_tiny_cap(monkeypatch):
    length = 4096
    q, k, v = _inputs(length, seed=13)
    outs = []
    for cap in (None, 0.01):
        if cap is None:
            monkeypatch.delenv("SEMBLO_KV_OUTER_PARTIALS_CAP_MB", raising=False)
        else:
            monkeypatch.setenv("SEMBLO_KV_OUTER_PARTIALS_CAP_MB", str(cap))
        layer = _layer(f"cap.streamed.{cap}", 512, seed=13)
        out = torch.empty(length, 8 * 128, dtype=torch.bfloat16, device=DEV)
        layer.prefill_streamed(q, q, k, k, v, out, 1024)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1])
