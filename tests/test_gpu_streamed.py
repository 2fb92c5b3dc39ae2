"""Layer-major streamed prefill on the GPU (the reference's StreamedPrefillSession,
model.py:1431-1531, driven as PrefillStreamer.run drives it, streamed_prefill.py:
496-545 and 710-736): keys of every slice, the index fitted once on the whole prompt,
then the queries of every slice in chunks counted from the slice's start.

  * slices that are a multiple of the query chunk: the same index and the same output
    as the whole-prompt path, bit for bit (the same chunks, the same keys read back
    from the packed store through the inverse map);
  * ragged slices: every chunk against fp64, dense-prefix chunks over every earlier key,
    sparse chunks over the GPU's own key sets (recorded plans), with no query off
    tolerance, and their selection against the oracle's up to counted near-ties.
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import assert_close_bf16, attention_reference, check_recorded_chunk

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(name, chunk=512, seed=5):
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    cfg = SembloRuntimeConfig(num_q_heads=8, num_kv_heads=2, head_dim=128, query_chunk_size=chunk,
                              codebook_seed=seed, layer_idx=0)
    layer = SembloAttention(cfg, layer_name=name)
    layer.plan_log = []
    return layer


def _inputs(length, seed=5):
    from semblo_amd.synthetic import mixture_layer
    return mixture_layer(length, 8, 2, 128, mixtures=32, seg=(32, 256), seed=seed)


def test_streamed_slices_equal_the_whole_prompt_path():
    length = 4096
    inp = _inputs(length)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    whole = _layer("test.streamed.whole")
    out_w = torch.empty(length, 8 * 128, dtype=torch.bfloat16, device=DEV)
    whole.prefill(q, q, k, k, v, out_w)
    streamed = _layer("test.streamed.slices")
    out_s = torch.empty_like(out_w)
    streamed.prefill_streamed(q, q, k, k, v, out_s, 2048)
    torch.cuda.synchronize()
    a, b = whole.index, streamed.index
    for name in ("codebooks", "posting_positions", "bucket_indptr", "bucket_sizes", "packed_kv"):
        assert torch.equal(getattr(a, name).cpu(), getattr(b, name).cpu()), name
    assert torch.equal(out_w.cpu(), out_s.cpu())
    assert streamed.arena is not None and streamed.index.original_kv is None


@pytest.mark.parametrize("slice_tokens", [1000, 1536])
def test_streamed_ragged_slices_match_fp64(slice_tokens):
    length, hkv, d = 4096, 2, 128
    inp = _inputs(length, seed=6)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    layer = _layer(f"test.streamed.{slice_tokens}", seed=6)
    out = torch.empty(length, 8 * d, dtype=torch.bfloat16, device=DEV)
    layer.prefill_streamed(q, q, k, k, v, out, slice_tokens)
    torch.cuda.synchronize()
    got = out.view(length, 8, d).cpu()
    idx = layer.index
    target = length // 16
    sparse = {r["chunk_start"] for r in layer.plan_log}
    # the chunks: counted from each slice's start (model.py:906-972)
    starts = [s + a for s in range(0, length, slice_tokens)
              for a in range(0, min(slice_tokens, length - s), 512)]
    assert sparse == {cs for cs in starts if cs > 4 * target}
    for cs in starts:
        if cs in sparse:
            continue
        ce = min(cs + 512, (cs // slice_tokens + 1) * slice_tokens, length) - 1
        p = torch.arange(cs, ce + 1)
        keys = (torch.arange(length)[None, :] <= p[:, None])[:, None, :].expand(-1, hkv, -1)
        want = attention_reference(inp.q[cs:ce + 1], keys, inp.k, inp.v, d ** -0.5)
        assert_close_bf16(got[cs:ce + 1], want, f"dense chunk {cs}")
    near = 0
    for rec in layer.plan_log:
        rep = check_recorded_chunk(rec, inp.q, inp.q, inp.k, inp.v, idx, got, target=target,
                                   tag=f"streamed {slice_tokens}")
        near += rep["near_ties"]
    print(f"slices of {slice_tokens}: {len(starts)} chunks ({len(sparse)} sparse), "
          f"{near} near-tie selection differences")


def test_streamed_session_refuses_out_of_order_use():
    layer = _layer("test.streamed.errors")
    session = layer.begin_streamed_prefill(1024)
    q = torch.zeros(16, 8, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="before ingest"):
        session.queries(q, q, 0)
    with pytest.raises(RuntimeError, match="no slice was staged"):
        session.ingest()
    k = torch.zeros(512, 2, 128, dtype=torch.bfloat16, device=DEV)
    session.keys(k, k, k, 0, 512)
    with pytest.raises(RuntimeError, match="512 of 1024 positions"):
        session.ingest()
