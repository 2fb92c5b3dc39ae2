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
        session.attend(q, q, 0)
    with pytest.raises(RuntimeError, match="no slice was staged"):
        session.ingest()
    k = torch.zeros(512, 2, 128, dtype=torch.bfloat16, device=DEV)
    session.stage_keys(k, k, k, 0, 512)
    with pytest.raises(RuntimeError, match="512 of 1024 positions"):
        session.ingest()


class _Projections:
    """A stand-in for the model around the layer: Q, K, V and a gate projected from
    hidden states, rotate-half RoPE on Q and K, the gated output projected back.  All
    in fp64 and rounded to bf16 once, so a row's projection does not depend on how
    many rows a call carries (a slice's or the whole prompt's)."""

    def __init__(self, hidden=256, hq=8, hkv=2, d=128, seed=0):
        g = torch.Generator().manual_seed(seed)
        self.hq, self.hkv, self.d = hq, hkv, d

        def w(rows, cols):
            return (torch.randn(rows, cols, generator=g, dtype=torch.float64) * rows ** -0.5).to(DEV)
        self.wq, self.wk, self.wv = w(hidden, hq * d), w(hidden, hkv * d), w(hidden, hkv * d)
        self.wg, self.wo = w(hidden, hq * d), w(hq * d, hidden)
        self.inv = (1.0 / 10000 ** (torch.arange(0, d, 2, dtype=torch.float64) / d)).to(DEV)
        self.calls = 0

    def rope(self, x, pos):
        p = (pos[0] if pos.ndim == 2 else pos).to(torch.float64)
        ang = p[:, None] * self.inv[None, :]
        cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]
        x1, x2 = x[..., : self.d // 2], x[..., self.d // 2:]
        return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], -1)

    def project_qkv(self, pos, h):
        self.calls += 1
        x = h.to(torch.float64)
        n = x.shape[0]
        qp = (x @ self.wq).view(n, self.hq, self.d)
        kp = (x @ self.wk).view(n, self.hkv, self.d)
        v = (x @ self.wv).view(n, self.hkv, self.d)
        bf = torch.bfloat16
        return (self.rope(qp, pos).to(bf), self.rope(kp, pos).to(bf), v.to(bf), qp.to(bf), kp.to(bf),
                (x @ self.wg).to(bf))

    def finish_output(self, attn, gate):
        return ((attn.to(torch.float64) * torch.sigmoid(gate.to(torch.float64))) @ self.wo).to(torch.bfloat16)


def _hidden(length, width=256, seed=7):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(length, width, generator=g).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("grid", [False, True])
def test_streamed_session_driven_by_hidden_states(grid):
    """The reference's calls (PrefillStreamer._sparse_layer, streamed_prefill.py:710-736):
    begin with the prompt's positions (a [T] row or an M-RoPE grid [3, T]), keys(rope,
    hidden, s, e) per slice, ingest, queries(rope, positions, hidden, s) per slice.  The
    layer's output rows equal the whole-prompt path's attention over the same
    projections, gated and projected out, bit for bit."""
    length, slice_tokens = 4096, 1024
    proj = _Projections()
    h = _hidden(length)
    flat = torch.arange(length, device=DEV)
    positions = flat.expand(3, length) if grid else flat
    q_post, k_post, v, q_pre, k_pre, gate = proj.project_qkv(flat, h)
    whole = _layer("test.streamed.hidden.whole")
    attn = torch.empty(length, 8 * 128, dtype=torch.bfloat16, device=DEV)
    whole.prefill(q_post, q_pre, k_pre, k_post, v, attn)
    want = proj.finish_output(attn, gate)

    layer = _layer("test.streamed.hidden")
    layer.attach_projections(proj.project_qkv, proj.finish_output)
    rope_positions, flat_positions = layer._positions_for_runtime(positions)
    session = layer.begin_streamed_prefill(positions)
    spans = [(s, min(length, s + slice_tokens)) for s in range(0, length, slice_tokens)]
    calls = proj.calls
    for s, e in spans:
        session.keys(layer._slice_positions(rope_positions, s, e), h[s:e], s, e)
    session.ingest()
    got = torch.empty_like(want)
    for s, e in spans:
        got[s:e] = session.queries(layer._slice_positions(rope_positions, s, e), flat_positions[s:e],
                                   h[s:e], s)
    session.finish()
    torch.cuda.synchronize()
    assert proj.calls - calls == 2 * len(spans)        # one projection per slice and pass
    assert torch.equal(got.cpu(), want.cpu())
    assert layer.arena is not None


def test_token_order_session_driven_by_hidden_states():
    """The reference's token-order call (TokenOuterPrefillSession.slice, token_outer_prefill.py:
    173-196): slice(hidden, s, e) per slice, the rotary positions taken from the session's
    prompt positions.  The output rows equal the projection-taking path's, gated and
    projected out, bit for bit, before and after the fit."""
    length, chunk = 4096, 512
    proj = _Projections(seed=1)
    h = _hidden(length, seed=8)
    flat = torch.arange(length, device=DEV)
    q_post, k_post, v, q_pre, k_pre, gate = proj.project_qkv(flat, h)
    base = _layer("test.token.hidden.base", chunk=chunk)
    attn = torch.empty(length, 8 * 128, dtype=torch.bfloat16, device=DEV)
    base.prefill_token_order(q_post, q_pre, k_pre, k_post, v, attn, chunk, fit_tokens=1024)
    want = proj.finish_output(attn, gate)

    layer = _layer("test.token.hidden", chunk=chunk)
    layer.attach_projections(proj.project_qkv, proj.finish_output)
    session = layer.begin_token_outer_prefill(flat, chunk, fit_tokens=1024)
    got = torch.empty_like(want)
    for s in range(0, length, chunk):
        e = min(length, s + chunk)
        got[s:e] = session.slice(h[s:e], s, e)
    session.finish()
    torch.cuda.synchronize()
    assert session.fit_at < length                       # slices on both sides of the fit
    assert torch.equal(got.cpu(), want.cpu())
