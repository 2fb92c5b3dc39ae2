"""The reference's inner seams that the HIP build replaces, each called directly:

  build_reverse_index / sbsa_reverse_index   kv_outer.py:254-329    against ref.reverse_index
  fused_chunk_attention (one call)           fused_prefill.py:219-482
  fused_decode_attention (out + LSE)         fused_prefill.py:625-718
  merge_paged_attention_results              paged_attention.py:50-80
  flat_mixture_scores_qtiled                 fused_select.py:1250-1357
"""
from __future__ import annotations

from pathlib import Path

import pytest
import torch

from gpu_util import (assert_close_bf16, check_recorded_chunk, compare_selection,
                      oracle_select)
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
DEV = "cuda"


@pytest.mark.parametrize("q,hkv,c,density", [(700, 4, 128, 0.07), (1, 2, 64, 0.5),
                                             (333, 1, 256, 0.0), (2048, 2, 1024, 0.01)])
def test_reverse_index_matches_the_oracle(q, hkv, c, density):
    """The CSR transpose of the per-query masks, bit for bit: counts, row starts and the
    ascending query lists; each query's rank points back at itself.  Clusters with no
    visible rows are left out (the reference's ``live``)."""
    from semblo_amd.kv_outer import build_reverse_index
    gen = torch.Generator().manual_seed(q + c)
    sel = torch.rand(q, hkv, c, generator=gen) < density
    live = torch.randint(0, 3, (hkv, c), generator=gen, dtype=torch.int32)   # 0: dead
    qmask = ref.pack_bits(sel)
    qvals, counts, indptr, nnz, qrank = build_reverse_index(qmask.to(DEV), live.to(DEV),
                                                            num_queries=q)
    torch.cuda.synchronize()
    want_counts, want_indptr, want_qvals = ref.reverse_index(sel, live > 0)
    n = int(nnz.item())
    assert n == int(want_indptr[-1])
    assert torch.equal(counts.cpu(), want_counts)
    assert torch.equal(indptr.cpu().long(), want_indptr)
    assert torch.equal(qvals[:n].cpu(), want_qvals)
    m = sel & (live > 0)[None]
    qi, h, cl = torch.nonzero(m, as_tuple=True)
    slot = want_indptr[h * c + cl] + qrank.cpu()[qi, h, cl].long()
    assert torch.equal(want_qvals[slot].long(), qi)
    print(f"Q={q} Hkv={hkv} C={c}: {n} entries")


def _layer_index(length, hq, hkv, d, seed):
    from semblo_amd.state import ProductPostingIndex
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(length, hq, hkv, d, mixtures=32, seg=(32, 256), seed=seed)
    k, v = inp.k.to(DEV), inp.v.to(DEV)
    idx = ProductPostingIndex.build(k, torch.arange(length, device=DEV), codebook_seed=seed,
                                    router_pass=True)
    idx.pack_prompt_kv(k, v)
    idx.original_kv = (k, v)
    return inp, idx


@pytest.mark.parametrize("cs", [1024, 2560])
def test_fused_chunk_attention_in_one_call(cs):
    """The seam as the reference calls it: a dense-prefix chunk (cs <= 4K) and a sparse
    chunk, each one call; the sparse one against fp64 over its recorded key sets."""
    from semblo_amd.fused_prefill import CausalSnapshot, fused_chunk_attention
    from semblo_amd.model import SembloQueryState
    from semblo_amd.trivial_router import trivial_router_vectors
    length, hq, hkv, d = 4096, 8, 2, 128
    inp, idx = _layer_index(length, hq, hkv, d, seed=41)
    target = 256
    ce = cs + 511
    q = inp.q.to(DEV)
    qc = q[cs:ce + 1]
    vec = trivial_router_vectors(qc, 1)
    qs = SembloQueryState(vec.view(1, *vec.shape[:2], 1, d),
                          torch.ones(1, vec.shape[0], hq, 1, device=DEV))
    log = []
    out = fused_chunk_attention(qc, qs, idx, torch.arange(cs, ce + 1, device=DEV),
                                CausalSnapshot(idx), cs, ce, temperature=0.1, beta=0.25,
                                target_tokens=target, sm_scale=d ** -0.5, plan_log=log)
    torch.cuda.synchronize()
    full = torch.zeros(length, hq, d, dtype=torch.bfloat16)
    full[cs:ce + 1] = out.cpu()
    if cs <= 4 * target:
        assert not log
        p = torch.arange(cs, ce + 1)
        keys = (torch.arange(length)[None, :] <= p[:, None])[:, None, :].expand(-1, hkv, -1)
        from gpu_util import attention_reference
        want = attention_reference(inp.q[cs:ce + 1], keys, inp.k, inp.v, d ** -0.5)
        assert_close_bf16(out.cpu(), want, "dense chunk")
    else:
        assert len(log) == 1
        rep = check_recorded_chunk(log[0], inp.q, inp.q, inp.k, inp.v, idx, full, target=target,
                                   tag="one call")
        print(f"chunk {cs}: {rep}")


def _csr_sel(csr, idx):
    from test_gpu_decode import _csr_to_sel
    return _csr_to_sel(csr.cpu(), idx)


def test_fused_decode_attention_returns_out_and_lse():
    """fused_decode_attention: one query over the packed prompt, selection against the full
    cluster sizes; the output and its natural-log LSE against fp64 over the GPU's own
    selection (itself against the oracle's up to near-ties)."""
    from semblo_amd.fused_prefill import fused_decode_attention
    from semblo_amd.model import SembloQueryState
    from semblo_amd.synthetic import decode_queries
    from semblo_amd.trivial_router import trivial_router_vectors
    length, hq, hkv, d = 4096, 16, 4, 256
    inp, idx = _layer_index(length, hq, hkv, d, seed=43)
    qs, _, _ = decode_queries(inp, 4, hq, seed=1)
    c = idx.num_buckets
    packed = idx.packed_kv.cpu()
    empty = torch.zeros(0, hkv, d)
    for t in range(4):
        q = qs[t:t + 1].to(DEV)
        vec = trivial_router_vectors(q, 1)
        state = SembloQueryState(vec.view(1, 1, hq, 1, d), torch.ones(1, 1, hq, 1, device=DEV))
        csr = torch.empty(3 * hkv * c + 2 * hkv, dtype=torch.int32, device=DEV)
        res = fused_decode_attention(q, state, idx, torch.tensor([length], device=DEV),
                                     temperature=0.1, beta=0.25, target_tokens=256,
                                     sm_scale=d ** -0.5, csr_out=csr)
        torch.cuda.synchronize()
        sel = _csr_sel(csr, idx)
        exp = oracle_select(ref.trivial_router_vectors(q.cpu(), 1), idx.codebooks.cpu(),
                            idx.bucket_sizes.cpu()[None], temperature=0.1, beta=0.25, target=256)
        compare_selection(sel[None], exp["sel"], exp["score"], exp["theta"])
        want, lse = ref.decode_reference(q[0].cpu(), packed, idx.bucket_indptr.cpu(),
                                         idx.bucket_sizes.cpu(), sel, empty, empty, d ** -0.5,
                                         with_lse=True)
        assert res.output.shape == (1, hq, d) and res.logsumexp.shape == (1, hq)
        assert_close_bf16(res.output[0].cpu(), want, f"decode query {t}")
        assert torch.allclose(res.logsumexp[0].cpu().double(), lse, rtol=1e-4, atol=1e-3), \
            (res.logsumexp[0].cpu(), lse)


def test_merge_paged_attention_results_is_the_attention_of_the_union():
    """Attention over two disjoint key sets merged by LSE equals the attention over their
    union (fp64), and the merge matches the oracle's closed form."""
    from semblo_amd.fused_prefill import PagedSparseAttentionResult, merge_paged_attention_results
    gen = torch.Generator().manual_seed(7)
    hq, d, n = 8, 128, 900
    q = torch.randn(hq, d, generator=gen)
    k = torch.randn(n, d, generator=gen)
    v = torch.randn(n, d, generator=gen)
    split = torch.rand(n, generator=gen) < 0.3
    k[split] *= 2.0                                 # the two sides carry different LSEs

    def attend(mask):
        s = (q.double() @ k[mask].double().T) * d ** -0.5
        return torch.softmax(s, -1) @ v[mask].double(), torch.logsumexp(s, -1)

    oa, la = attend(split)
    ob, lb = attend(~split)
    ou, lu = attend(torch.ones(n, dtype=torch.bool))
    a = PagedSparseAttentionResult(oa.to(torch.bfloat16)[None].to(DEV), la.float()[None].to(DEV))
    b = PagedSparseAttentionResult(ob.to(torch.bfloat16)[None].to(DEV), lb.float()[None].to(DEV))
    m = merge_paged_attention_results(a, b)
    assert m.output.dtype == torch.bfloat16
    assert_close_bf16(m.output[0].cpu(), ou, "merged")
    assert torch.allclose(m.logsumexp[0].cpu().double(), lu, atol=1e-5)
    mo, ml = ref.lse_merge(a.output.cpu(), a.logsumexp.cpu(), b.output.cpu(), b.logsumexp.cpu())
    assert torch.allclose(m.logsumexp.cpu().double(), ml, atol=1e-6)
    assert_close_bf16(m.output.cpu(), mo, "merged vs oracle")
    with pytest.raises(ValueError):
        merge_paged_attention_results(a, PagedSparseAttentionResult(b.output, None))


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("select_*.pt")))
def test_flat_mixture_scores_qtiled(name):
    """The scorer alone: [Q, Hkv, C] mixture probabilities against the reference's
    torch-form values (golden) and the oracle."""
    from semblo_amd.fused_select import flat_mixture_scores_qtiled
    g = torch.load(GOLDEN / name, weights_only=True)
    q, hq, d = g["vectors"].shape
    prob = flat_mixture_scores_qtiled(g["vectors"].to(DEV).view(q, hq, 1, d), None,
                                      g["codebooks"].to(DEV), temperature=float(g["tau"])).cpu()
    assert prob.shape == g["prob"].shape
    assert torch.allclose(prob, g["prob"], rtol=2e-4, atol=1e-6)
    mine = ref.mixture_probs(g["vectors"], None, g["codebooks"], float(g["tau"]))
    assert torch.allclose(prob, mine.float(), rtol=2e-4, atol=1e-6)
