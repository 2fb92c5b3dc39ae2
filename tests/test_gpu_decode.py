"""S7-S9 on the GPU: the sparse decode step (suffix write, routing, selection against
the full cluster sizes, split attention over the prompt CSR and the suffix, merge).

Attention is checked against fp64 over exactly the selected clusters' rows plus
the visible suffix (as tests/test_fused_decode_v3.py:98-124 of the reference
does), selection against the oracle's up to near-ties, and the step captured
in a HIP graph against the same steps run eagerly (bit-exact).
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import assert_close_bf16, compare_selection, oracle_select
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _Layer:
    def __init__(self, hq, hkv, d):
        self.num_heads, self.num_kv_heads, self.head_dim = hq, hkv, d


def _setup(length, hq, hkv, d, seed, reserve=512, shuffle=True):
    from semblo_amd.arena import DecodeArena
    from semblo_amd.state import ProductPostingIndex
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(length, hq, hkv, d, mixtures=32, seg=(32, 256), seed=seed)
    k, v = inp.k.to(DEV), inp.v.to(DEV)
    idx = ProductPostingIndex.build(k, torch.arange(length, device=DEV), codebook_seed=seed,
                                    router_pass=True)
    idx.pack_prompt_kv(k, v)
    gen = torch.Generator().manual_seed(seed) if shuffle else None
    arena = DecodeArena(idx, reserve=reserve, shuffle_blocks=gen)
    return inp, idx, arena


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


@pytest.mark.parametrize("cfg", [dict(length=4096, hq=16, hkv=4, d=256, seed=1),
                                 dict(length=3000, hq=8, hkv=2, d=128, seed=2),
                                 dict(length=2048, hq=8, hkv=1, d=128, seed=3),      # G = 8
                                 dict(length=2048, hq=4, hkv=4, d=256, seed=4),      # G = 1
                                 # two prompt splits and one suffix split per head and a large budget: each
                                 # split takes its rows in two rounds (384 rows at D = 128,
                                 # 192 at D = 256)
                                 dict(length=4096, hq=8, hkv=2, d=128, seed=6, splits=2, suffix_splits=1, target=2048),
                                 dict(length=4096, hq=16, hkv=4, d=256, seed=7, splits=2, suffix_splits=1, target=1024),
                                 # a budget of the whole prompt selects every live cluster: the
                                 # reference's dense decode case (tests/test_dense_prompt_decode.py),
                                 # here through the same step
                                 dict(length=2048, hq=8, hkv=2, d=128, seed=8, target=2048),
                                 dict(length=1000, hq=16, hkv=4, d=256, seed=9, target=4096)])
def test_decode_steps_match_fp64_over_selection_and_suffix(cfg):
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.synthetic import decode_queries
    length, hq, hkv, d = cfg["length"], cfg["hq"], cfg["hkv"], cfg["d"]
    inp, idx, arena = _setup(length, hq, hkv, d, cfg["seed"])
    steps = 40
    qs, kn, vn = decode_queries(inp, steps, hq, seed=cfg["seed"])
    layer = _Layer(hq, hkv, d)
    target = cfg.get("target", length // 16)
    splits = cfg.get("splits", 16)
    c = idx.num_buckets
    csr = torch.empty(3 * hkv * c + 2 * hkv, dtype=torch.int32, device=DEV)
    out = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(hq, dtype=torch.float32, device=DEV)
    packed = idx.packed_kv.cpu()
    near = 0
    for t in range(steps):
        pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
        q = qs[t:t + 1].to(DEV)
        fused_decode_step(layer, arena, q_post=q, q_pre=q, positions=pos, k_post=kn[t:t + 1].to(DEV),
                          v_states=vn[t:t + 1].to(DEV), output=out, temperature=0.1, beta=0.25,
                          target_tokens=target, sm_scale=d ** -0.5, num_splits=splits, iters=16,
                          suffix_splits=cfg.get("suffix_splits"), out_lse=lse, csr_out=csr)
        torch.cuda.synchronize()
        sel = _csr_to_sel(csr.cpu(), idx)
        want, want_lse = ref.decode_reference(q[0].cpu(), packed, idx.bucket_indptr.cpu(),
                                              idx.bucket_sizes.cpu(), sel, kn[:t + 1].cpu(),
                                              vn[:t + 1].cpu(), d ** -0.5, with_lse=True)
        assert_close_bf16(out.view(hq, d).cpu(), want, f"step {t}")
        # natural-log LSE of the scaled scores, the merge's convention; the reference's
        # tolerance (tests/test_dense_prompt_decode.py:64)
        torch.testing.assert_close(lse.cpu().double(), want_lse, atol=2e-3, rtol=1e-4)
        if target >= length:
            assert torch.equal(sel, idx.bucket_sizes.cpu() > 0), "a whole-prompt budget selects every cluster"
        vec = ref.trivial_router_vectors(q.cpu(), 1)
        exp = oracle_select(vec, idx.codebooks.cpu(), idx.bucket_sizes.cpu()[None],
                            temperature=0.1, beta=0.25, target=target)
        rep = compare_selection(sel[None], exp["sel"], exp["score"], exp["theta"])
        near += rep["near_ties"]
        # the suffix store holds every generated token at its table slot
        ks, vs = arena.suffix_rows(torch.arange(length, length + t + 1), 0)
        assert torch.equal(ks.cpu(), kn[:t + 1, 0].cpu())
    print(f"{cfg}: {steps} steps, {near} near-tie selection differences")


def test_decode_step_replays_in_a_hip_graph():
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.synthetic import decode_queries
    length, hq, hkv, d = 4096, 16, 4, 256
    layer = _Layer(hq, hkv, d)
    inp, idx_a, arena_a = _setup(length, hq, hkv, d, 5, shuffle=False)
    _, idx_b, arena_b = _setup(length, hq, hkv, d, 5, shuffle=False)
    steps = 12
    qs, kn, vn = decode_queries(inp, steps, hq, seed=5)
    kw = dict(temperature=0.1, beta=0.25, target_tokens=length // 16, sm_scale=d ** -0.5,
              num_splits=32, iters=16)
    # eager reference run
    eager = []
    out = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    for t in range(steps):
        pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
        fused_decode_step(layer, arena_a, q_post=qs[t:t + 1].to(DEV), q_pre=qs[t:t + 1].to(DEV),
                          positions=pos, k_post=kn[t:t + 1].to(DEV), v_states=vn[t:t + 1].to(DEV),
                          output=out, **kw)
        eager.append(out.clone())
    # captured run: static inputs, one capture, replays with eager work in between
    s_q = torch.empty(1, hq, d, dtype=torch.bfloat16, device=DEV)
    s_k = torch.empty(1, hkv, d, dtype=torch.bfloat16, device=DEV)
    s_v = torch.empty(1, hkv, d, dtype=torch.bfloat16, device=DEV)
    s_pos = torch.tensor([length], dtype=torch.int32, device=DEV)
    s_out = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    s_q.copy_(qs[0:1])
    s_k.copy_(kn[0:1])
    s_v.copy_(vn[0:1])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):       # warm-up allocates the workspace outside the capture
        fused_decode_step(layer, arena_b, q_post=s_q, q_pre=s_q, positions=s_pos, k_post=s_k,
                          v_states=s_v, output=s_out, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fused_decode_step(layer, arena_b, q_post=s_q, q_pre=s_q, positions=s_pos, k_post=s_k,
                          v_states=s_v, output=s_out, **kw)
    for t in range(steps):
        s_q.copy_(qs[t:t + 1])
        s_k.copy_(kn[t:t + 1])
        s_v.copy_(vn[t:t + 1])
        s_pos.fill_(length + t)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(s_out, eager[t]), f"replay {t} differs from the eager step"


def test_layer_decode_refuses_a_step_past_the_suffix_reserve():
    """The suffix store holds suffix_reserve generated positions; the layer's decode
    refuses the step after them instead of dropping its token (counted on the host)."""
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    from semblo_amd.synthetic import decode_queries, mixture_layer
    length, hq, hkv, d, reserve = 1024, 8, 2, 128, 32
    cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=512,
                              suffix_reserve=reserve)
    layer = SembloAttention(cfg, layer_name="test.decode.reserve")
    inp = mixture_layer(length, hq, hkv, d, mixtures=16, seed=8)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    out = torch.empty(length, hq * d, dtype=torch.bfloat16, device=DEV)
    layer.prefill(q, q, k, k, v, out)
    qs, kn, vn = decode_queries(inp, reserve + 1, hq, seed=8)
    dec = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    for t in range(reserve):
        pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
        layer.decode(pos, qs[t:t + 1].to(DEV), qs[t:t + 1].to(DEV), kn[t:t + 1].to(DEV),
                     vn[t:t + 1].to(DEV), dec)
    torch.cuda.synchronize()
    pos = torch.tensor([length + reserve], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="suffix_reserve"):
        layer.decode(pos, qs[-1:].to(DEV), qs[-1:].to(DEV), kn[-1:].to(DEV), vn[-1:].to(DEV), dec)


def _csr_to_arena_sel(csr, arena):
    """[Hkv, C_arena] bool: the clusters of the arena whose runs the step's CSR names."""
    hkv, c = arena.sizes.shape
    n = hkv * c
    rstart = csr[:n].view(hkv, c)
    rcount = csr[3 * n:3 * n + hkv]
    indptr, sizes = arena.indptr.cpu(), arena.sizes.cpu()
    sel = torch.zeros(hkv, c, dtype=torch.bool)
    for h in range(hkv):
        for p in range(int(rcount[h])):
            cand = torch.nonzero((indptr[h, :-1] == int(rstart[h, p])) & (sizes[h] > 0)).flatten()
            assert cand.numel() == 1
            sel[h, cand[0]] = True
    return sel


def test_capacity_arena_step_captured_before_any_request_replays_for_each():
    """vLLM's FULL graph mode (arena.py:1-27 of the reference): the step is captured
    once, on a capacity-shaped arena holding a one-token index, before any request.
    Each request's index is then adopted into the same buffers (one with fewer clusters
    than the arena: its tail clusters are empty, with zero descriptors), and the same
    graph, fed through fixed input buffers, runs every step: the same bits as the step
    run eagerly, fp64 attention over the CSR's clusters and the suffix, natural-log LSE,
    and the selection of the oracle over the arena's padded descriptors and sizes."""
    from semblo_amd.arena import DecodeArena
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.state import ProductPostingIndex
    from semblo_amd.synthetic import decode_queries, mixture_layer
    hq, hkv, d, cap, ncl, target = 8, 2, 128, 4096, 128, 256
    layer = _Layer(hq, hkv, d)
    arena = DecodeArena.with_capacity(capacity=cap, num_kv_heads=hkv, head_dim=d, num_clusters=ncl,
                                      reserve=512, suffix_splits=4, device=DEV)
    bf = torch.bfloat16
    qb = torch.zeros(1, hq, d, dtype=bf, device=DEV)
    kb = torch.zeros(1, hkv, d, dtype=bf, device=DEV)
    vb = torch.zeros(1, hkv, d, dtype=bf, device=DEV)
    pos = torch.full((1,), cap, dtype=torch.int32, device=DEV)
    out = torch.empty(1, hq * d, dtype=bf, device=DEV)
    lse = torch.empty(hq, dtype=torch.float32, device=DEV)
    csr = torch.empty(3 * hkv * ncl + 2 * hkv, dtype=torch.int32, device=DEV)

    def step():
        fused_decode_step(layer, arena, q_post=qb, q_pre=qb, positions=pos, k_post=kb, v_states=vb,
                          output=out, temperature=0.1, beta=0.25, target_tokens=target,
                          sm_scale=d ** -0.5, num_splits=16, iters=16, out_lse=lse, csr_out=csr)

    step()                                   # warm-up on the one-token index: makes the workspace
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for length, seed, min_log2 in ((3000, 21, 3), (2048, 22, 7)):
        inp = mixture_layer(length, hq, hkv, d, mixtures=32, seg=(32, 256), seed=seed)
        k, v = inp.k.to(DEV), inp.v.to(DEV)
        idx = ProductPostingIndex.build(k, torch.arange(length, device=DEV), codebook_seed=seed,
                                        router_pass=True, flat_min_clusters_log2=min_log2)
        idx.pack_prompt_kv(k, v)
        assert idx.num_buckets <= ncl
        arena.adopt(idx)
        assert int(arena.prompt_length_t.item()) == length
        qs, kn, vn = decode_queries(inp, 6, hq, seed=seed)
        for t in range(6):
            qb.copy_(qs[t:t + 1].to(DEV))
            kb.copy_(kn[t:t + 1].to(DEV))
            vb.copy_(vn[t:t + 1].to(DEV))
            pos.fill_(length + t)
            graph.replay()
            torch.cuda.synchronize()
            got, got_lse, got_csr = out.clone(), lse.clone(), csr.clone()
            step()                            # the same step, eagerly
            torch.cuda.synchronize()
            assert torch.equal(got, out) and torch.equal(got_lse, lse) and torch.equal(got_csr, csr)
            sel = _csr_to_arena_sel(got_csr.cpu(), arena)
            assert not bool(sel[:, idx.num_buckets:].any())
            want, want_lse = ref.decode_reference(qs[t].cpu(), arena.packed_kv.cpu(), arena.indptr.cpu(),
                                                  arena.sizes.cpu(), sel, kn[:t + 1].cpu(), vn[:t + 1].cpu(),
                                                  d ** -0.5, with_lse=True)
            assert_close_bf16(got.view(hq, d).cpu(), want, f"L={length} step {t}")
            torch.testing.assert_close(got_lse.cpu().double(), want_lse, atol=2e-3, rtol=1e-4)
            vec = ref.trivial_router_vectors(qs[t:t + 1].cpu(), 1)
            exp = oracle_select(vec, arena.codebooks.cpu(), arena.sizes.cpu()[None], temperature=0.1,
                                beta=0.25, target=target)
            compare_selection(sel[None], exp["sel"], exp["score"], exp["theta"])


def test_layer_decodes_two_requests_on_its_capacity_arena():
    """A layer with decode_capacity keeps one arena across requests: each prefill's index
    is adopted into it (here 64 clusters into an arena of 128), nothing moves, and the
    layer's decode steps select on the capacity budget rule (an explicit target here):
    the same bits as the step run directly, fp64 over the CSR's clusters and the suffix."""
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.model import SembloAttention
    from semblo_amd.synthetic import decode_queries, mixture_layer
    hq, hkv, d = 8, 2, 128
    cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=512,
                              target_tokens=256, flat_min_clusters_log2=3, decode_capacity=262144,
                              suffix_reserve=64)
    layer = SembloAttention(cfg, layer_name="test.decode.capacity")
    arena = layer.capacity_arena(DEV)
    assert arena.num_clusters == 128
    ptrs = [t.data_ptr() for t in (arena.codebooks, arena.sizes, arena.indptr, arena.packed_kv,
                                   arena.suffix_kv, arena.suffix_table)]
    assert layer.decode_budget() == 256
    c = arena.num_clusters
    csr = torch.empty(3 * hkv * c + 2 * hkv, dtype=torch.int32, device=DEV)
    for length, seed in ((4096, 31), (2048, 32)):
        inp = mixture_layer(length, hq, hkv, d, mixtures=16, seed=seed)
        q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
        out = torch.empty(length, hq * d, dtype=torch.bfloat16, device=DEV)
        layer.prefill(q, q, k, k, v, out)
        assert layer.arena is arena and layer.index.num_buckets == 64
        assert [t.data_ptr() for t in (arena.codebooks, arena.sizes, arena.indptr, arena.packed_kv,
                                       arena.suffix_kv, arena.suffix_table)] == ptrs
        qs, kn, vn = decode_queries(inp, 5, hq, seed=seed)
        dec = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
        again = torch.empty_like(dec)
        for t in range(5):
            pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
            qt, kt, vt = qs[t:t + 1].to(DEV), kn[t:t + 1].to(DEV), vn[t:t + 1].to(DEV)
            layer.decode(pos, qt, qt, kt, vt, dec)
            fused_decode_step(layer, arena, q_post=qt, q_pre=qt, positions=pos, k_post=kt, v_states=vt,
                              output=again, temperature=cfg.selection_temperature,
                              beta=cfg.bucket_size_penalty, target_tokens=layer.decode_budget(),
                              sm_scale=layer.scaling, num_splits=cfg.decode_num_splits, iters=cfg.iters,
                              suffix_splits=cfg.decode_suffix_splits, csr_out=csr)
            torch.cuda.synchronize()
            assert torch.equal(dec, again)
            sel = _csr_to_arena_sel(csr.cpu(), arena)
            assert not bool(sel[:, 64:].any())
            want = ref.decode_reference(qs[t].cpu(), arena.packed_kv.cpu(), arena.indptr.cpu(),
                                        arena.sizes.cpu(), sel, kn[:t + 1].cpu(), vn[:t + 1].cpu(),
                                        d ** -0.5)
            assert_close_bf16(dec.view(hq, d).cpu(), want, f"L={length} step {t}")
