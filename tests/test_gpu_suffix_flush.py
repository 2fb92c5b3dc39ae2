"""The suffix flush on the GPU (semblo/vllm_plugin/suffix_flush.py): generated tokens
move from the exact suffix into the clusters every `every` steps, keeping the newest
`keep` exact.

After every flush the arena's store is checked against the oracle's layout
(oracle.flush_store: each cluster's old rows, then its newcomers in position order,
runs page-aligned), with the newcomers' clusters against the oracle's nearest
cluster up to fp32 near-ties; every decode step's output against fp64 attention over
the selected clusters of the flushed store plus the exact suffix from the moved-up
prompt length; and a captured step replayed across flushes against the same steps
run eagerly (bit-exact).  Tolerance: 2e-2 abs + 1e-2 rel (bf16).
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import assert_close_bf16, compare_selection, oracle_select
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
NEAR_REL = 1e-4


class _Layer:
    def __init__(self, hq, hkv, d):
        self.num_heads, self.num_kv_heads, self.head_dim = hq, hkv, d


def _setup(length, hq, hkv, d, seed, reserve, room, shuffle=True):
    from semblo_amd.arena import DecodeArena
    from semblo_amd.state import ProductPostingIndex
    from semblo_amd.synthetic import mixture_layer
    inp = mixture_layer(length, hq, hkv, d, mixtures=32, seg=(32, 256), seed=seed)
    k, v = inp.k.to(DEV), inp.v.to(DEV)
    idx = ProductPostingIndex.build(k, torch.arange(length, device=DEV), codebook_seed=seed,
                                    router_pass=True)
    idx.pack_prompt_kv(k, v)
    gen = torch.Generator().manual_seed(seed) if shuffle else None
    arena = DecodeArena(idx, reserve=reserve, shuffle_blocks=gen, flush_room=room)
    return inp, idx, arena


def _csr_to_sel(csr, arena):
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


def _check_store(arena, state, keys_all, v_all, frm, to, align):
    """The arena after moving positions [frm, to) against the oracle's layout; returns the
    number of newcomers whose cluster is an fp32 near-tie away from the oracle's."""
    from semblo_amd.token_outer_prefill import nearest_cluster
    hkv = arena.sizes.shape[0]
    kp = keys_all[frm:to].to(DEV)
    got = nearest_cluster(kp, arena.codebooks).cpu()                   # the flush's kernel
    near = 0
    for h in range(hkv):
        want, sim = ref.nearest_cluster(keys_all[frm:to, h], arena.codebooks[h].cpu(), return_sim=True)
        for i in torch.nonzero(got[h].long() != want).flatten().tolist():
            a, b = float(sim[i, want[i]]), float(sim[i, got[h, i]])
            assert abs(a - b) <= NEAR_REL * max(abs(a), 1e-6), (h, i, a, b)
            near += 1
    runs, sizes, indptr = ref.flush_store(state["posting"], state["indptr"], state["sizes"], got.long(),
                                          frm, align)
    assert torch.equal(arena.sizes.cpu().long(), sizes)
    assert torch.equal(arena.indptr.cpu().long(), indptr)
    posting = arena.posting.cpu()
    packed = arena.packed_kv.cpu()
    new_posting = torch.full_like(posting, -1)
    for h in range(hkv):
        for b, lst in enumerate(runs[h]):
            st = int(indptr[h, b])
            row = posting[h, st:st + len(lst)]
            assert row.tolist() == lst, (h, b)
            new_posting[h, st:st + len(lst)] = row
            if lst:
                pos = torch.tensor(lst)
                assert torch.equal(packed[0, st:st + len(lst), h], keys_all[pos, h])
                assert torch.equal(packed[1, st:st + len(lst), h], v_all[pos, h])
    state.update(posting=new_posting, sizes=sizes, indptr=indptr)
    return near


@pytest.mark.parametrize("cfg", [dict(length=2048, hq=8, hkv=2, d=128, seed=21, keep=48, every=32),
                                 dict(length=3000, hq=16, hkv=4, d=256, seed=22, keep=64, every=40)])
def test_decode_with_suffix_flush_matches_fp64_and_the_oracle_store(cfg):
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.suffix_flush import maybe_flush
    from semblo_amd.synthetic import decode_queries
    length, hq, hkv, d = cfg["length"], cfg["hq"], cfg["hkv"], cfg["d"]
    keep, every = cfg["keep"], cfg["every"]
    inp, idx, arena = _setup(length, hq, hkv, d, cfg["seed"], reserve=512, room=1024)
    steps = 200
    qs, kn, vn = decode_queries(inp, steps, hq, seed=cfg["seed"])
    keys_all = torch.cat([inp.k.cpu(), kn.cpu()])                      # pre-RoPE = post here
    v_all = torch.cat([inp.v.cpu(), vn.cpu()])
    layer = _Layer(hq, hkv, d)
    target = length // 16
    c = idx.num_buckets
    csr = torch.empty(3 * hkv * c + 2 * hkv, dtype=torch.int32, device=DEV)
    out = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    state = dict(posting=arena.posting.cpu(), sizes=arena.sizes.cpu(), indptr=arena.indptr.cpu())
    flushes, near_ids, near_sel = 0, 0, 0
    for t in range(steps):
        rng = maybe_flush(arena, keep, every)
        if rng is not None:
            torch.cuda.synchronize()
            near_ids += _check_store(arena, state, keys_all, v_all, rng[0], rng[1], arena.page_align)
            assert int(arena.prompt_length_t.item()) == rng[1] == arena.prompt_length
            flushes += 1
        arena.steps += 1
        pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
        q = qs[t:t + 1].to(DEV)
        fused_decode_step(layer, arena, q_post=q, q_pre=q, positions=pos, k_post=kn[t:t + 1].to(DEV),
                          v_states=vn[t:t + 1].to(DEV), k_pre=kn[t:t + 1].to(DEV), output=out,
                          temperature=0.1, beta=0.25, target_tokens=target, sm_scale=d ** -0.5,
                          num_splits=16, iters=16, csr_out=csr)
        torch.cuda.synchronize()
        sel = _csr_to_sel(csr.cpu(), arena)
        plen = arena.prompt_length
        want = ref.decode_reference(q[0].cpu(), arena.packed_kv.cpu(), arena.indptr.cpu(),
                                    arena.sizes.cpu(), sel, kn[plen - length:t + 1].cpu(),
                                    vn[plen - length:t + 1].cpu(), d ** -0.5)
        assert_close_bf16(out.view(hq, d).cpu(), want, f"step {t}")
        vec = ref.trivial_router_vectors(q.cpu(), 1)
        exp = oracle_select(vec, arena.codebooks.cpu(), arena.sizes.cpu()[None], temperature=0.1,
                            beta=0.25, target=target)
        near_sel += compare_selection(sel[None], exp["sel"], exp["score"], exp["theta"])["near_ties"]
    assert flushes == (steps - 1 - (keep + every)) // every + 1
    print(f"{cfg}: {flushes} flushes, {near_ids} near-tie cluster ids, {near_sel} near-tie selections")


def test_captured_step_replays_across_flushes():
    """Every address the step reads is fixed and the prompt length is read on the device,
    so one capture replays correctly while flushes move tokens between replays."""
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.suffix_flush import maybe_flush
    from semblo_amd.synthetic import decode_queries
    length, hq, hkv, d, keep, every = 2048, 8, 2, 128, 40, 24
    layer = _Layer(hq, hkv, d)
    inp, _, arena_a = _setup(length, hq, hkv, d, 23, reserve=512, room=1024, shuffle=False)
    _, _, arena_b = _setup(length, hq, hkv, d, 23, reserve=512, room=1024, shuffle=False)
    steps = 120
    qs, kn, vn = decode_queries(inp, steps, hq, seed=23)
    kw = dict(temperature=0.1, beta=0.25, target_tokens=length // 16, sm_scale=d ** -0.5,
              num_splits=16, iters=16)
    eager = []
    out = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    for t in range(steps):
        maybe_flush(arena_a, keep, every)
        arena_a.steps += 1
        pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
        fused_decode_step(layer, arena_a, q_post=qs[t:t + 1].to(DEV), q_pre=qs[t:t + 1].to(DEV),
                          positions=pos, k_post=kn[t:t + 1].to(DEV), v_states=vn[t:t + 1].to(DEV),
                          k_pre=kn[t:t + 1].to(DEV), output=out, **kw)
        eager.append(out.clone())
    s_q = qs[0:1].to(DEV).clone()
    s_k = kn[0:1].to(DEV).clone()
    s_v = vn[0:1].to(DEV).clone()
    s_pos = torch.tensor([length], dtype=torch.int32, device=DEV)
    s_out = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):       # warm-up allocates the workspace outside the capture
        fused_decode_step(layer, arena_b, q_post=s_q, q_pre=s_q, positions=s_pos, k_post=s_k,
                          v_states=s_v, k_pre=s_k, output=s_out, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fused_decode_step(layer, arena_b, q_post=s_q, q_pre=s_q, positions=s_pos, k_post=s_k,
                          v_states=s_v, k_pre=s_k, output=s_out, **kw)
    moved = 0
    for t in range(steps):
        if maybe_flush(arena_b, keep, every) is not None:
            moved += 1
        arena_b.steps += 1
        s_q.copy_(qs[t:t + 1])
        s_k.copy_(kn[t:t + 1])
        s_v.copy_(vn[t:t + 1])
        s_pos.fill_(length + t)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(s_out, eager[t]), f"replay {t} differs from the eager step"
    assert moved == arena_a.flushes == (steps - 1 - (keep + every)) // every + 1


def test_layer_decode_flushes_under_the_environment(monkeypatch):
    """SEMBLO_SUFFIX_FLUSH_EVERY through the layer: a generation longer than the suffix
    store runs (the store holds only the exact suffix), and the arena's prompt length
    advanced on the host and on the device alike."""
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    from semblo_amd.synthetic import decode_queries, mixture_layer
    monkeypatch.setenv("SEMBLO_SUFFIX_FLUSH_EVERY", "64")
    monkeypatch.setenv("SEMBLO_SUFFIX_KEEP_EXACT", "128")
    monkeypatch.setenv("SEMBLO_SUFFIX_FLUSH_ROOM", "2048")
    length, hq, hkv, d, reserve = 1024, 8, 2, 128, 768
    cfg = SembloRuntimeConfig(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, query_chunk_size=512,
                              suffix_reserve=reserve)
    layer = SembloAttention(cfg, layer_name="test.flush.env")
    inp = mixture_layer(length, hq, hkv, d, mixtures=16, seed=24)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    out = torch.empty(length, hq * d, dtype=torch.bfloat16, device=DEV)
    layer.prefill(q, q, k, k, v, out)
    steps = reserve + 200
    qs, kn, vn = decode_queries(inp, steps, hq, seed=24)
    dec = torch.empty(1, hq * d, dtype=torch.bfloat16, device=DEV)
    for t in range(steps):
        pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
        layer.decode(pos, qs[t:t + 1].to(DEV), qs[t:t + 1].to(DEV), kn[t:t + 1].to(DEV),
                     vn[t:t + 1].to(DEV), dec, k_pre=kn[t:t + 1].to(DEV))
    torch.cuda.synchronize()
    arena = layer.arena
    assert arena.flushes == (steps - 1 - 192) // 64 + 1
    assert int(arena.prompt_length_t.item()) == arena.prompt_length == length + steps - 1 - \
        ((steps - 1 - 192) % 64) - 128
    assert int(arena.sizes.sum()) == arena.prompt_length * hkv
    assert torch.isfinite(dec.float()).all()
