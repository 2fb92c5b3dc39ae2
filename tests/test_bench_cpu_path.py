"""The bench's torch CPU path (the reported CPU baseline) computes the same attention as
the oracle's fp64 reference: the sparse prefill over the selected clusters' causal rows
plus the chunk window, dense-prefix chunks over every earlier key, and the decode step
over the selected clusters and the suffix."""
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "semantic-block-sparse-attention_amd"))

import bench  # noqa: E402
from oracle import reference_cpu as ref  # noqa: E402
from semblo_amd.synthetic import decode_queries, mixture_layer  # noqa: E402


def _layer(length=2048, hq=4, hkv=2, d=64, seed=3):
    inp = mixture_layer(length, hq, hkv, d, mixtures=16, seg=(32, 128), seed=seed,
                        dtype=torch.float32, device="cpu")
    idx = ref.build_flat_index(ref.routing_normalize_keys(inp.k), codebook_seed=0)
    return inp, idx


def test_cpu_prefill_matches_the_oracle_per_chunk():
    inp, idx = _layer()
    length, hq, d = inp.q.shape
    target, chunk = length // 16, 256
    cluster_of = bench._cluster_of(idx, length)
    got = bench.cpu_prefill(ref, inp.q, inp.k, inp.v, idx, cluster_of, chunk=chunk, target=target,
                            dense_x=4, temperature=0.1, beta=0.25, heads=range(inp.k.shape[1]))
    for c0 in (0, 512, 1024, 1792):                  # dense (<= 4K), dense, sparse, sparse
        n = 16
        wstart = ref.chunk_window_start(c0, target, 4)
        sel = None
        sizes = ref.causal_sizes_at(idx["posting"], idx["indptr"], idx["sizes"], c0)
        if wstart > 0:
            vec = ref.trivial_router_vectors(inp.q[c0:c0 + chunk], 1)
            prob = ref.mixture_probs(vec, None, idx["codebooks"], 0.1)
            sel = ref.theta_select(prob, sizes[None], beta=0.25, target_tokens=target,
                                   g_union=chunk)["sel"][:n]
        want = ref.prefill_chunk_reference(inp.q[c0:c0 + n], inp.k, inp.v, idx["posting"],
                                           idx["indptr"], sizes, sel, c0, wstart, d ** -0.5)
        assert torch.allclose(got[c0:c0 + n].double(), want, atol=1e-4, rtol=1e-4), c0


def test_cpu_decode_step_matches_the_oracle():
    inp, idx = _layer(seed=5)
    length, hq, d = inp.q.shape
    hkv = inp.k.shape[1]
    target = length // 16
    cluster_of = bench._cluster_of(idx, length)
    qs, kn, vn = decode_queries(inp, 3, hq, seed=1, dtype=torch.float32)
    outs = []
    orig = bench._attend

    def spy(q, k, v, mask, scale):
        o = orig(q, k, v, mask, scale)
        outs.append(o)
        return o

    bench._attend = spy
    try:
        bench.cpu_decode(ref, qs, kn, vn, inp.k, inp.v, idx, cluster_of, target=target,
                         temperature=0.1, beta=0.25, heads=range(hkv))
    finally:
        bench._attend = orig
    packed = ref.pack_prompt_kv(idx["posting"], inp.k, inp.v)
    for t in range(3):
        vec = ref.trivial_router_vectors(qs[t:t + 1], 1)
        prob = ref.mixture_probs(vec, None, idx["codebooks"], 0.1)
        sel = ref.theta_select(prob, idx["sizes"][None], beta=0.25, target_tokens=target)["sel"][0]
        want = ref.decode_reference(qs[t], packed, idx["indptr"], idx["sizes"], sel, kn[:t + 1],
                                    vn[:t + 1], d ** -0.5)
        got = torch.cat([outs[t * hkv + h][0] for h in range(hkv)])
        assert torch.allclose(got.double(), want, atol=1e-4, rtol=1e-4), t
