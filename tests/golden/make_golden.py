"""Write the golden vectors that pin the CPU oracle to the reference's own code.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden.py /root/reference

It imports the reference's pure-torch block build and, under the Triton CPU
interpreter, its selection kernels, and writes inputs/outputs as small
tensor files under tests/golden/.  The reference itself is never copied: only
the vectors are kept.

  kmeans_*.pt   ProductPostingIndex.build (state.py:477-948) on CPU, paper
                settings (flat unit 2048, whole routing, 8 fit iterations,
                page alignment 16); kmeans_sink* with SEMBLO_SINK_TOKENS set
                (cluster 0 reserved for the first positions).  The keys are regenerated from the seed by
                tests/golden/synth.py; a checksum of them is stored.
  router_*.pt   trivial_router_vectors (trivial_router.py:48-75) through its
                torch path off the GPU (:55-61), on seeded bf16 queries with
                rows of tiny, huge, zero and single-spike norms mixed in.
  select_*.pt   theta_select_bitmask_flat (fused_select.py:806-919) with the
                torch-form scores (SEMBLO_FLAT_TORCH_SCORES=1, fused_select.py:
                865-910) and the RESIDENT _streaming_select_kernel
                (fused_select.py:551-717) run by the Triton interpreter on CPU.
                (The interpreter's bf16 tl.dot gives degenerate scores, so the
                tensor-core scorer itself is pinned by its fp64 closed form.)
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

import torch  # noqa: E402

from synth import golden_keys, keys_checksum  # noqa: E402

KMEANS_CASES = [
    # name, L, Hkv, D, seed, codebook_seed, min_log2
    ("kmeans_l512_d64", 512, 2, 64, 11, 0, 7),
    ("kmeans_l2048_d128", 2048, 2, 128, 12, 3, 5),
    ("kmeans_l4096_d128_mix", 4096, 1, 128, 13, 0, 7),
]


def make_kmeans(ref_root: str) -> None:
    os.environ.update({
        "SEMBLO_FLAT_UNIT_TOKENS": "2048",
        "SEMBLO_FA3_ALIGN": "16",
        "SEMBLO_ROUTING_NORMALIZE": "whole",
    })
    from semblo.vllm_plugin.routing_map import routing_normalize
    from semblo.vllm_plugin.state import ProductPostingIndex
    for name, length, hkv, d, seed, cseed, min_log2 in KMEANS_CASES:
        os.environ["SEMBLO_FLAT_MIN_CLUSTERS_LOG2"] = str(min_log2)
        k_pre = golden_keys(length, hkv, d, seed, mixture=name.endswith("_mix"))
        product = routing_normalize(k_pre, 2)
        index = ProductPostingIndex.build(
            product, torch.arange(length), num_centroids=128, kmeans_iters=4,
            kmeans_sample_size=8192, codebook_seed=cseed, flat_unit_tokens=2048,
            flat_min_clusters_log2=min_log2, page_align=16)
        out = dict(
            length=torch.tensor(length), hkv=torch.tensor(hkv), d=torch.tensor(d),
            seed=torch.tensor(seed), codebook_seed=torch.tensor(cseed),
            min_log2=torch.tensor(min_log2), keys_checksum=keys_checksum(k_pre),
            product=product.contiguous(),
            codebooks=index.codebooks.contiguous(),
            posting=index.posting_positions.contiguous(),
            indptr=index.bucket_indptr.contiguous(),
            sizes=index.bucket_sizes.contiguous(),
            inverse=index.inverse_positions().contiguous(),
        )
        if length > 1024:
            out.pop("product")       # regenerated from the seed; keeps the file small
        torch.save(out, HERE / f"{name}.pt")
        print(name, "C =", int(index.bucket_sizes.shape[1]), "width =",
              int(index.posting_positions.shape[1]))


KMEANS_SINK_CASES = [
    # name, L, Hkv, D, seed, codebook_seed, min_log2, sink (SEMBLO_SINK_TOKENS)
    ("kmeans_sink32_l2048_d128", 2048, 2, 128, 14, 5, 5, 32),
    ("kmeans_sink64_l4096_d128", 4096, 1, 128, 15, 1, 7, 64),
]


def make_kmeans_sink(ref_root: str) -> None:
    """The fitted partition with an attention sink (state.py:757-782): positions
    0..S-1 are cluster 0, the others fitted into C-1 clusters."""
    os.environ.update({
        "SEMBLO_FLAT_UNIT_TOKENS": "2048",
        "SEMBLO_FA3_ALIGN": "16",
        "SEMBLO_ROUTING_NORMALIZE": "whole",
    })
    from semblo.vllm_plugin.routing_map import routing_normalize
    from semblo.vllm_plugin.state import ProductPostingIndex
    for name, length, hkv, d, seed, cseed, min_log2, sink in KMEANS_SINK_CASES:
        os.environ["SEMBLO_FLAT_MIN_CLUSTERS_LOG2"] = str(min_log2)
        os.environ["SEMBLO_SINK_TOKENS"] = str(sink)
        try:
            k_pre = golden_keys(length, hkv, d, seed, mixture=name.endswith("_mix"))
            product = routing_normalize(k_pre, 2)
            index = ProductPostingIndex.build(
                product, torch.arange(length), num_centroids=128, kmeans_iters=4,
                kmeans_sample_size=8192, codebook_seed=cseed, flat_unit_tokens=2048,
                flat_min_clusters_log2=min_log2, page_align=16)
        finally:
            os.environ.pop("SEMBLO_SINK_TOKENS", None)
        out = dict(
            length=torch.tensor(length), hkv=torch.tensor(hkv), d=torch.tensor(d),
            seed=torch.tensor(seed), codebook_seed=torch.tensor(cseed),
            min_log2=torch.tensor(min_log2), sink=torch.tensor(sink),
            keys_checksum=keys_checksum(k_pre),
            codebooks=index.codebooks.contiguous(),
            posting=index.posting_positions.contiguous(),
            indptr=index.bucket_indptr.contiguous(),
            sizes=index.bucket_sizes.contiguous(),
            inverse=index.inverse_positions().contiguous(),
        )
        torch.save(out, HERE / f"{name}.pt")
        print(name, "C =", int(index.bucket_sizes.shape[1]), "sink size",
              index.bucket_sizes[:, 0].tolist())


SELECT_CASES = [
    # name, Q, Hq, Hkv, D, C, nb, g_union, target, beta, tau, seed
    ("select_q64_c128", 64, 8, 2, 128, 128, 2, 32, 512, 0.25, 0.1, 21),
    ("select_q40_c128_b0", 40, 4, 2, 64, 128, 5, 8, 300, 0.0, 0.05, 22),
    ("select_q16_c256_allfit", 16, 4, 1, 64, 256, 1, 16, 10 ** 6, 0.25, 0.1, 23),
]


def make_select(ref_root: str) -> None:
    os.environ["TRITON_INTERPRET"] = "1"
    from semblo.vllm_plugin import fused_select as fs
    for name, q, hq, hkv, d, c, nb, g, target, beta, tau, seed in SELECT_CASES:
        gen = torch.Generator().manual_seed(seed)
        raw = torch.randn(q, hq, d, generator=gen)
        vectors = torch.nn.functional.normalize(raw, dim=-1).to(torch.bfloat16)
        cb = torch.randn(hkv, c, d, generator=gen)
        cb = torch.nn.functional.normalize(cb, dim=-1)
        codebooks = torch.stack(list(cb.chunk(2, dim=-1)), dim=1).to(torch.bfloat16).contiguous()
        sizes = torch.randint(0, 200, (nb, hkv, c), generator=gen, dtype=torch.int32)
        sizes[:, :, ::5] = 0
        logmix = torch.zeros(q, hq, 1)
        bitmask = torch.zeros(nb, hkv, c // 32, dtype=torch.int32)
        qmask = torch.zeros(q, hkv, c // 32, dtype=torch.int32)
        # The torch form of the scorer (SEMBLO_FLAT_TORCH_SCORES=1); the prob it
        # hands to the select kernel is captured on the way in.
        seen = {}
        real = fs._run_streaming_select

        def capture(prob, *a, **kw):
            seen["prob"] = prob.clone()
            out = real(prob, *a, **kw)
            return out
        fs._run_streaming_select = capture
        os.environ["SEMBLO_FLAT_TORCH_SCORES"] = "1"
        try:
            counts, tokens = fs.theta_select_bitmask_flat(
                vectors.view(q, hq, 1, d), logmix, codebooks, sizes, bitmask,
                temperature=tau, beta=beta, target_tokens=target, g_union=g, iters=16,
                qmask=qmask)
        finally:
            fs._run_streaming_select = real
            os.environ.pop("SEMBLO_FLAT_TORCH_SCORES", None)
        prob_in = seen["prob"]
        torch.save(dict(vectors=vectors, codebooks=codebooks, sizes=sizes, prob=prob_in,
                        bitmask=bitmask, qmask=qmask, counts=counts, tokens=tokens,
                        g_union=torch.tensor(g), target=torch.tensor(target),
                        beta=torch.tensor(beta), tau=torch.tensor(tau)),
                   HERE / f"{name}.pt")
        print(name, "selected per query", counts.float().mean().item())


ROUTER_CASES = [
    # name, Q, Hq, D, factors, seed
    ("router_q48_h4_d256", 48, 4, 256, 1, 31),
    ("router_q32_h8_d128_f2", 32, 8, 128, 2, 32),
    # tiny halves: the intermediate bf16 rounding shows in the output
    ("router_q256_h4_d16_f2", 256, 4, 16, 2, 33),
]


def router_inputs(q: int, hq: int, d: int, seed: int) -> torch.Tensor:
    """Seeded bf16 queries [Q, Hq, D]: Gaussian rows, then every 5th row scaled by
    1e-3, every 7th by 1e3, row 3 zero and row 4 a single spike."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(q, hq, d, generator=gen)
    x[::5] *= 1e-3
    x[::7] *= 1e3
    x[3] = 0.0
    x[4] = 0.0
    x[4, :, 7] = 5.0
    return x.to(torch.bfloat16)


def make_router(ref_root: str) -> None:
    from semblo.vllm_plugin.trivial_router import trivial_router_vectors
    for name, q, hq, d, factors, seed in ROUTER_CASES:
        x = router_inputs(q, hq, d, seed)
        out = trivial_router_vectors(x, factors)          # CPU tensor: the torch path
        torch.save(dict(x=x, factors=torch.tensor(factors), out=out.contiguous()),
                   HERE / f"{name}.pt")
        print(name, tuple(out.shape))


if __name__ == "__main__":
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    which = sys.argv[2] if len(sys.argv) > 2 else "all"
    if which in ("all", "kmeans"):
        make_kmeans(ref)
    if which in ("all", "kmeans_sink"):
        make_kmeans_sink(ref)
    if which in ("all", "select"):
        make_select(ref)
    if which in ("all", "router"):
        make_router(ref)
