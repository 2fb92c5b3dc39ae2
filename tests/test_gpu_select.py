"""S0/S2/S3 on the GPU against the oracle and the reference's golden vectors.

Selected sets must equal the oracle's except for near-ties (score within
1e-4 relative of the cut), which are counted and printed.  The bisection's
own arithmetic is checked bit-exact by feeding the kernel's scores back to
the oracle's bisection.
"""
from __future__ import annotations

from pathlib import Path

import pytest
import torch

from gpu_util import bf16_rounding_near_ties, compare_selection, oracle_select
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
DEV = "cuda"


def _select_gpu(vectors, codebooks, sizes, *, tau, beta, target, g_union, logmix=None):
    from semblo_amd.fused_select import theta_select_bitmask_flat
    q, hq, d = vectors.shape
    hkv, _, c, _ = codebooks.shape
    nb = max(sizes.shape[0], (q + g_union - 1) // g_union)    # one bitmask row per query block
    bitmask = torch.zeros(nb, hkv, c // 32, dtype=torch.int32, device=DEV)
    qmask = torch.zeros(q, hkv, c // 32, dtype=torch.int32, device=DEV)
    prob = torch.empty(q, hkv, c, dtype=torch.float32, device=DEV)
    theta = torch.empty(q, hkv, dtype=torch.float32, device=DEV)
    counts, tokens = theta_select_bitmask_flat(
        vectors.to(DEV).view(q, hq, 1, d), logmix, codebooks.to(DEV), sizes.to(DEV).contiguous(),
        bitmask, temperature=tau, beta=beta, target_tokens=target, g_union=g_union, qmask=qmask,
        prob_out=prob, theta_out=theta)
    torch.cuda.synchronize()
    return dict(qmask=qmask.cpu(), bitmask=bitmask.cpu(), counts=counts.cpu(),
                tokens=tokens.cpu(), prob=prob.cpu(), theta=theta.cpu())


def _router_exact(x: torch.Tensor, factors: int) -> list:
    """fp64 values before each of the router's two roundings (the second from the
    oracle's rounded first stage)."""
    q, h, d = x.shape
    halves = x.double().view(q, h, factors, d // factors)
    s1 = halves / halves.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    xf = x.float().view(q, h, factors, d // factors)
    u1 = (xf / xf.norm(dim=-1, keepdim=True).clamp_min(1e-12)).to(torch.bfloat16).double()
    s2 = u1 / u1.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    return [s1.reshape(q, h, d), s2.reshape(q, h, d)]


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("router_*.pt")))
def test_router_matches_the_reference_golden(name):
    """S0 against the reference's own router output: bit-exact except values whose
    pre-rounding value lies within 1e-4 of a bf16 rounding midpoint (fp32 norms summed
    in another order), which are counted."""
    from semblo_amd.trivial_router import trivial_router_vectors
    g = torch.load(GOLDEN / name, weights_only=True)
    x, f = g["x"], int(g["factors"])
    got = trivial_router_vectors(x.to(DEV), f).cpu()
    n = bf16_rounding_near_ties(got, g["out"], _router_exact(x, f))
    print(f"{name}: {n} of {got.numel()} values differ, all rounding near-ties")


def test_router_matches_the_oracle():
    from semblo_amd.trivial_router import trivial_router_vectors
    x = (torch.randn(257, 16, 256, generator=torch.Generator().manual_seed(0)) * 3).to(torch.bfloat16)
    got = trivial_router_vectors(x.to(DEV), 1).cpu()
    want = ref.trivial_router_vectors(x, 1)
    n = bf16_rounding_near_ties(got, want, _router_exact(x, 1))
    print(f"router: {n} of {got.numel()} bf16 values differ, all rounding near-ties")


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("select_*.pt")))
def test_selection_matches_the_reference_golden(name):
    g = torch.load(GOLDEN / name, weights_only=True)
    tau, beta, target, gu = float(g["tau"]), float(g["beta"]), float(g["target"]), int(g["g_union"])
    out = _select_gpu(g["vectors"], g["codebooks"], g["sizes"], tau=tau, beta=beta,
                      target=target, g_union=gu)
    # the probabilities: same quantity as the reference's, up to summation order
    assert torch.allclose(out["prob"], g["prob"], rtol=2e-4, atol=1e-6)
    # the bisection on the kernel's own scores is the oracle's (bit-exact arithmetic)
    mine = ref.theta_select(out["prob"], g["sizes"], beta=beta, target_tokens=target, g_union=gu)
    assert torch.equal(mine["qmask"], out["qmask"])
    assert torch.equal(mine["counts"], out["counts"])
    assert torch.equal(mine["tokens"], out["tokens"])
    assert torch.equal(mine["bitmask"], out["bitmask"])
    # against the reference's own selection: equal up to near-ties
    want = ref.theta_select(g["prob"], g["sizes"], beta=beta, target_tokens=target, g_union=gu)
    sel_gpu = ref.unpack_bits(out["qmask"], g["codebooks"].shape[2])
    sel_ref = ref.unpack_bits(g["qmask"], g["codebooks"].shape[2])
    rep = compare_selection(sel_gpu, sel_ref, want["score"], want["theta"], out["theta"])
    print(f"{name}: {rep}")


@pytest.mark.parametrize("shape", [(512, 16, 4, 256, 128), (300, 8, 2, 128, 128),
                                   (128, 16, 4, 256, 256), (64, 4, 4, 128, 512)])
def test_selection_matches_the_oracle_on_mixture_scores(shape):
    q, hq, hkv, d, c = shape
    gen = torch.Generator().manual_seed(q + c)
    cents = torch.nn.functional.normalize(torch.randn(hkv, c, d, generator=gen), dim=-1)
    pick = torch.randint(0, c, (q, hq), generator=gen)
    raw = cents[torch.arange(hq) // (hq // hkv)][None].expand(q, -1, -1, -1)
    raw = raw.gather(2, pick[..., None, None].expand(-1, -1, 1, d))[:, :, 0]
    raw = raw + 0.6 * torch.randn(q, hq, d, generator=gen) / d ** 0.5
    vectors = ref.trivial_router_vectors(raw.to(torch.bfloat16), 1)
    codebooks = torch.stack(list(cents.chunk(2, dim=-1)), dim=1).to(torch.bfloat16).contiguous()
    sizes = torch.randint(0, 600, (1, hkv, c), generator=gen, dtype=torch.int32)
    sizes[..., ::9] = 0
    target = int(sizes.sum() // hkv // 16)
    out = _select_gpu(vectors, codebooks, sizes, tau=0.1, beta=0.25, target=target, g_union=q)
    want = oracle_select(vectors, codebooks, sizes, temperature=0.1, beta=0.25, target=target,
                         g_union=q)
    sel_gpu = ref.unpack_bits(out["qmask"], c)
    rep = compare_selection(sel_gpu, want["sel"], want["score"], want["theta"], out["theta"])
    print(f"shape {shape}: {rep}")
    # counts and tokens follow the selection
    assert torch.equal(out["counts"], sel_gpu.sum(-1).to(torch.int32))
    assert torch.equal(out["tokens"], (sel_gpu * sizes[0][None]).sum(-1).to(torch.int32))


def test_all_fit_and_dead_clusters():
    q, hq, hkv, d, c = 40, 8, 2, 128, 128
    gen = torch.Generator().manual_seed(3)
    vectors = ref.trivial_router_vectors(torch.randn(q, hq, d, generator=gen).to(torch.bfloat16), 1)
    cents = torch.nn.functional.normalize(torch.randn(hkv, c, d, generator=gen), dim=-1)
    codebooks = torch.stack(list(cents.chunk(2, dim=-1)), dim=1).to(torch.bfloat16).contiguous()
    sizes = torch.randint(1, 50, (1, hkv, c), generator=gen, dtype=torch.int32)
    sizes[..., ::4] = 0
    out = _select_gpu(vectors, codebooks, sizes, tau=0.1, beta=0.25, target=10 ** 7, g_union=8)
    sel = ref.unpack_bits(out["qmask"], c)
    assert torch.equal(sel, (sizes[0] > 0)[None].expand_as(sel))
    out = _select_gpu(vectors, codebooks, torch.zeros_like(sizes), tau=0.1, beta=0.25, target=100,
                      g_union=8)
    assert int(out["counts"].sum()) == 0 and int(out["qmask"].abs().sum()) == 0
