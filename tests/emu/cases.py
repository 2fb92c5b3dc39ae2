"""Cases run against the emulated library (tests/emu/session.py): the library's host
code on CPU tensors, checked against the oracle as the GPU tests do.  Each case
raises (or the emulation aborts) on a mismatch or a memory fault."""
from __future__ import annotations

import sys
from pathlib import Path

import torch

TESTS = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(TESTS))

from gpu_util import assert_close_bf16, attention_reference, cluster_position_mask  # noqa: E402
from oracle import reference_cpu as ref  # noqa: E402


def _index(k, length, seed):
    from semblo_amd.state import ProductPostingIndex
    idx = ProductPostingIndex.build(k, torch.arange(length), codebook_seed=seed, router_pass=True)
    return idx


def sparse_chunk(length: int, hq: int, hkv: int, d: int, cs: int, ce: int, seed: int,
                 grid: int = 0) -> None:
    """One sparse chunk of the KV-outer prefill (selection, reverse index, work
    list, attention, combine) against fp64 attention over the chunk's own
    selection (kv_outer.py:482-816)."""
    from semblo_amd.fused_select import theta_select_bitmask_flat
    from semblo_amd.kv_outer import kv_outer_attention
    from semblo_amd.synthetic import mixture_layer
    from semblo_amd.trivial_router import trivial_router_vectors
    length, hq, hkv, d, cs, ce, seed = map(int, (length, hq, hkv, d, cs, ce, seed))
    inp = mixture_layer(length, hq, hkv, d, mixtures=16, seg=(32, 256), seed=seed)
    q, k, v = inp.q, inp.k, inp.v
    idx = _index(k, length, seed)
    idx.pack_prompt_kv(k, v)
    target = length // 16
    c = idx.bucket_sizes.shape[1]
    qc = q[cs:ce + 1]
    qn = qc.shape[0]
    sizes = idx.causal_sizes(cs)
    vec = trivial_router_vectors(qc, 1)
    qmask = torch.empty(qn, hkv, c // 32, dtype=torch.int32)
    theta_select_bitmask_flat(vec.view(qn, hq, 1, d), None, idx.codebooks, sizes[None], None,
                              temperature=0.1, beta=0.25, target_tokens=target, g_union=32,
                              qmask=qmask)
    out, _ = kv_outer_attention(qc, idx.packed_kv, qmask, sizes, idx.bucket_indptr,
                                sm_scale=d ** -0.5, local_kv=(k[cs:ce + 1], v[cs:ce + 1]),
                                chunk_start=cs, wstart=cs, grid=int(grid) or None)
    sel = ref.unpack_bits(qmask, c)
    pos = cluster_position_mask(idx.posting_positions, idx.bucket_indptr, sizes, length)
    keys = torch.einsum("qhc,hcl->qhl", sel.double(), pos.double()) > 0
    p = torch.arange(cs, ce + 1)
    win = (torch.arange(length)[None, :] >= cs) & (torch.arange(length)[None, :] <= p[:, None])
    keys |= win[:, None, :]
    want = attention_reference(qc, keys, k, v, d ** -0.5)
    err = assert_close_bf16(out, want, f"emulated sparse chunk L={length} G={hq // hkv} D={d}")
    print(f"sparse chunk L={length} Hq={hq} Hkv={hkv} D={d} chunk {cs}-{ce}: max err {err:.3g}")


def dense_chunk(length: int, hq: int, hkv: int, d: int, cs: int, ce: int, seed: int) -> None:
    """A dense-prefix chunk (exact causal attention, fused_prefill.py:155-189)."""
    from semblo_amd.kv_outer import dense_causal_attention
    from semblo_amd.synthetic import mixture_layer
    length, hq, hkv, d, cs, ce, seed = map(int, (length, hq, hkv, d, cs, ce, seed))
    inp = mixture_layer(length, hq, hkv, d, mixtures=8, seed=seed)
    out = dense_causal_attention(inp.q[cs:ce + 1], inp.k, inp.v, sm_scale=d ** -0.5, chunk_start=cs)
    p = torch.arange(cs, ce + 1)
    keys = (torch.arange(length)[None, :] <= p[:, None])[:, None, :].expand(-1, hkv, -1)
    want = attention_reference(inp.q[cs:ce + 1], keys, inp.k, inp.v, d ** -0.5)
    err = assert_close_bf16(out, want, f"emulated dense chunk {cs}-{ce}")
    print(f"dense chunk L={length} Hq={hq} Hkv={hkv} D={d} chunk {cs}-{ce}: max err {err:.3g}")



def decode_steps(length: int, hq: int, hkv: int, d: int, seed: int, steps: int = 4,
                 splits: int = 8, target: int = 0) -> None:
    """Decode steps over the prompt's selection and the suffix store
    (fused_decode.py:393-521) against fp64 over the step's own selection.  A
    large ``target`` with few ``splits`` gives each split several rounds of rows."""
    from semblo_amd.arena import DecodeArena
    from semblo_amd.fused_decode import fused_decode_step
    from semblo_amd.synthetic import decode_queries, mixture_layer
    length, hq, hkv, d, seed, steps, splits, target = map(int, (length, hq, hkv, d, seed, steps, splits, target))
    target = target or length // 16
    inp = mixture_layer(length, hq, hkv, d, mixtures=16, seg=(32, 256), seed=seed)
    idx = _index(inp.k, length, seed)
    idx.pack_prompt_kv(inp.k, inp.v)
    arena = DecodeArena(idx, reserve=64, shuffle_blocks=torch.Generator().manual_seed(seed))

    class _Layer:
        num_heads, num_kv_heads, head_dim = hq, hkv, d

    qs, kn, vn = decode_queries(inp, steps, hq, seed=seed)
    c = idx.num_buckets
    n = hkv * c
    csr = torch.empty(3 * n + 2 * hkv, dtype=torch.int32)
    out = torch.empty(1, hq * d, dtype=torch.bfloat16)
    packed = idx.packed_kv
    indptr, sizes = idx.bucket_indptr, idx.bucket_sizes
    for t in range(steps):
        pos = torch.tensor([length + t], dtype=torch.int32)
        fused_decode_step(_Layer(), arena, q_post=qs[t:t + 1], q_pre=qs[t:t + 1], positions=pos,
                          k_post=kn[t:t + 1], v_states=vn[t:t + 1], output=out, temperature=0.1,
                          beta=0.25, target_tokens=target, sm_scale=d ** -0.5,
                          num_splits=splits, iters=16, csr_out=csr)
        sel = torch.zeros(hkv, c, dtype=torch.bool)
        rstart = csr[:n].view(hkv, c)
        for h in range(hkv):
            for p in range(int(csr[3 * n + h])):
                cand = torch.nonzero((indptr[h, :-1] == rstart[h, p]) & (sizes[h] > 0)).flatten()
                assert cand.numel() == 1
                sel[h, cand[0]] = True
        want = ref.decode_reference(qs[t], packed, indptr, sizes, sel, kn[:t + 1], vn[:t + 1], d ** -0.5)
        err = assert_close_bf16(out.view(hq, d), want, f"emulated decode step {t}")
    print(f"decode L={length} Hq={hq} Hkv={hkv} D={d}: {steps} steps, max err {err:.3g}")


def towering_dense(beta: float, length: int = 1024, cs: int = 512, ce: int = 767) -> None:
    """A key far above every score of the first tile: the items are redone with the
    rows' true maxima (dense chunk), and the result is exact causal attention."""
    from semblo_amd.kv_outer import dense_causal_attention
    beta, length, cs, ce = float(beta), int(length), int(cs), int(ce)
    gen = torch.Generator().manual_seed(17)
    hq, hkv, d = 8, 2, 128
    u = torch.randn(d, generator=gen)
    q = (3 * u + torch.randn(length, hq, d, generator=gen)).to(torch.bfloat16)
    k = torch.randn(length, hkv, d, generator=gen)
    v = torch.randn(length, hkv, d, generator=gen).to(torch.bfloat16)
    k[450] = beta * u
    k = k.to(torch.bfloat16)
    out = dense_causal_attention(q[cs:ce + 1], k, v, sm_scale=d ** -0.5, chunk_start=cs)
    p = torch.arange(cs, ce + 1)
    keys = (torch.arange(length)[None, :] <= p[:, None])[:, None, :].expand(-1, hkv, -1)
    want = attention_reference(q[cs:ce + 1], keys, k, v, d ** -0.5)
    err = assert_close_bf16(out, want, f"emulated towering key, beta {beta}")
    print(f"towering dense beta {beta}: max err {err:.3g}")


def towering_sparse(hq: int, hkv: int, d: int, grid: int, length: int = 1024, cs: int = 512,
                    ce: int = 767) -> None:
    """Keys of which every 97th lies far along the queries' common direction: items
    holding one past their first tile are redone (sparse chunk)."""
    from semblo_amd.fused_select import theta_select_bitmask_flat
    from semblo_amd.kv_outer import kv_outer_attention
    from semblo_amd.trivial_router import trivial_router_vectors
    hq, hkv, d, grid, length, cs, ce = map(int, (hq, hkv, d, grid, length, cs, ce))
    gen = torch.Generator().manual_seed(23)
    u = torch.randn(d, generator=gen)
    q = (3 * u + torch.randn(length, hq, d, generator=gen)).to(torch.bfloat16)
    k = torch.randn(length, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(length, hkv, d, generator=gen).to(torch.bfloat16)
    k_att = k.clone()
    k_att[97::97] = (3.0 * u).to(torch.bfloat16)
    idx = _index(k, length, 5)
    idx.pack_prompt_kv(k_att, v)
    c = idx.bucket_sizes.shape[1]
    qc = q[cs:ce + 1]
    qn = qc.shape[0]
    sizes = idx.causal_sizes(cs)
    vec = trivial_router_vectors(qc, 1)
    qmask = torch.empty(qn, hkv, c // 32, dtype=torch.int32)
    theta_select_bitmask_flat(vec.view(qn, hq, 1, d), None, idx.codebooks, sizes[None], None,
                              temperature=0.1, beta=0.25, target_tokens=length // 16, g_union=32,
                              qmask=qmask)
    out, _ = kv_outer_attention(qc, idx.packed_kv, qmask, sizes, idx.bucket_indptr,
                                sm_scale=d ** -0.5, local_kv=(k_att[cs:ce + 1], v[cs:ce + 1]),
                                chunk_start=cs, wstart=cs, grid=grid or None)
    sel = ref.unpack_bits(qmask, c)
    pos = cluster_position_mask(idx.posting_positions, idx.bucket_indptr, sizes, length)
    keys = torch.einsum("qhc,hcl->qhl", sel.double(), pos.double()) > 0
    p = torch.arange(cs, ce + 1)
    win = (torch.arange(length)[None, :] >= cs) & (torch.arange(length)[None, :] <= p[:, None])
    keys |= win[:, None, :]
    want = attention_reference(qc, keys, k_att, v, d ** -0.5)
    err = assert_close_bf16(out, want, f"emulated towering keys, sparse, G={hq // hkv} D={d}")
    print(f"towering sparse G={hq // hkv} D={d} grid {grid}: max err {err:.3g}")

def _debug_dense(length: int, hq: int, hkv: int, d: int, cs: int, ce: int, seed: int) -> None:
    from semblo_amd.kv_outer import dense_causal_attention
    from semblo_amd.synthetic import mixture_layer
    length, hq, hkv, d, cs, ce, seed = map(int, (length, hq, hkv, d, cs, ce, seed))
    inp = mixture_layer(length, hq, hkv, d, mixtures=8, seed=seed)
    out = dense_causal_attention(inp.q[cs:ce + 1], inp.k, inp.v, sm_scale=d ** -0.5, chunk_start=cs)
    p = torch.arange(cs, ce + 1)
    keys = (torch.arange(length)[None, :] <= p[:, None])[:, None, :].expand(-1, hkv, -1)
    want = attention_reference(inp.q[cs:ce + 1], keys, inp.k, inp.v, d ** -0.5)
    bad = (out.double() - want).abs() > 0.02 + 0.01 * want.abs()
    print("bad per query:", bad.sum(dim=(1, 2)).tolist())
    print("bad per head:", bad.sum(dim=(0, 2)).tolist())
    print("bad per dim (first 64):", bad.sum(dim=(0, 1)).tolist()[:64])
    q0 = int(bad.sum(dim=(1, 2)).argmax())
    print("query", q0, "head 0 got", out[q0, 0, :8].tolist(), "want", want[q0, 0, :8].tolist())
    torch.set_printoptions(precision=3, linewidth=200)
    print("dims 64..95 got ", out[q0, 0, 64:96])
    print("dims 64..95 want", want[q0, 0, 64:96].float())
    print("dims 96..127 got ", out[q0, 0, 96:128])
    print("dims 96..127 want", want[q0, 0, 96:128].float())
    print("bad dims of q0 h0:", torch.nonzero(bad[q0, 0]).flatten().tolist())


def gpu_tests(*node_ids: str) -> None:
    """GPU test functions (tests/test_gpu_*.py node ids) against the emulated library:
    each module's device is set to the CPU before pytest collects it, so the tests
    run unchanged, every kernel under the address sanitizer."""
    import importlib
    import pytest
    sys.path.insert(0, str(TESTS / "golden"))      # as tests/conftest.py does
    for node in node_ids:
        mod = importlib.import_module(Path(node.split("::")[0]).stem)
        mod.DEV = "cpu"
    rc = pytest.main([str(TESTS / n) for n in node_ids] +
                     ["-m", "gpu", "-q", "-p", "no:cacheprovider", "-p", "no:randomly"])
    if rc != 0:
        raise SystemExit(f"emulated GPU tests failed: pytest exit {int(rc)}")
    print(f"emulated GPU tests: {len(node_ids)} node ids passed")
