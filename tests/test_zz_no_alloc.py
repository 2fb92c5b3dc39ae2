"""sbsa_decode_step_noalloc (the decode step whose scratch is the library's static per-GPU
array) against sbsa_decode_step with its workspace: bit-equal output, LSE and CSR, on two
calls in a row, the second with a smaller layer."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _decode_layer(length, hq, hkv, d, seed, num_clusters=None):
    from semblo_amd.arena import DecodeArena
    from semblo_amd.state import ProductPostingIndex
    from semblo_amd.synthetic import decode_queries, mixture_layer
    inp = mixture_layer(length, hq, hkv, d, mixtures=32, seed=seed, device=DEV)
    kw = {"num_clusters": num_clusters} if num_clusters else {}
    idx = ProductPostingIndex.build(inp.k, torch.arange(length, device=DEV), codebook_seed=seed,
                                    router_pass=True, **kw)
    idx.pack_prompt_kv(inp.k, inp.v)
    arena = DecodeArena(idx, reserve=64)
    qs, kn, vn = decode_queries(inp, 2, hq, seed=seed)
    return idx, arena, qs, kn, vn


class _Layer:
    def __init__(self, hq, hkv, d):
        self.num_heads, self.num_kv_heads, self.head_dim = hq, hkv, d


@pytest.mark.parametrize("shape", [(8192, 16, 4, 256, 256, 120), (2048, 8, 2, 128, None, 24)])
def test_decode_step_without_allocation_matches_the_workspace_entry_point(shape):
    from semblo_amd import _lib
    from semblo_amd.fused_decode import fused_decode_step
    length, hq, hkv, d, c_force, splits = shape
    print(f"no-alloc decode: L={length} Hq={hq} Hkv={hkv} D={d} C={c_force} splits={splits}",
          flush=True)
    idx, arena, qs, kn, vn = _decode_layer(length, hq, hkv, d, seed=length, num_clusters=c_force)
    c = idx.num_buckets
    need = _lib.query("sbsa_decode_workspace_bytes", hq, hkv, c, d, splits, 8)
    assert need <= _lib.query("sbsa_decode_scratch_bytes")
    layer = _Layer(hq, hkv, d)
    kw = dict(temperature=0.1, beta=0.25, target_tokens=length // 16, sm_scale=d ** -0.5,
              num_splits=splits, iters=16, suffix_splits=8)
    for t in range(2):
        pos = torch.tensor([length + t], dtype=torch.int32, device=DEV)
        res = {}
        for no_alloc in (False, True):
            out = torch.full((1, hq * d), float("nan"), dtype=torch.bfloat16, device=DEV)
            lse = torch.full((hq,), float("nan"), dtype=torch.float32, device=DEV)
            csr = torch.full((3 * hkv * c + 2 * hkv,), -7, dtype=torch.int32, device=DEV)
            q = qs[t:t + 1]
            fused_decode_step(layer, arena, q_post=q, q_pre=q, positions=pos, k_post=kn[t:t + 1],
                              v_states=vn[t:t + 1], output=out, out_lse=lse, csr_out=csr,
                              no_alloc=no_alloc, **kw)
            torch.cuda.synchronize()
            res[no_alloc] = (out.cpu(), lse.cpu(), csr.cpu())
        assert not torch.isnan(res[True][0].float()).any()
        assert torch.equal(res[True][0], res[False][0]), f"step {t}: outputs differ"
        assert torch.equal(res[True][1], res[False][1]), f"step {t}: LSEs differ"
        # the CSR: rcount and rtokens, and each head's first rcount runs (entries past
        # them are left from earlier calls in both forms)
        n = hkv * c
        a, b = res[True][2], res[False][2]
        assert torch.equal(a[3 * n:], b[3 * n:]), f"step {t}: run counts differ"
        for h in range(hkv):
            k = int(a[3 * n + h])
            for part in range(3):
                lo = part * n + h * c
                assert torch.equal(a[lo:lo + k], b[lo:lo + k]), f"step {t}: CSR part {part} differs"
    print(f"no-alloc decode: 2 steps bit-equal (scratch {need} of "
          f"{_lib.query('sbsa_decode_scratch_bytes')} bytes)", flush=True)
