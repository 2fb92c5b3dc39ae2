"""The bf16 MFMA operand layouts the kernels assume, on a small argmax GEMM
(sbsa_kmeans_assign) against a CPU brute force."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,c,d", [(37, 64, 64), (300, 128, 128), (1000, 192, 256)])
def test_argmax_gemm_matches_brute_force(n, c, d):
    from semblo_amd import _lib
    gen = torch.Generator().manual_seed(n)
    x = torch.randn(n, d, generator=gen).to(torch.bfloat16)
    cent = torch.randn(c, d, generator=gen).to(torch.bfloat16)
    want = torch.argmax((x.float() @ cent.float().T).to(torch.bfloat16), dim=1)
    xd, cd = x.cuda(), cent.cuda()
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    _lib.call("sbsa_kmeans_assign", _lib.ptr(xd), d, None, n, _lib.ptr(cd), c, d,
              _lib.ptr(out), _lib.stream())
    torch.cuda.synchronize()
    got = out.cpu().long()
    sims = (x.float() @ cent.float().T).to(torch.bfloat16).float()
    # equal, or an exact tie of the rounded similarities resolved the same way
    same = got == want
    assert bool(same.all()) or bool((sims.gather(1, got[:, None]) == sims.gather(1, want[:, None])).all())
    assert float(same.float().mean()) > 0.99
