"""Routing vectors of the queries (trivial_router.py:48-75 of the reference), on HIP."""
from __future__ import annotations

import torch

from . import _lib


def trivial_router_vectors(x: torch.Tensor, factors: int = 1,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """[Q, Hq, D] bf16 -> [Q, Hq, D] bf16, normalised per factor (fp32, round, renormalise,
    round).  ``out`` (same shape, contiguous) receives the result without allocating."""
    if x.dtype != torch.bfloat16:
        raise ValueError("routing vectors are bfloat16")
    q, h, d = x.shape
    flat = x.reshape(q * h, d)
    if flat.stride(1) != 1:
        flat = flat.contiguous()
    if out is None:
        out = torch.empty(q, h, d, dtype=x.dtype, device=x.device)
    elif out.shape != x.shape or not out.is_contiguous():
        raise ValueError("out must be contiguous with the input's shape")
    _lib.call("sbsa_route_vectors", _lib.ptr(flat), q * h, flat.stride(0), d, factors,
              _lib.ptr(out), d, _lib.stream(x.device))
    return out
