"""Seeded key generators for the golden fixtures (CPU, deterministic for a torch version)."""
from __future__ import annotations

import torch


def golden_keys(length: int, hkv: int, d: int, seed: int, *, mixture: bool = False) -> torch.Tensor:
    """[L, Hkv, D] bf16 pre-RoPE keys.  ``mixture``: 16 Gaussian centres shared by
    runs of 32 consecutive tokens, noise 0.3 (the benchmark's key model, small)."""
    gen = torch.Generator().manual_seed(seed)
    if not mixture:
        return torch.randn(length, hkv, d, generator=gen).to(torch.bfloat16)
    centres = torch.randn(hkv, 16, d, generator=gen)
    seg = torch.randint(0, 16, ((length + 31) // 32,), generator=gen)
    which = seg.repeat_interleave(32)[:length]
    keys = centres[:, which].permute(1, 0, 2) + 0.3 * torch.randn(length, hkv, d, generator=gen)
    return keys.to(torch.bfloat16)


def keys_checksum(k: torch.Tensor) -> torch.Tensor:
    """A float64 fingerprint of the keys, to detect a generator that changed."""
    x = k.double().flatten()
    w = torch.arange(1, x.numel() + 1, dtype=torch.float64).remainder(97.0) + 1.0
    return torch.stack([(x * w).sum(), (x * x).sum()])
