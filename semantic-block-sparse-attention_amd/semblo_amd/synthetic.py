"""Seeded synthetic inputs of the benchmark configurations (Gaussian-mixture keys/queries).

Keys of each KV head come from M isotropic Gaussians with N(0, I) centres
and noise 0.3; runs of consecutive tokens (segments) share a centre drawn
uniformly from the M.  A query of q head j at position p is the centre of
p's segment (for j's KV head) plus noise 0.5, drawn independently per head.
Values are N(0, 1).  ``sinks`` > 0 scales the first keys to 8x their norm.
q_post = q_pre and k_post = k_pre (no RoPE in the layer benchmark).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class LayerInputs:
    q: torch.Tensor        # [L, Hq, D]
    k: torch.Tensor        # [L, Hkv, D]
    v: torch.Tensor        # [L, Hkv, D]
    seg_centre: torch.Tensor  # [L] centre index of each position
    centres: torch.Tensor  # [Hkv, M, D] fp32


def segment_lengths(length: int, gen: torch.Generator, *, lo: int, hi: int, log_uniform: bool):
    lens = []
    total = 0
    while total < length:
        if log_uniform:
            u = torch.rand(1, generator=gen).item()
            n = int(round(math.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))))
        else:
            n = int(torch.randint(lo, hi + 1, (1,), generator=gen).item())
        n = max(1, min(n, length - total))
        lens.append(n)
        total += n
    return torch.tensor(lens, dtype=torch.int64)


def mixture_layer(length: int, num_q_heads: int, num_kv_heads: int, head_dim: int, *,
                  mixtures: int, seg=(32, 256), log_uniform: bool = False, sinks: int = 0,
                  sigma_k: float = 0.3, sigma_q: float = 0.5, seed: int = 0,
                  dtype=torch.bfloat16, device="cpu", num_queries: int | None = None) -> LayerInputs:
    """Inputs of one layer.  Generated on ``device`` with a generator seeded there;
    ``num_queries`` (default all) limits the queries to the first positions."""
    cpu = torch.Generator().manual_seed(seed)
    lens = segment_lengths(length, cpu, lo=seg[0], hi=seg[1], log_uniform=log_uniform)
    seg_c = torch.randint(0, mixtures, (lens.numel(),), generator=cpu)
    which = seg_c.repeat_interleave(lens)[:length].to(device)
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    g = num_q_heads // num_kv_heads
    centres = torch.randn(num_kv_heads, mixtures, head_dim, generator=gen, device=device)
    k = centres[:, which].permute(1, 0, 2)
    k = k + sigma_k * torch.randn(length, num_kv_heads, head_dim, generator=gen, device=device)
    if sinks:
        k[:sinks] = k[:sinks] * 8.0
    nq = length if num_queries is None else int(num_queries)
    qc = centres[:, which[:nq]].permute(1, 0, 2).repeat_interleave(g, dim=1)
    q = qc + sigma_q * torch.randn(nq, num_q_heads, head_dim, generator=gen, device=device)
    v = torch.randn(length, num_kv_heads, head_dim, generator=gen, device=device)
    return LayerInputs(q=q.to(dtype).contiguous(), k=k.to(dtype).contiguous(),
                       v=v.to(dtype).contiguous(), seg_centre=which, centres=centres)


def decode_queries(inputs: LayerInputs, steps: int, num_q_heads: int, *, sigma_q: float = 0.5,
                   seed: int = 0, dtype=torch.bfloat16):
    """Decode-step queries and new K/V: each step's query follows a random segment centre."""
    centres = inputs.centres
    hkv, m, d = centres.shape
    g = num_q_heads // hkv
    dev = centres.device
    gen = torch.Generator(device=dev).manual_seed(seed + 7)
    pick = torch.randint(0, m, (steps,), generator=gen, device=dev)
    qc = centres[:, pick].permute(1, 0, 2).repeat_interleave(g, dim=1)
    q = qc + sigma_q * torch.randn(steps, num_q_heads, d, generator=gen, device=dev)
    kn = centres[:, pick].permute(1, 0, 2) + 0.3 * torch.randn(steps, hkv, d, generator=gen, device=dev)
    vn = torch.randn(steps, hkv, d, generator=gen, device=dev)
    return q.to(dtype).contiguous(), kn.to(dtype).contiguous(), vn.to(dtype).contiguous()


# The BASELINE configurations (shape only; 5 is the full model and is not built here).
CONFIGS = {
    1: dict(length=8192, hq=8, hkv=2, d=128, mixtures=64, seg=(32, 256), log_uniform=False,
            sinks=0, dtype=torch.float32, chunk=8192, decode_steps=16),
    2: dict(length=32768, hq=16, hkv=4, d=256, mixtures=256, seg=(32, 256), log_uniform=False,
            sinks=0, dtype=torch.bfloat16, chunk=8192, decode_steps=64, shuffle_suffix=True),
    3: dict(length=131072, hq=16, hkv=4, d=256, mixtures=1024, seg=(16, 2048), log_uniform=True,
            sinks=4, dtype=torch.bfloat16, chunk=8192, decode_steps=256),
    4: dict(length=524288, hq=16, hkv=4, d=256, mixtures=1024, seg=(16, 2048), log_uniform=True,
            sinks=0, dtype=torch.bfloat16, chunk=8192, decode_steps=128,
            order="token", fit_tokens=65536),
}
