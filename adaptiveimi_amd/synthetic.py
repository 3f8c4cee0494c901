"""Seeded synthetic inputs with the BASELINE config-0 distributions.

Keys: N(0,1) per channel times a per-(head, channel) log-normal(0,1) factor,
then Llama rotate-half RoPE (theta) at positions 0..T-1, cast to bf16.
Values: N(0,1) bf16.  Queries: for each q head, the mean of 16 distinct
random key rows of its KV group plus N(0, 0.5^2) noise, bf16.
Generated with torch on any device; the same seed gives the same tensors on
CPU and GPU only up to the device RNG, so parity tests generate on the CPU and
copy.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch


def rope(x: torch.Tensor, theta: float, positions: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE on [..., T, D] (fp32), angles computed in fp64."""
    D = x.shape[-1]
    half = D // 2
    inv = theta ** (-torch.arange(0, half, dtype=torch.float64, device=x.device) * 2.0 / D)
    ang = positions.to(torch.float64)[:, None] * inv[None, :]
    cos = torch.cos(ang).to(torch.float32)
    sin = torch.sin(ang).to(torch.float32)
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def make_kv(H: int, T: int, D: int = 128, theta: float = 500000.0, seed: int = 0,
            device: str = "cpu", position_offset: int = 0, chunk: int = 32768) -> Tuple[torch.Tensor, torch.Tensor]:
    """Keys/values [H, T, D] bf16 (generated in chunks to bound fp32 memory)."""
    g = torch.Generator(device=device).manual_seed(seed)
    scale = torch.exp(torch.randn((H, 1, D), generator=g, device=device))
    keys = torch.empty((H, T, D), dtype=torch.bfloat16, device=device)
    values = torch.empty((H, T, D), dtype=torch.bfloat16, device=device)
    for s in range(0, T, chunk):
        e = min(T, s + chunk)
        x = torch.randn((H, e - s, D), generator=g, device=device) * scale
        pos = torch.arange(s + position_offset, e + position_offset, device=device)
        keys[:, s:e] = rope(x, theta, pos).to(torch.bfloat16)
        values[:, s:e] = torch.randn((H, e - s, D), generator=g, device=device).to(torch.bfloat16)
    return keys, values


def make_queries(keys: torch.Tensor, groups: int, seed: int = 1, planted: int = 16,
                 noise_std: float = 0.5, n_queries: int = 1) -> torch.Tensor:
    """Queries [n_queries, H, G, D] bf16 built from planted key rows."""
    H, T, D = keys.shape
    dev = keys.device
    g = torch.Generator(device=dev).manual_seed(seed)
    out = torch.empty((n_queries, H, groups, D), dtype=torch.bfloat16, device=dev)
    for n in range(n_queries):
        for h in range(H):
            for j in range(groups):
                idx = torch.randperm(T, generator=g, device=dev)[:planted]
                base = keys[h, idx].to(torch.float32).mean(dim=0)
                noise = torch.randn((D,), generator=g, device=dev) * noise_std
                out[n, h, j] = (base + noise).to(torch.bfloat16)
    return out


def integer_kv(H: int, T: int, D: int = 128, lo: int = -4, hi: int = 4, seed: int = 0,
               device: str = "cpu") -> Tuple[torch.Tensor, torch.Tensor]:
    """Small-integer keys/values: every fp32 sum in the E-step and the
    scoring chain is exact, so ties are real and the tie rules are testable."""
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randint(lo, hi + 1, (H, T, D), generator=g, device=device).to(torch.bfloat16)
    v = torch.randint(lo, hi + 1, (H, T, D), generator=g, device=device).to(torch.bfloat16)
    return k, v
