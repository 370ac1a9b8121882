"""Seeded synthetic inputs for the benchmark configurations (no datasets or checkpoints exist here).

Values are N(0, 1) from torch's seeded generator (``torch.Generator(device).manual_seed(seed)``)
drawn in fp32 and rounded to the target dtype.  "2% outlier channels x8" selects
``round(0.02 * C)`` channels of the flattened trailing axis ``C = H * D`` (31 of 1536) with a seeded
permutation (CPU generator, seed + 1) and multiplies them by 8 before the dtype cast.
"""
from __future__ import annotations

import math
from typing import Sequence

import torch


def outlier_channels(C: int, seed: int, frac: float = 0.02) -> torch.Tensor:
    n = int(round(frac * C))
    g = torch.Generator().manual_seed(seed + 1)
    return torch.randperm(C, generator=g)[:n]


def normal_with_outliers(shape: Sequence[int], seed: int, *, dtype=torch.bfloat16, outlier_frac: float = 0.02,
                         factor: float = 8.0, device="cpu", trailing_dims: int = 2) -> torch.Tensor:
    """N(0,1) tensor of `shape`; outlier channels index the product of the last `trailing_dims` dims."""
    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(tuple(shape), generator=g, dtype=torch.float32, device=device)
    if outlier_frac > 0:
        tdims = min(trailing_dims, len(shape))
        C = int(math.prod(shape[len(shape) - tdims:]))
        ch = outlier_channels(C, seed, outlier_frac).to(device)
        flat = x.view(-1, C)
        flat[:, ch] *= factor
    return x.to(dtype)


def normal(shape: Sequence[int], seed: int, *, dtype=torch.bfloat16, device="cpu") -> torch.Tensor:
    g = torch.Generator(device=torch.device(device)).manual_seed(seed)
    return torch.randn(tuple(shape), generator=g, dtype=torch.float32, device=device).to(dtype)


def rope_interleaved(x: torch.Tensor, positions: torch.Tensor, rope_dim: int = 64, theta: float = 10000.0) -> torch.Tensor:
    """RoPE on the last `rope_dim` dims with interleaved pairs (aether_2b/modeling.py:55-57, :122-155,
    config=None branch): angle = pos * theta^(-2i/rope_dim); cos/sin rounded to x's dtype."""
    pass_part, rope = x[..., :-rope_dim], x[..., -rope_dim:]
    freqs = torch.arange(0, rope_dim, 2, device=x.device, dtype=torch.float32)
    inv_freq = 1.0 / (theta ** (freqs / rope_dim))
    ang = positions.float().unsqueeze(-1) * inv_freq
    cos = torch.repeat_interleave(ang.cos(), 2, dim=-1).to(x.dtype)
    sin = torch.repeat_interleave(ang.sin(), 2, dim=-1).to(x.dtype)
    while cos.dim() < rope.dim():
        cos = cos.unsqueeze(0)
        sin = sin.unsqueeze(0)
    x1, x2 = rope[..., ::2], rope[..., 1::2]
    rot = torch.stack((-x2, x1), dim=-1).flatten(-2)
    return torch.cat([pass_part, rope * cos + rot * sin], dim=-1)
