"""Synthetic KV / query generators for the benchmark configurations.

Distributions follow the benchmark definitions: each K/V vector has an iid
N(0, 1) direction, normalised, times a lognormal norm; the query is N(0, 1).
Everything is generated directly on the target device from a seeded
``torch.Generator`` so no host copies are involved.
"""

from __future__ import annotations

import math

import torch


def kv_bf16(shape: tuple[int, int, int, int], *, seed: int, mu: float = math.log(20.0), sigma: float = 0.3,
            device: torch.device | str = "cuda", outlier_channels: int = 0, outlier_scale: float = 10.0) -> torch.Tensor:
    """[B, H, N, D] bf16 with unit directions scaled by lognormal(mu, sigma) norms."""
    gen = torch.Generator(device=device).manual_seed(seed)
    B, H, N, D = shape
    x = torch.randn(B, H, N, D, generator=gen, device=device, dtype=torch.float32)
    x = x / x.norm(dim=-1, keepdim=True)
    nrm = torch.exp(mu + sigma * torch.randn(B, H, N, generator=gen, device=device, dtype=torch.float32))
    x = x * nrm[..., None]
    if outlier_channels:
        x[..., :outlier_channels] *= outlier_scale
    return x.to(torch.bfloat16)


def query_bf16(batch: int, heads: int, dim: int, *, seed: int, device: torch.device | str = "cuda") -> torch.Tensor:
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(batch, heads, dim, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
