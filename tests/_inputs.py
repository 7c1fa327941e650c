"""Seeded synthetic inputs shared by the tests and the benchmark.

Every tensor is drawn on the CPU from its own ``torch.Generator`` (x = seed 0, w = 1, bias = 2,
outlier rows = 3 by default), so the GPU kernels, the fp64 oracle and the CPU baseline see
identical bits.
"""
from __future__ import annotations

import torch


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, seed: int, scale: float = 1.0, dtype=torch.float32) -> torch.Tensor:
    t = torch.randn(*shape, generator=gen(seed), dtype=torch.float32)
    if scale != 1.0:
        t = t * scale
    return t.to(dtype)


def outlier_rows(x: torch.Tensor, frac: float, lo: float, hi: float, seed: int = 3) -> torch.Tensor:
    """Scale round(frac*M) seeded rows of fp32 ``x`` so that each one's |max| is drawn from
    U[lo, hi] (the C4 configuration). Returns the modified copy."""
    x = x.clone()
    M = x.shape[0]
    n = int(round(frac * M))
    g = gen(seed)
    rows = torch.randperm(M, generator=g)[:n]
    t = lo + (hi - lo) * torch.rand(n, generator=g, dtype=torch.float64)
    for r, target in zip(rows.tolist(), t.tolist()):
        amax = x[r].abs().max().item()
        x[r] = (x[r].double() * (target / amax)).float()
    return x
