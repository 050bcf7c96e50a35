"""Seeded synthetic inputs shared by the GPU parity tests and the benchmark.

Inputs follow the BASELINE configs: fp16 ~N(0,1) keys/values with a seeded set
of outlier key channels scaled by a factor, boost indices from the mean |K|
of seeded calibration tokens ranked in descending order (the profiler's
convention, kitty/sensitivity.py:164-207), pages placed through a shuffled
free list.
"""
from __future__ import annotations

import numpy as np
import torch


def calibrate_boost_idx(calib: torch.Tensor, d_boost: int, sentinel: int) -> torch.Tensor:
    """calib (N, H, D) fp16 calibration keys -> boost_idx (H, D) uint8:
    rank in descending mean |K| for the top d_boost channels, else sentinel."""
    score = calib.float().abs().mean(0)                      # (H, D)
    order = torch.argsort(score, dim=-1, descending=True, stable=True)
    H, D = score.shape
    bi = torch.full((H, D), sentinel, dtype=torch.uint8)
    for r in range(d_boost):
        bi[torch.arange(H), order[:, r]] = r
    return bi


def outlier_keys(gen: torch.Generator, shape, H: int, D: int, n_outlier: int, factor: float,
                 channels: torch.Tensor = None):
    """Random N(0,1) keys (..., H, D) with n_outlier channels per head scaled."""
    k = torch.randn(*shape, H, D, generator=gen)
    if channels is None:
        channels = torch.stack([torch.randperm(D, generator=gen)[:n_outlier] for _ in range(H)])
    for h in range(H):
        k[..., h, channels[h]] *= factor
    return k.half(), channels


def random_pools(gen: torch.Generator, P: int, H: int, D: int, G: int, d_boost: int, bi: torch.Tensor,
                 rng: np.random.Generator = None):
    """Pools filled with arbitrary valid encodings: random code bytes, positive
    fp16 scales and integer zero points within each channel's code range.
    Every byte pattern is a valid packed page, so this exercises the decode
    path on all code values without running a quantiser.  With `rng`, the
    code bytes come from numpy (much faster for GB-sized pools)."""
    sentinel = min(d_boost + 1, 255)

    def code_bytes(shape):
        if rng is not None:
            return torch.from_numpy(rng.integers(0, 256, size=shape, dtype=np.uint8))
        return torch.randint(0, 256, shape, generator=gen, dtype=torch.uint8)

    kb = code_bytes((P, H, D, G // 4))
    kh = code_bytes((P, H, d_boost, G // 4))
    mq = torch.where(bi < sentinel, 15, 3).float()              # (H, D)
    ks = (torch.rand(P, H, D, generator=gen) * 0.6 + 0.05)
    kz = torch.floor(torch.rand(P, H, D, generator=gen) * (mq + 1)).clamp(max=mq)
    km = torch.stack([ks, kz], dim=2).half()
    vp = code_bytes((P, H, G, D // 4))
    vs = torch.rand(P, H, G, generator=gen) * 0.6 + 0.3
    vz = torch.floor(torch.rand(P, H, G, generator=gen) * 4).clamp(max=3)
    vm = torch.stack([vs, vz], dim=3).half()
    return kb, kh, km, vp, vm


def ragged_lengths(seed: int, B: int, lo: int, hi: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(lo, hi + 1, size=B)
