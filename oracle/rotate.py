"""Oracle: fp32 rotation and sort-based clipping.

Restates AscendOscarAttentionBackendImpl._rotate_clip (oscar_ascend/backend.py:129-147).
Test infrastructure only.
"""
from __future__ import annotations

import torch


def clip_index(ratio: float, D: int) -> int:
    """backend.py:141 — idx = min(int(ratio * D), D - 1) (Python float product)."""
    return min(int(ratio * D), D - 1)


def clip(x_rot: torch.Tensor, ratio: float) -> torch.Tensor:
    """backend.py:131-144 — clamp each vector to +-(sorted |x|)[idx].

    A ratio of 0 (or below) leaves the vector unchanged.
    """
    if ratio <= 0.0:
        return x_rot
    idx = clip_index(ratio, x_rot.shape[-1])
    thr = x_rot.abs().sort(dim=-1).values[..., idx:idx + 1]
    return torch.clamp(x_rot, -thr, thr)


def rotate_clip(x: torch.Tensor, R: torch.Tensor, ratio: float) -> torch.Tensor:
    """backend.py:129-147 — (x.float() @ R) then clip; fp32 result."""
    return clip(torch.matmul(x.float(), R.float()), ratio)


def seeded_rotation(D: int, seed: int) -> torch.Tensor:
    """Orthogonal D x D matrix: Q factor of a seeded Gaussian (the reference's
    test/probe recipe, tests/test_backend.py:167-168, delivery/probe_prefill.py:131)."""
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(D, D, generator=g)).Q.contiguous()
