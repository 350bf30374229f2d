"""Seeded synthetic inputs of the benchmark / parity workloads.

K/V are fp32 N(0, 1) with four fixed outlier channels scaled x8, cast to the
model dtype (bf16); queries are bf16 N(0, 1); rotations are the Q factor of a
seeded Gaussian matrix (the reference's own test recipe,
tests/test_backend.py:167-168).  Everything is generated on the CPU with an
explicit torch.Generator so the GPU run and the CPU oracle see identical bits.
"""
from __future__ import annotations

import torch

OUTLIER_CHANNELS = (7, 71, 135, 199)
OUTLIER_SCALE = 8.0


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def kv(n: int, hk: int, D: int, seed: int, dtype=torch.bfloat16):
    """(key, value) [n, hk, D] with the outlier channels scaled."""
    g = gen(seed)
    scale = torch.ones(D)
    scale[list(c for c in OUTLIER_CHANNELS if c < D)] = OUTLIER_SCALE
    k = (torch.randn(n, hk, D, generator=g) * scale).to(dtype)
    v = (torch.randn(n, hk, D, generator=g) * scale).to(dtype)
    return k, v


def queries(n: int, hq: int, D: int, seed: int, dtype=torch.bfloat16):
    return torch.randn(n, hq, D, generator=gen(seed)).to(dtype)


def rotation(D: int, seed: int) -> torch.Tensor:
    return torch.linalg.qr(torch.randn(D, D, generator=gen(seed))).Q.contiguous()


def rotations(D: int, seed: int):
    return rotation(D, seed), rotation(D, seed + 1)


def page_permutation(num_pages: int, seed: int) -> torch.Tensor:
    return torch.randperm(num_pages, generator=gen(seed)).to(torch.int32)


def slots_for(block_row: torch.Tensor, start: int, count: int, bs: int) -> torch.Tensor:
    """Physical slots of absolute positions start .. start+count-1 of one request."""
    pos = torch.arange(start, start + count)
    return block_row[pos // bs].to(torch.int64) * bs + pos % bs
