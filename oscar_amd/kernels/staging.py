"""Host wrapper of the FP32 window (staging arena) write kernel.

Replaces the torch body of the reference's _staging_write
(oscar_ascend/backend.py:439-481): no host synchronisation (no ``nonzero``,
no ``.tolist()`` of device data), last writer per seat decided on the GPU.
"""
from __future__ import annotations

import torch

from . import _lib


def arena_geometry(bs: int, sink: int, recent: int, staging: int):
    """backend.py:421-430 — (sink_eff, sink_pages, tail_pages, rows)."""
    sink_eff = (sink // bs) * bs
    sink_pages = sink_eff // bs
    tail_pages = (recent + bs - 1) // bs + 1
    rows = max((staging + bs - 1) // bs, sink_pages + tail_pages + 2)
    return sink_eff, sink_pages, tail_pages, rows


IMAGE_HALFS = 16 * 64 * 8      # one operand image of a 32-token tile: 16 blocks x 64 lanes x 8


def _k_image_order() -> torch.Tensor:
    """Feature at (g, m, u) of the K image: 128g + 16(m // 2) + 4(m % 2) + u // 2 + 8(u % 2)."""
    g = torch.arange(2).view(2, 1, 1)
    m = torch.arange(16).view(1, 16, 1)
    u = torch.arange(8).view(1, 1, 8)
    return (128 * g + 16 * (m // 2) + 4 * (m % 2) + u // 2 + 8 * (u % 2)).reshape(-1)


def _v_image_tokens() -> torch.Tensor:
    """Token at (s, gs, u) of the V image: 16s + 8gs + (0, 2, 1, 3, 4, 6, 5, 7)[u]."""
    order = torch.tensor([0, 2, 1, 3, 4, 6, 5, 7])
    s = torch.arange(2).view(2, 1, 1)
    gs = torch.arange(2).view(1, 2, 1)
    return (16 * s + 8 * gs + order.view(1, 1, 8)).reshape(-1)


def image_shape(rows: int, bs: int, hk: int) -> tuple:
    """Shape of the V operand image of an arena: a high and a low fp16 part
    per lane slot."""
    return (rows, bs // 32, hk, 2 * IMAGE_HALFS)


def k_image_shape(rows: int, bs: int, hk: int) -> tuple:
    """Shape of the K operand image: a high and a low fp16 part per tile."""
    return (rows, bs // 32, hk, 2 * IMAGE_HALFS)


def check_arena(stage_k, stage_v, owner, bs: int, hk: int, d: int) -> int:
    """Raise unless (stage_k, stage_v, owner) is an arena the kernels can
    index from its geometry: contiguous fp32 [rows, bs, Hk, D] values and an
    int64 [rows, bs] owner table on one device.  Returns rows."""
    rows = owner.shape[0] if owner.ndim == 2 else -1
    want = (rows, bs, hk, d)
    if owner.dtype != torch.int64 or tuple(owner.shape) != (rows, bs) or not owner.is_contiguous():
        raise ValueError(f"staging owner must be a contiguous int64 [rows, {bs}] tensor")
    for t in (stage_k, stage_v):
        if t.dtype != torch.float32 or tuple(t.shape) != want or not t.is_contiguous() or t.device != owner.device:
            raise ValueError(f"staging values must be contiguous fp32 {want} tensors on the owner's device")
    return rows


def winner_buffer(rows: int, bs: int, device) -> torch.Tensor:
    """The seat-winner buffer of an arena's bulk writes: int64, one key per
    seat, then the call epoch and an arrival counter; zero once, kept across
    calls (the kernels never need it reset)."""
    return torch.zeros(rows * bs + 2, dtype=torch.int64, device=device)


def check_winner(winner, rows: int, bs: int) -> None:
    if winner is None or winner.dtype != torch.int64 or winner.ndim != 1 or winner.numel() != rows * bs + 2 \
            or not winner.is_contiguous():
        raise ValueError(f"seat winners must be a contiguous int64 [{rows * bs + 2}] buffer (winner_buffer)")


def check_images(k_image, v_image, rows: int, bs: int, hk: int) -> None:
    """Raise unless the operand images are absent together or are contiguous
    fp16 tensors of the arena's K and V image shapes (the kernels index them
    from the arena geometry alone)."""
    if k_image is None and v_image is None:
        return
    kwant, vwant = k_image_shape(rows, bs, hk), image_shape(rows, bs, hk)
    if k_image is None or v_image is None or tuple(k_image.shape) != kwant or tuple(v_image.shape) != vwant \
            or k_image.dtype != torch.float16 or v_image.dtype != torch.float16 \
            or not (k_image.is_contiguous() and v_image.is_contiguous()):
        raise ValueError(f"staging operand images must be contiguous fp16 {kwant} (K) and {vwant} (V)")


def stage_images(stage_k: torch.Tensor, stage_v: torch.Tensor):
    """fp16 operand images of a whole arena (the layout oscar_staging_write
    maintains incrementally): K [rows][bs/32][Hk][part][m][lane = t + 32g][slot],
    V [rows][bs/32][Hk][q][b][s][lane = m + 32gs][part][slot] with feature
    64q + 4(m // 2) + 2b + m % 2; part 0 = RNE fp16(x), part 1 = RNE
    fp16(x - part 0)."""
    rows, bs, hk, d = stage_k.shape
    if d != 256 or bs % 32:
        raise ValueError("operand images need D = 256 and a block size that is a multiple of 32")
    T = bs // 32
    dev = stage_k.device
    xf = stage_k.view(rows, T, 32, hk, d).float()[..., _k_image_order().to(dev)]
    hi = xf.to(torch.float16)
    lo = (xf - hi.float()).to(torch.float16)
    parts = []
    for x in (hi, lo):
        x = x.view(rows, T, 32, hk, 2, 16, 8).permute(0, 1, 3, 5, 4, 2, 6)  # [r, T, hk, m, g, t, u]
        parts.append(x.reshape(rows, T, hk, IMAGE_HALFS))
    kimg = torch.cat(parts, -1).contiguous()
    yf = stage_v.view(rows, T, 32, hk, d).float().permute(0, 1, 3, 4, 2)   # [r, T, hk, f, tok]
    yf = yf[..., _v_image_tokens().to(dev)].reshape(rows, T, hk, d, 2, 2, 8)  # [r, T, hk, f, s, gs, u]
    yh = yf.to(torch.float16)
    y = torch.stack((yh, (yf - yh.float()).to(torch.float16)), -2)          # [r, T, hk, f, s, gs, part, u]
    y = y.reshape(rows, T, hk, 4, 16, 2, 2, 2, 2, 2, 8)                     # f = (q, bl, b, e)
    y = y.permute(0, 1, 2, 3, 5, 7, 8, 4, 6, 9, 10)                          # [r, T, hk, q, b, s, gs, (bl, e), part, u]
    vimg = y.reshape(rows, T, hk, 2 * IMAGE_HALFS).contiguous()
    return kimg, vimg


def staging_write(key, value, slot_mapping, qsl_dev, seq_dev, num_requests: int, num_kv_heads: int,
                  head_size: int, block_size: int, sink_eff: int, recent: int, R_k, R_v,
                  stage_k, stage_v, owner, winner, k_image=None, v_image=None) -> None:
    N = slot_mapping.shape[0]
    if N == 0 or num_requests == 0:
        return
    kr = key[:N].reshape(N, -1)
    vr = value[:N].reshape(N, -1)
    if kr.dtype != torch.bfloat16 or vr.dtype != torch.bfloat16:
        raise ValueError("staging write takes bf16 key/value")
    if kr.stride(1) != 1 or vr.stride(0) != kr.stride(0) or vr.stride(1) != 1:
        kr, vr = kr.contiguous(), vr.contiguous()
    slots = slot_mapping.to(torch.int64).contiguous()
    check_arena(stage_k, stage_v, owner, block_size, num_kv_heads, head_size)
    check_images(k_image, v_image, owner.shape[0], block_size, num_kv_heads)
    check_winner(winner, owner.shape[0], block_size)
    _lib.call("oscar_staging_write", _lib.ptr(kr), _lib.ptr(vr), kr.stride(0), _lib.ptr(slots), N,
              _lib.ptr(qsl_dev), _lib.ptr(seq_dev), num_requests, num_kv_heads, head_size, block_size,
              owner.shape[0], sink_eff, recent, _lib.ptr(R_k), _lib.ptr(R_v), _lib.ptr(stage_k),
              _lib.ptr(stage_v), _lib.ptr(owner), _lib.ptr(winner), _lib.ptr(k_image), _lib.ptr(v_image),
              _lib.stream_handle(key.device))
