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


def staging_write(key, value, slot_mapping, qsl_dev, seq_dev, num_requests: int, num_kv_heads: int,
                  head_size: int, block_size: int, sink_eff: int, recent: int, R_k, R_v,
                  stage_k, stage_v, owner, winner) -> None:
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
    _lib.call("oscar_staging_write", _lib.ptr(kr), _lib.ptr(vr), kr.stride(0), _lib.ptr(slots), N,
              _lib.ptr(qsl_dev), _lib.ptr(seq_dev), num_requests, num_kv_heads, head_size, block_size,
              owner.shape[0], sink_eff, recent, _lib.ptr(R_k), _lib.ptr(R_v), _lib.ptr(stage_k),
              _lib.ptr(stage_v), _lib.ptr(owner), _lib.ptr(winner), _lib.stream_handle(key.device))
