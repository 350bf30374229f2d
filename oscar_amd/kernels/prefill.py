"""Host wrapper of the prefill-continuation kernel (kernel 3).

Replaces the reference's per-request dense read path for long requests
(oscar_ascend/backend.py:361-415: oscar_full_dequant + _stage_splice +
oscar_prefill / the vendor fused attention op, prefill.py:21-72): one launch
computes causal attention of the request's new tokens over its INT2 history
(owner-matched FP32 window values override) plus themselves, dequantizing
history tiles in LDS; nothing is materialised in HBM.
"""
from __future__ import annotations

import torch

from ..format import check_d
from . import _lib
from .quant import cache_geometry


def prefill_continuation(q_rot, k_rot, v_rot, kc, vc, bt_row, cached_len: int, scale: float,
                         stage=None) -> torch.Tensor:
    """q_rot [N, Hq, D], k_rot / v_rot [N, Hk, D] (rotated, any float dtype);
    returns the rotated-V-domain output, fp32 [N, Hq, D]."""
    N, hq, d = q_rot.shape
    check_d(d)
    hk = k_rot.shape[1]
    dev = q_rot.device
    out = torch.empty(N, hq, d, dtype=torch.float32, device=dev)
    if N == 0:
        return out
    q = q_rot.float().contiguous()
    k = k_rot.float().contiguous()
    v = v_rot.float().contiguous()
    bt = bt_row.to(device=dev, dtype=torch.int32).contiguous().reshape(-1)
    bs, pages, kst, vst = cache_geometry(kc, vc)
    if stage is not None:
        sk, sv, owner = stage[:3]
        sk, sv = sk.float().contiguous(), sv.float().contiguous()
        owner = owner.to(torch.int64).contiguous()
        rows = owner.shape[0]
    else:
        sk = sv = owner = None
        rows = 0
    _lib.call("oscar_prefill_continuation", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), N, hq, hk, d,
              _lib.ptr(kc), _lib.ptr(vc), bs, pages, *kst, *vst, _lib.ptr(bt), bt.numel(),
              int(cached_len), _lib.ptr(sk), _lib.ptr(sv), _lib.ptr(owner), rows, float(scale),
              _lib.ptr(out), _lib.stream_handle(dev))
    return out
