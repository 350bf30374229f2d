"""Host wrapper of the fused short-step write kernel (oscar_step_write).

For a step of at most MAX_STEP_TOKENS new tokens (MTP decode), one launch
does what the reference does before its paged read
(oscar_ascend/backend.py:150-189, 261-269, 291-295, 439-481): q/k/v rotated
in fp32, the INT2 write of k/v (clip, quantize, pack, slot write) and the
FP32 window write with its fp16 operand images.  Returns the rotated q, k, v
the read kernels take.
"""
from __future__ import annotations

import ctypes

import torch

from ..format import check_d
from . import _lib, decode, staging
from .quant import cache_geometry

MAX_STEP_TOKENS = 1024


def _rows(x: torch.Tensor, N: int, features: int) -> tuple[torch.Tensor, int]:
    if x.dtype != torch.bfloat16:
        raise ValueError(f"step write takes bf16 query/key/value, got {x.dtype}")
    rows = x[:N].reshape(N, -1)
    if rows.shape[1] != features:
        raise ValueError(f"expected {features} features per token, got {rows.shape[1]}")
    if rows.stride(1) != 1:
        rows = rows.contiguous()
    return rows, rows.stride(0)


def step_write(query, key, value, R_k, R_v, slot_mapping, qsl, seqs, k_cache, v_cache, clip_k: int,
               clip_v: int, num_heads: int, num_kv_heads: int, stage=None, sink_eff: int = 0, recent: int = 0,
               out=None):
    """query [N, Hq*D] / key, value [N, Hk*D] bf16 (any leading shape), R_k / R_v fp32 [D, D];
    qsl / seqs host lists; stage = (stage_k, stage_v, owner, k_image, v_image) or None.
    Returns (q_rot [N, Hq, D], k_rot [N, Hk, D], v_rot [N, Hk, D]) fp32 (``out``: those three, reused)."""
    N = slot_mapping.shape[0]
    D = R_k.shape[0]
    check_d(D)
    if N > MAX_STEP_TOKENS:
        raise ValueError(f"step write takes at most {MAX_STEP_TOKENS} tokens, got {N}")
    dev = query.device
    if out is None:
        out = (torch.empty(N, num_heads, D, dtype=torch.float32, device=dev),
               torch.empty(N, num_kv_heads, D, dtype=torch.float32, device=dev),
               torch.empty(N, num_kv_heads, D, dtype=torch.float32, device=dev))
    if N == 0:
        return out
    qr, qs = _rows(query, N, num_heads * D)
    kr, ks = _rows(key, N, num_kv_heads * D)
    vr, vs = _rows(value, N, num_kv_heads * D)
    if ks != vs:
        kr, vr = kr.contiguous(), vr.contiguous()
        ks = kr.stride(0)
    for t in (R_k, R_v):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.device != dev:
            raise ValueError("rotations must be contiguous fp32 tensors on the query's device")
    slots = slot_mapping.to(device=dev, dtype=torch.int64).contiguous()
    B = len(qsl) - 1
    if len(seqs) < B:
        raise ValueError("one sequence length per request")
    lay = decode.request_layout(qsl, seqs[:B])
    qstart, seq_t = lay.qstart, lay.seq_t
    bs, pages, kst, vst = cache_geometry(k_cache, v_cache)
    if stage is not None:
        sk, sv, owner = stage[0], stage[1], stage[2]
        kimg = stage[3] if len(stage) > 3 else None
        vimg = stage[4] if len(stage) > 4 else None
        rows = owner.shape[0]
        if owner.dtype != torch.int64 or owner.shape[1] != bs:
            raise ValueError("staging owner must be int64 [rows, block_size]")
        staging.check_images(kimg, vimg, rows, bs, num_kv_heads)
    else:
        sk = sv = owner = kimg = vimg = None
        rows = 0
    _lib.call("oscar_step_write", _lib.ptr(qr), qs, _lib.ptr(kr), _lib.ptr(vr), ks, N, num_heads, num_kv_heads, D,
              _lib.ptr(R_k), _lib.ptr(R_v), _lib.ptr(slots), ctypes.addressof(qstart), ctypes.addressof(seq_t), B,
              _lib.ptr(k_cache), _lib.ptr(v_cache), bs, pages, *kst, *vst, clip_k, clip_v, _lib.ptr(sk),
              _lib.ptr(sv), _lib.ptr(owner), _lib.ptr(kimg), _lib.ptr(vimg), rows, int(sink_eff), int(recent),
              _lib.ptr(out[0]), _lib.ptr(out[1]), _lib.ptr(out[2]), _lib.stream_handle(dev))
    return out
