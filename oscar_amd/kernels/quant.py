"""Host wrappers of the quantize-write kernels (kernel 1).

Mirrors the reference store seam ``oscar_store_triton(k_rot, v_rot, k_cache,
v_cache, slot_mapping)`` (oscar_ascend/kernels/store_kernel.py:247-279) plus
the rotate/clip step that precedes it (oscar_ascend/backend.py:129-147).
"""
from __future__ import annotations

import torch

from ..format import HEAD_DIM, check_d
from . import _lib, staging


def clip_index(ratio: float, D: int) -> int:
    """Sorted-|x| index of the clip threshold, -1 for no clip
    (backend.py:131, 141: ``min(int(ratio * D), D - 1)`` when ratio > 0)."""
    return min(int(ratio * D), D - 1) if ratio > 0.0 else -1


def cache_geometry(k_cache: torch.Tensor, v_cache: torch.Tensor):
    """(block_size, pages, K byte strides, V byte strides) of contiguous paged caches
    (pages, block_size, Hk, W) viewed as uint8 (backend.py:202-216)."""
    k8, v8 = k_cache.view(torch.uint8), v_cache.view(torch.uint8)
    if k8.ndim != 4 or v8.ndim != 4 or not k8.is_contiguous() or not v8.is_contiguous():
        raise ValueError("OSCAR requires contiguous [blocks, tokens, heads, bytes] caches")
    if k8.shape[:3] != v8.shape[:3]:
        raise ValueError("K and V caches must share (blocks, block_size, heads)")
    return k8.shape[1], k8.shape[0], tuple(k8.stride()[:3]), tuple(v8.stride()[:3])


def _check_device(*tensors):
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("OSCAR kernels take device tensors")


def rotation_operand(R: torch.Tensor) -> torch.Tensor:
    """Operand of rotation R [D, D] (x_rot = x @ R), uint8 bytes on R's device:
    the MFMA tiles (bf16 high + low parts), then R in fp32 for short writes."""
    D = R.shape[0]
    check_d(D)
    if R.shape != (D, D):
        raise ValueError("rotation must be square")
    _check_device(R)
    R = R.float().contiguous()
    nbytes = _lib.load().oscar_rotation_operand_bytes(D)
    if nbytes == 0:
        raise _lib.OscarKernelError(f"unsupported head size {D} (kernels are written for D = {HEAD_DIM})")
    out = torch.empty(nbytes, dtype=torch.uint8, device=R.device)
    _lib.call("oscar_rotation_operand", _lib.ptr(R), _lib.ptr(out), D, _lib.stream_handle(R.device))
    return out


def rotate_rows(x: torch.Tensor, operand: torch.Tensor, out_dtype=torch.float32, out=None) -> torch.Tensor:
    """x @ R on MFMA for every D-feature row of x ([..., D], bf16 or fp32), R
    given by its operand (rotation_operand); fp32 or bf16 result of x's shape,
    written into `out` when given (a contiguous tensor of that shape).
    Replaces the prefill route's fp32 rotations (backend.py:392-413)."""
    D = x.shape[-1]
    check_d(D)
    if x.dtype not in (torch.bfloat16, torch.float32) or out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("rotate_rows takes bf16 or fp32 rows and returns fp32 or bf16")
    _check_device(x, operand)
    rows = x.numel() // D
    xr = x.reshape(rows, D)
    if xr.stride(1) != 1 or xr.data_ptr() % 16 or (xr.stride(0) * xr.element_size()) % 16:
        xr = xr.contiguous()
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    if out.dtype != out_dtype or out.shape != x.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of x's shape and the output dtype")
    orr = out.view(rows, D)
    _lib.call("oscar_rotate_rows", _lib.ptr(xr), int(x.dtype == torch.float32), xr.stride(0), rows, D,
              _lib.ptr(operand), _lib.ptr(orr), int(out_dtype == torch.bfloat16), orr.stride(0),
              _lib.stream_handle(x.device))
    return out


def _token_rows(x: torch.Tensor, N: int, hk: int, D: int, dtype) -> tuple[torch.Tensor, int]:
    if x.dtype != dtype:
        raise ValueError(f"expected {dtype}, got {x.dtype}")
    rows = x[:N].reshape(N, -1)
    if rows.shape[1] != hk * D:
        raise ValueError("input does not have Hk * D features per token")
    if rows.stride(1) != 1:
        rows = rows.contiguous()
    return rows, rows.stride(0)


def quant_write_prerotated(k_rot, v_rot, k_cache, v_cache, slot_mapping, clip_k: int, clip_v: int) -> None:
    """Clip + quantize + pack + write pre-rotated fp32 K/V [N, Hk, D]."""
    N, hk, D = k_rot.shape
    check_d(D)
    if N == 0:
        return
    _check_device(k_rot, v_rot, k_cache, v_cache, slot_mapping)
    kr, ks = _token_rows(k_rot, N, hk, D, torch.float32)
    vr, vs = _token_rows(v_rot, N, hk, D, torch.float32)
    if ks != vs:
        kr, vr = kr.contiguous(), vr.contiguous()
        ks = kr.stride(0)
    slots = slot_mapping[:N].to(torch.int64).contiguous()
    bs, pages, kst, vst = cache_geometry(k_cache, v_cache)
    _lib.call("oscar_quant_write_prerotated", _lib.ptr(kr), _lib.ptr(vr), N, hk, D, ks,
              _lib.ptr(slots), _lib.ptr(k_cache), _lib.ptr(v_cache), bs, pages, *kst, *vst,
              clip_k, clip_v, _lib.stream_handle(k_rot.device))


def quant_write(key, value, rot_k_op, rot_v_op, k_cache, v_cache, slot_mapping, clip_k: int,
                clip_v: int, num_kv_heads: int, head_size: int, window=None) -> None:
    """Fused rotate + clip + quantize + pack + write of bf16 K/V: the rotation
    runs on MFMA, or in fp32 for writes of at most 2048 key + value vectors.
    window: None, or (query_start, seq_lens, num_requests, sink_eff, recent,
    stage_k, stage_v, owner, winner, k_image, v_image) -- the step's request
    layout (int32 device tensors) and the window arena, whose write (the
    reference's _staging_write, backend.py:439-481) then comes from the same
    rotated values in the same call."""
    N = slot_mapping.shape[0]
    if N == 0:
        return
    hk, D = num_kv_heads, head_size
    check_d(D)
    _check_device(key, value, k_cache, v_cache, slot_mapping, rot_k_op, rot_v_op)
    kr, ks = _token_rows(key, N, hk, D, torch.bfloat16)
    vr, vs = _token_rows(value, N, hk, D, torch.bfloat16)
    if ks != vs:
        kr, vr = kr.contiguous(), vr.contiguous()
        ks = kr.stride(0)
    slots = slot_mapping.to(torch.int64).contiguous()
    bs, pages, kst, vst = cache_geometry(k_cache, v_cache)
    common = (_lib.ptr(kr), _lib.ptr(vr), N, hk, D, ks, _lib.ptr(rot_k_op), _lib.ptr(rot_v_op), _lib.ptr(slots),
              _lib.ptr(k_cache), _lib.ptr(v_cache), bs, pages, *kst, *vst, clip_k, clip_v)
    if window is None:
        _lib.call("oscar_quant_write", *common, _lib.stream_handle(key.device))
        return
    qsl, seqs, B, sink_eff, recent, sk, sv, owner, winner, kimg, vimg = window
    rows = staging.check_arena(sk, sv, owner, bs, hk, D)
    staging.check_images(kimg, vimg, rows, bs, hk)
    staging.check_winner(winner, rows, bs)
    for t in (qsl, seqs):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError("the request layout must be contiguous int32 device tensors")
    _lib.call("oscar_quant_write_window", *common, _lib.ptr(qsl), _lib.ptr(seqs), B, rows, sink_eff, recent,
              _lib.ptr(sk), _lib.ptr(sv), _lib.ptr(owner), _lib.ptr(winner), _lib.ptr(kimg), _lib.ptr(vimg),
              _lib.stream_handle(key.device))
