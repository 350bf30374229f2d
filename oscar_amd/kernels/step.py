"""Host wrapper of the fused short-step write kernel (oscar_step_write).

For a step of at most MAX_STEP_TOKENS new tokens (MTP decode), one launch
does what the reference does before its paged read
(oscar_ascend/backend.py:150-189, 261-269, 291-295, 439-481): q/k/v rotated
in fp32, the INT2 write of k/v (clip, quantize, pack, slot write) and the
FP32 window write with its fp16 operand images.  Returns the rotated q, k, v
the read kernels take.

``MtpLayer`` / ``mtp_step`` / ``mtp_forward`` drive oscar_mtp_forward, the
whole forward of a short step in one library call: the layer's half of the
arguments (rotations, caches, window arena) is validated and packed once per
layer, the step's half (request layout, slot mapping, block table, scratch)
once per step and shared by its layers, and each call passes only the
activations and the output.
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
        staging.check_arena(sk, sv, owner, bs, num_kv_heads, D)
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


_p, _i32, _i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64


class MtpLayerArgs(ctypes.Structure):
    """struct oscar_mtp_layer (include/oscar_amd.h)."""
    _fields_ = [("rot_k", _p), ("rot_v", _p), ("rot_v_t", _p), ("k_cache", _p), ("v_cache", _p),
                ("num_pages", _i64), ("k_stride_page", _i64), ("k_stride_token", _i64), ("k_stride_head", _i64),
                ("v_stride_page", _i64), ("v_stride_token", _i64), ("v_stride_head", _i64),
                ("block_size", _i32), ("num_heads", _i32), ("num_kv_heads", _i32), ("head_size", _i32),
                ("clip_index_k", _i32), ("clip_index_v", _i32), ("scale", ctypes.c_float), ("stage_rows", _i32),
                ("stage_k", _p), ("stage_v", _p), ("stage_owner", _p), ("stage_k_image", _p),
                ("stage_v_image", _p), ("sink_eff", _i32), ("recent", _i32)]


class MtpStepArgs(ctypes.Structure):
    """struct oscar_mtp_step (include/oscar_amd.h)."""
    _fields_ = [("num_tokens", _i32), ("num_requests", _i32), ("max_query_len", _i32), ("max_history", _i64),
                ("query_start_loc", _p), ("seq_lens", _p), ("slot_mapping", _p), ("block_table", _p),
                ("block_table_stride", _i64), ("block_table_cols", _i32), ("num_heads", _i32),
                ("num_kv_heads", _i32), ("tiles_per_split", _i32), ("q_rot", _p), ("k_rot", _p), ("v_rot", _p),
                ("workspace", _p), ("workspace_size", ctypes.c_size_t)]


class MtpLayer:
    """The layer half of oscar_mtp_forward, checked and packed once: R_k, R_v,
    R_v^T (fp32 [D, D]), the paged caches and the window arena (stage =
    (stage_k, stage_v, owner, k_image, v_image) or None).  Holds the tensors
    it points at; ``bound_to`` says whether the same tensors are still the
    layer's (identity, so a rebound cache or replaced rotation rebuilds)."""

    __slots__ = ("tensors", "ids", "args", "ref", "num_heads", "num_kv_heads", "head_size")

    def __init__(self, R_k, R_v, R_v_t, k_cache, v_cache, num_heads: int, num_kv_heads: int, clip_k: int,
                 clip_v: int, scale: float, stage=None, sink_eff: int = 0, recent: int = 0):
        D = R_k.shape[0]
        check_d(D)
        dev = k_cache.device
        for t in (R_k, R_v, R_v_t):
            if tuple(t.shape) != (D, D) or t.dtype != torch.float32 or not t.is_contiguous() or t.device != dev:
                raise ValueError("rotations must be contiguous fp32 [D, D] tensors on the caches' device")
        bs, pages, kst, vst = cache_geometry(k_cache, v_cache)
        if bs % 32:
            raise ValueError("paged decode needs a cache block size that is a multiple of 32")
        if k_cache.shape[2] != num_kv_heads or num_heads % num_kv_heads:
            raise ValueError("caches must hold num_kv_heads heads, and num_heads must be a multiple of it")
        arena = (None,) * 5
        rows = 0
        if stage is not None:
            arena = tuple(stage[:5]) if len(stage) >= 5 else tuple(stage[:3]) + (None, None)
            rows = staging.check_arena(arena[0], arena[1], arena[2], bs, num_kv_heads, D)
            if arena[3] is None:
                raise ValueError("the MTP forward needs the arena's fp16 operand images")
            staging.check_images(arena[3], arena[4], rows, bs, num_kv_heads)
            if arena[0].device != dev:
                raise ValueError("the window arena must be on the caches' device")
        self.tensors = (R_k, R_v, R_v_t, k_cache, v_cache) + arena
        self.ids = tuple(map(id, self.tensors))     # stable: the tensors are held here
        self.num_heads, self.num_kv_heads, self.head_size = num_heads, num_kv_heads, D
        ptrs = [_lib.ptr(t) for t in self.tensors]
        self.args = MtpLayerArgs(*ptrs[:5], pages, *kst, *vst, bs, num_heads, num_kv_heads, D, clip_k, clip_v,
                                 float(scale), rows, *ptrs[5:], int(sink_eff), int(recent))
        self.ref = ctypes.addressof(self.args)

    def bound_to(self, *tensors) -> bool:
        """True when ``tensors`` (R_k, R_v, R_v^T, k_cache, v_cache and the
        five arena tensors) are exactly the ones this was built from."""
        return tuple(map(id, tensors)) == self.ids


class MtpStep:
    """The step half of oscar_mtp_forward: the request layout (host arrays),
    slot mapping, block table and the step's scratch (q_rot / k_rot / v_rot
    and the decode workspace).  Shared by every layer of the step; launches
    through it are ordered by their stream, which is part of its cache key."""

    __slots__ = ("layout", "num_tokens", "tensors", "args", "ref", "reusable")

    def __init__(self, layout: decode.RequestLayout, num_tokens: int, slot_mapping, block_table, num_heads: int,
                 num_kv_heads: int, head_size: int, device: torch.device):
        N = num_tokens
        if sum(layout.lengths) != N or layout.qsl[0] != 0:
            raise ValueError("query_start_loc must cover the step's tokens from 0")
        if layout.max_q > decode.MAX_QUERY_LEN:
            raise ValueError(f"the MTP forward takes at most {decode.MAX_QUERY_LEN} query tokens per request")
        B = len(layout.lengths)
        slots, bt = slot_mapping, block_table
        # Tensors the engine owns are used in place, so their contents are
        # read at launch; converted copies tie this step to their contents.
        self.reusable = True
        if slots.dtype != torch.int64 or slots.device != device or not slots.is_contiguous():
            slots = slots.to(device=device, dtype=torch.int64).contiguous()
            self.reusable = False
        if slots.ndim != 1 or slots.shape[0] < N:
            raise ValueError("slot_mapping must hold a slot per token")
        if bt.ndim != 2 or bt.shape[0] < B:
            raise ValueError("block table must be [requests, pages]")
        if bt.dtype != torch.int32 or bt.device != device or bt.stride(1) != 1:
            bt = bt.to(device=device, dtype=torch.int32).contiguous()
            self.reusable = False
        D = head_size
        q_rot = torch.empty(N, num_heads, D, dtype=torch.float32, device=device)
        k_rot = torch.empty(N, num_kv_heads, D, dtype=torch.float32, device=device)
        v_rot = torch.empty_like(k_rot)
        need = _lib.load().oscar_paged_decode_workspace_bytes(B, num_kv_heads, num_heads, max(layout.max_q, 1),
                                                              layout.max_hist, 0)
        ws = decode.workspace(device, need)
        self.layout, self.num_tokens = layout, N
        self.tensors = (slots, bt, q_rot, k_rot, v_rot, ws)
        self.args = MtpStepArgs(N, B, layout.max_q, layout.max_hist, ctypes.addressof(layout.qstart),
                                ctypes.addressof(layout.seq_t), _lib.ptr(slots), _lib.ptr(bt), bt.stride(0),
                                bt.shape[1], num_heads, num_kv_heads, 0, _lib.ptr(q_rot), _lib.ptr(k_rot),
                                _lib.ptr(v_rot), _lib.ptr(ws), ws.numel())
        self.ref = ctypes.addressof(self.args)


_LAST_STEP: list = [None]


def mtp_step(qsl, seqs, num_tokens: int, slot_mapping, block_table, num_heads: int, num_kv_heads: int,
             head_size: int, max_q_len: int, device: torch.device, stream: int, reuse: bool = True):
    """The MtpStep of a step, or None when a request's query length is
    outside 0 .. max_q_len (the step then takes the general route).  While
    consecutive calls (the layers of one step) pass the same layout, slot
    mapping, block table, head counts and stream, the step built by the
    first is returned; ``reuse=False`` (graph capture) always builds one."""
    B = len(qsl) - 1
    if B < 1 or len(seqs) < B:
        return None
    lay = decode.request_layout(qsl, seqs[:B])
    key = (lay, num_tokens, slot_mapping.data_ptr(), block_table.data_ptr(), tuple(block_table.shape),
           num_heads, num_kv_heads, max_q_len, device, stream)
    hit = _LAST_STEP[0]
    if reuse and hit is not None and hit[0] == key:
        return hit[1]
    if lay.qsl[0] != 0 or lay.qsl[-1] != num_tokens or any(n > max_q_len for n in lay.lengths):
        st = None
    else:
        st = MtpStep(lay, num_tokens, slot_mapping, block_table, num_heads, num_kv_heads, head_size, device)
    if reuse and (st is None or st.reusable):
        _LAST_STEP[0] = (key, st)
    return st


def _row_stride(x: torch.Tensor, N: int, features: int) -> int:
    """Elements between consecutive tokens of x read as [tokens][features]
    rows with contiguous features; -1 when x is not such a view."""
    shape, st = x.shape, x.stride()
    if shape[0] < N:
        return -1
    if len(shape) == 2:
        return st[0] if shape[1] == features and st[1] == 1 else -1
    if len(shape) == 3:
        return st[0] if shape[1] * shape[2] == features and st[2] == 1 and st[1] == shape[2] else -1
    return -1


def mtp_forward(layer: MtpLayer, st: MtpStep, query, key, value, out, stream: int) -> torch.Tensor:
    """One layer's forward of a short step through oscar_mtp_forward: query
    [N, Hq*D] (or [N, Hq, D]) and key / value [N, Hk*D] bf16, out [>= N, Hq*D]
    bf16 or fp32 in the model domain (rows past N untouched)."""
    N = st.num_tokens
    hq, hk, D = layer.num_heads, layer.num_kv_heads, layer.head_size
    for x in (query, key, value):
        if x.dtype != torch.bfloat16:
            raise ValueError(f"the MTP forward takes bf16 query/key/value, got {x.dtype}")
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("the MTP forward writes a bf16 or fp32 output")
    qs = _row_stride(query, N, hq * D)
    ks = _row_stride(key, N, hk * D)
    vs = _row_stride(value, N, hk * D)
    if qs < 0:
        query, qs = _rows(query, N, hq * D)
    if ks < 0 or vs != ks:
        key = _rows(key, N, hk * D)[0].contiguous()
        value = _rows(value, N, hk * D)[0].contiguous()
        ks = key.stride(0)
    os_ = _row_stride(out, N, hq * D)
    if os_ < 0:
        raise ValueError("the output must hold Hq * D contiguous features per token")
    status = _lib.load().oscar_mtp_forward(layer.ref, st.ref, query.data_ptr(), qs, key.data_ptr(),
                                           value.data_ptr(), ks, out.data_ptr(), os_,
                                           int(out.dtype == torch.bfloat16), stream)
    if status != 0:
        raise _lib.OscarKernelError(f"oscar_mtp_forward failed: {_lib.STATUS.get(status, status)}")
    return out
