"""Host wrapper of the paged MTP decode kernel (kernel 2).

Mirrors the reference seam ``oscar_paged_attention_triton(q, k, v, kc, vc, bt,
qsl, seqs, scale, stage=None)`` (oscar_ascend/kernels/paged_attention.py:272-360):
same arguments and meaning, rotated-domain fp32 inputs, rotated-V-domain fp32
output [n, Hq, D].  ``stage`` is the arena (stage_k, stage_v, owner[, k_image,
v_image]); the kernel reads the window through the owner tags and the fp16
operand images, which are built from the fp32 arena when not given.  ``qsl``/``seqs`` are host lists (the reference's
metadata_batch_lists); they are validated exactly like the reference's
query_layout (paged_attention.py:20-38) and handed to the library as host
arrays, which it places in the kernel arguments.
"""
from __future__ import annotations

import ctypes
import itertools

import torch

from ..format import check_d
from . import _lib, staging
from .quant import cache_geometry

MAX_QUERY_LEN = 16          # rows per request <= 16 tokens x group (backend.py:277)

def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch for one launch's split partials, from torch's caching allocator:
    a block freed after a launch is reused by later launches on the same
    stream only, so launches on different streams never share partials."""
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def validate_layout(qsl, seqs):
    """paged_attention.py:20-38 — lengths must be >= 0 and <= their sequence."""
    lengths = [b - a for a, b in itertools.pairwise(qsl)]
    if len(seqs) != len(lengths) or any(n < 0 or s < n for n, s in zip(lengths, seqs)):
        raise ValueError("Invalid OSCAR query/sequence lengths")
    return lengths


class RequestLayout:
    """A step's request layout, validated once and shared by the launches of
    every layer in the step: query lengths, the longest query and history,
    and the host int32 arrays (query starts, sequence lengths) the library
    copies into its kernel arguments."""

    __slots__ = ("qsl", "seqs", "lengths", "max_q", "max_hist", "qstart", "seq_t")

    def __init__(self, qsl, seqs):
        self.qsl = tuple(int(x) for x in qsl)
        self.seqs = tuple(int(x) for x in seqs)
        self.lengths = validate_layout(self.qsl, self.seqs)
        self.max_q = max(self.lengths, default=0)
        self.max_hist = max((s - m for s, m in zip(self.seqs, self.lengths)), default=0)
        self.qstart = (ctypes.c_int32 * max(len(self.qsl), 1))(*self.qsl)
        self.seq_t = (ctypes.c_int32 * max(len(self.seqs), 1))(*self.seqs)


_LAST_LAYOUT: list = [None]


def request_layout(qsl, seqs) -> RequestLayout:
    """The RequestLayout of (qsl, seqs), reused while consecutive calls (the
    layers of one step) pass the same lengths."""
    key = (tuple(qsl), tuple(seqs))
    hit = _LAST_LAYOUT[0]
    if hit is None or hit[0] != key:
        hit = (key, RequestLayout(*key))
        _LAST_LAYOUT[0] = hit
    return hit[1]


class DecodePlan:
    """Device-resident arguments of one decode launch; ``launch`` only enqueues.

    Keeps every tensor it points at alive.  Launching a plan repeatedly (or
    capturing it in a HIP graph) re-runs the same decode on the current stream.
    """

    def __init__(self, args: tuple, out: torch.Tensor, keep: list, entry: str = "oscar_paged_decode"):
        self.args = args
        self.out = out
        self.keep = keep
        self.entry = entry

    def launch(self) -> torch.Tensor:
        _lib.call(self.entry, *self.args, _lib.stream_handle(self.out.device))
        return self.out


def _stage_operands(stage, bs: int, hk: int):
    """(owner int64, k image, v image, rows) of an arena (stage_k, stage_v,
    owner[, k_image, v_image]); the fp16 images are built when not given."""
    owner = stage[2]
    if owner.shape[1] != bs:
        raise ValueError("staging arena block size must equal the cache block size")
    owner = owner.to(torch.int64).contiguous()
    rows = owner.shape[0]
    if len(stage) >= 5 and stage[3] is not None:
        kimg, vimg = stage[3], stage[4]
    else:
        kimg, vimg = staging.stage_images(stage[0], stage[1])
    staging.check_images(kimg, vimg, rows, bs, hk)
    return owner, kimg, vimg, rows


def plan(q, k, v, kc, vc, bt, qsl, seqs, scale: float, stage=None, out=None,
         tiles_per_split: int = 0, out_rotation=None) -> DecodePlan:
    """One decode launch pair.  Without ``out_rotation`` the output is fp32
    [n, Hq, D] in the rotated-V domain.  With ``out_rotation`` = R_v^T (fp32
    [D, D]) the merge applies it and writes ``out`` (required: [n, Hq * D] or
    [n, Hq, D], fp32 or bf16, unit feature stride) in the model domain."""
    n, hq, d = q.shape
    check_d(d)
    hk = k.shape[1]
    lay = request_layout(qsl, seqs)
    if sum(lay.lengths) != n:
        raise ValueError("Query layout does not match actual query tokens")
    max_q, max_hist = lay.max_q, lay.max_hist
    if max_q > MAX_QUERY_LEN:
        raise ValueError(f"paged decode supports at most {MAX_QUERY_LEN} query tokens per request")
    dev = q.device
    q = q.float().contiguous()
    k = k.float().contiguous()
    v = v.float().contiguous()
    if bt.ndim != 2:
        raise ValueError("block table must be [requests, pages]")
    bt = bt.to(device=dev, dtype=torch.int32).contiguous()
    # Request layout as host int32 arrays: the library copies it into the
    # kernel arguments (no device metadata round trip).
    qstart, seq_t = lay.qstart, lay.seq_t
    bs, pages, kst, vst = cache_geometry(kc, vc)
    if stage is not None:
        owner, kimg, vimg, rows = _stage_operands(stage, bs, hk)
    else:
        owner = kimg = vimg = None
        rows = 0
    B = len(lay.lengths)
    if bs % 32:
        raise ValueError("paged decode needs a cache block size that is a multiple of 32")
    need = _lib.load().oscar_paged_decode_workspace_bytes(B, hk, hq, max(max_q, 1), max_hist, tiles_per_split)
    ws = workspace(dev, need)
    common = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), n, hq, hk, d, _lib.ptr(kc), _lib.ptr(vc), bs,
              pages, *kst, *vst, _lib.ptr(bt), bt.stride(0), bt.shape[1], ctypes.addressof(qstart),
              ctypes.addressof(seq_t), B, max_q, max_hist, _lib.ptr(owner), _lib.ptr(kimg), _lib.ptr(vimg), rows,
              float(scale), int(tiles_per_split))
    keep = [q, k, v, kc, vc, bt, qstart, seq_t, owner, kimg, vimg, ws]
    if out_rotation is None:
        if out is None:
            out = torch.empty(n, hq, d, dtype=torch.float32, device=dev)
        return DecodePlan(common + (_lib.ptr(out), _lib.ptr(ws), ws.numel()), out, keep)
    rot = out_rotation
    if rot.shape != (d, d) or rot.dtype != torch.float32 or not rot.is_contiguous() or rot.device != dev:
        raise ValueError("out_rotation must be a contiguous fp32 [D, D] tensor on the query's device")
    if out is None or out.shape[0] < n or out.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out_rotation needs an fp32 or bf16 output with a row per query token")
    rows_out = out.reshape(out.shape[0], -1)
    if rows_out.shape[1] != hq * d or rows_out.stride(1) != 1 or rows_out.data_ptr() != out.data_ptr():
        raise ValueError("output rows must hold Hq * D contiguous features")
    args = common + (_lib.ptr(rot), _lib.ptr(out), rows_out.stride(0), int(out.dtype == torch.bfloat16),
                     _lib.ptr(ws), ws.numel())
    return DecodePlan(args, out, keep + [rot], entry="oscar_paged_decode_rotated")


def paged_attention(q, k, v, kc, vc, bt, qsl, seqs, scale: float, stage=None, out_rotation=None,
                    out=None) -> torch.Tensor:
    """Rotated-domain paged MTP attention; returns fp32 [n, Hq, D], or with
    ``out_rotation`` (R_v^T) writes ``out`` in the model domain and returns it."""
    if q.shape[0] == 0:
        return out if out is not None else torch.empty(q.shape, dtype=torch.float32, device=q.device)
    return plan(q, k, v, kc, vc, bt, qsl, seqs, scale, stage, out=out, out_rotation=out_rotation).launch()


def decode_only_plan(q, kc, vc, bt, seqs, scale: float, stage=None, sink_tokens: int = 0,
                     recent_tokens: int = 0, out=None, tiles_per_split: int = 0) -> DecodePlan:
    """The DecodeOnly read (backend.py:321-358, 500-611): one rotated query
    per request [B, Hq, D] over its whole history [0, seqs[i]); with a window
    arena, staged values only in the reference's windowed segments (the sink
    when fully staged, the staged run ending at seq - 1 inside the recent
    window).  ``seqs`` is a host list; returns fp32 [B, Hq, D] rotated-V."""
    B, hq, d = q.shape
    check_d(d)
    if len(seqs) != B or any(s < 0 for s in seqs):
        raise ValueError("DecodeOnly needs one query token and a non-negative length per request")
    if bt.ndim != 2 or bt.shape[0] < B:
        raise ValueError("block table must be [requests, pages]")
    dev = q.device
    q = q.float().contiguous()
    bt = bt.to(device=dev, dtype=torch.int32).contiguous()
    seq_t = (ctypes.c_int32 * max(B, 1))(*[int(x) for x in seqs])
    max_hist = max(seqs, default=0)
    bs, pages, kst, vst = cache_geometry(kc, vc)
    hk = kc.shape[2]
    if bs % 32:
        raise ValueError("paged decode needs a cache block size that is a multiple of 32")
    owner = kimg = vimg = None
    rows = 0
    if stage is not None:
        owner, kimg, vimg, rows = _stage_operands(stage, bs, hk)
    need = _lib.load().oscar_decode_only_workspace_bytes(B, hk, hq, max_hist, tiles_per_split)
    ws = workspace(dev, need)
    if out is None:
        out = torch.empty(B, hq, d, dtype=torch.float32, device=dev)
    args = (_lib.ptr(q), hq, hk, d, _lib.ptr(kc), _lib.ptr(vc), bs, pages, *kst, *vst, _lib.ptr(bt),
            bt.stride(0), bt.shape[1], ctypes.addressof(seq_t), B, max_hist, _lib.ptr(owner), _lib.ptr(kimg),
            _lib.ptr(vimg), rows, int(sink_tokens), int(recent_tokens), float(scale), int(tiles_per_split),
            _lib.ptr(out), _lib.ptr(ws), ws.numel())
    return DecodePlan(args, out, [q, kc, vc, bt, seq_t, owner, kimg, vimg, ws], entry="oscar_decode_only")


def decode_only(q, kc, vc, bt, seqs, scale: float, stage=None, sink_tokens: int = 0,
                recent_tokens: int = 0) -> torch.Tensor:
    """Rotated-domain DecodeOnly attention; returns fp32 [B, Hq, D]."""
    if q.shape[0] == 0:
        return torch.empty(q.shape, dtype=torch.float32, device=q.device)
    return decode_only_plan(q, kc, vc, bt, seqs, scale, stage, sink_tokens, recent_tokens).launch()
