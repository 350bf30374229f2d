"""Oracle: OSCAR INT2 numeric contract (slot layout, quantize, pack, dequant).

Restates oscar_ascend/format.py.  Test infrastructure only (see oracle/__init__).

Logical 160-byte slot per (token, kv-head), split across the two caches:

    K slot  [0:2] K scale   [2:4] K zero   [4:6] V scale   [6:8] V zero
            [8:32] pad (never written)     [32:32+D/4] K codes
    V slot  [0:D/4] V codes

fp16 meta is little-endian; code k of byte b is bits [2k, 2k+2) of that byte
(value index 4b+k).
"""
from __future__ import annotations

import torch

BITS = 2                      # format.py:19
LEVELS = 4                    # format.py:20
VALUES_PER_BYTE = 4           # format.py:21
D_DEFAULT = 256               # format.py:22
SLOT_SIZE = 160               # format.py:26
META_BYTES = 8                # format.py:28
PAD_BYTES = 24                # format.py:29
K_IDX_OFF = 32                # format.py:30
V_IDX_OFF = 96                # format.py:31
K_SLOT_BYTES = V_IDX_OFF      # format.py:32
V_SLOT_BYTES = SLOT_SIZE - V_IDX_OFF   # format.py:33
DEQUANT_TOL = 1e-5            # format.py:36
DECODE_TOL = 1e-4             # format.py:37
SCALE_FLOOR = 2.0 ** -14      # format.py:38


def check_d(D: int) -> None:
    """format.py:41-45 — D must pack 4 codes/byte and fit the 64 code bytes."""
    if D % VALUES_PER_BYTE:
        raise ValueError(f"D={D} is not a multiple of {VALUES_PER_BYTE}")
    if D // VALUES_PER_BYTE > K_SLOT_BYTES - META_BYTES - PAD_BYTES:
        raise ValueError(f"D={D} does not fit one slot")


def vector_scales(x: torch.Tensor):
    """format.py:51-64 — per-vector (scale, zero), both already rounded to fp16.

    scale = (max - min) / 3 in fp32, replaced by 2^-14 unless strictly greater;
    zero = min.  Both go through an fp32 -> fp16 (round-to-nearest-even) cast
    and back, so the returned fp32 values are exactly representable in fp16.
    """
    x = x.float()
    lo = x.amin(dim=-1, keepdim=True)
    hi = x.amax(dim=-1, keepdim=True)
    scale = (hi - lo) / (LEVELS - 1)
    scale = torch.where(scale > SCALE_FLOOR, scale, torch.full_like(scale, SCALE_FLOOR))
    return scale.to(torch.float16).float(), lo.to(torch.float16).float()


def codes(x: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """format.py:82 — q = clamp(floor((x - zero) / scale + 0.5), 0, 3), int32.

    Every step is a separate fp32 op (subtract, IEEE divide, add 0.5, floor).
    """
    x = x.float()
    q = torch.floor((x - zero) / scale + 0.5)
    return torch.clamp(q, 0, LEVELS - 1).to(torch.int32)


def pack(q: torch.Tensor) -> torch.Tensor:
    """format.py:83-87 — byte b = sum_k q[4b+k] << 2k, as uint8 [.., D/4]."""
    q = q.to(torch.int32) & (LEVELS - 1)
    grouped = q.reshape(*q.shape[:-1], q.shape[-1] // VALUES_PER_BYTE, VALUES_PER_BYTE)
    weights = torch.tensor([1, 4, 16, 64], dtype=torch.int32, device=q.device)
    return (grouped * weights).sum(dim=-1).to(torch.uint8)


def quantize(x: torch.Tensor):
    """format.py:67-88 — fp32 [.., D] -> (packed uint8 [.., D/4], scale, zero)."""
    scale, zero = vector_scales(x)
    return pack(codes(x, scale, zero)), scale, zero


def unpack(packed: torch.Tensor, D: int) -> torch.Tensor:
    """format.py:99-110 — uint8 [.., D/4] -> int32 codes [.., D]."""
    p = packed.to(torch.int32)
    parts = [(p >> (2 * k)) & (LEVELS - 1) for k in range(VALUES_PER_BYTE)]
    return torch.stack(parts, dim=-1).reshape(*p.shape[:-1], D)


def dequant(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, D: int) -> torch.Tensor:
    """format.py:91-96 — code * scale + zero in fp32 (separate multiply and add)."""
    return unpack(packed, D).float() * scale + zero


def f16_le(x: torch.Tensor):
    """format.py:113-119 — fp16 value -> (low byte, high byte) uint8."""
    bits = x.contiguous().to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    return (bits & 0xFF).to(torch.uint8), (bits >> 8).to(torch.uint8)


def f16_from_le(lo: torch.Tensor, hi: torch.Tensor) -> torch.Tensor:
    """format.py:122-125 — (low, high) uint8 -> fp16 value as fp32."""
    bits = lo.to(torch.int32) | (hi.to(torch.int32) << 8)
    bits = torch.where(bits >= 0x8000, bits - 0x10000, bits)
    return bits.to(torch.int16).view(torch.float16).float()


def make_slot_bytes(k_rot: torch.Tensor, v_rot: torch.Tensor) -> torch.Tensor:
    """format.py:131-154 — rotated K/V [N, H, D] -> logical slots [N, H, 160] uint8.

    Pad bytes [8:32) are zero in the logical slot.
    """
    N, H, D = k_rot.shape
    check_d(D)
    nb = D // VALUES_PER_BYTE
    kp, ks, kz = quantize(k_rot)
    vp, vs, vz = quantize(v_rot)
    slot = torch.zeros(N, H, SLOT_SIZE, dtype=torch.uint8)
    for j, value in enumerate((ks, kz, vs, vz)):
        lo, hi = f16_le(value)
        slot[..., 2 * j] = lo[..., 0]
        slot[..., 2 * j + 1] = hi[..., 0]
    slot[..., K_IDX_OFF:K_IDX_OFF + nb] = kp
    slot[..., V_IDX_OFF:V_IDX_OFF + nb] = vp
    return slot


def parse_slot_bytes(slot: torch.Tensor, D: int):
    """format.py:157-167 — logical slots [.., 160] -> (k, v) fp32 [.., D]."""
    check_d(D)
    nb = D // VALUES_PER_BYTE
    meta = [f16_from_le(slot[..., 2 * j:2 * j + 1], slot[..., 2 * j + 1:2 * j + 2]) for j in range(4)]
    k = dequant(slot[..., K_IDX_OFF:K_IDX_OFF + nb], meta[0], meta[1], D)
    v = dequant(slot[..., V_IDX_OFF:V_IDX_OFF + nb], meta[2], meta[3], D)
    return k, v
