"""OSCAR INT2 slot layout constants (product side).

Same numeric contract as the reference's oscar_ascend/format.py:19-45 (the
layout is a format both sides must agree on byte for byte, so the constants
are identical by necessity).  The quantizer itself lives in the HIP kernels.
"""
from __future__ import annotations

BITS = 2
LEVELS = 4
VALUES_PER_BYTE = 4
HEAD_DIM = 256              # the HIP kernels are written for D = 256
SLOT_SIZE = 160             # logical slot: K slot bytes [0, 96) + V slot bytes [0, 64)
META_BYTES = 8              # K scale, K zero, V scale, V zero (fp16 little-endian)
PAD_BYTES = 24              # K slot [8, 32), never written
K_IDX_OFF = 32              # K codes at K slot + 32
V_IDX_OFF = 96              # V codes at logical offset 96 = V slot + 0
K_SLOT_BYTES = 96
V_SLOT_BYTES = 64
SCALE_FLOOR = 2.0 ** -14


def check_d(D: int) -> None:
    """format.py:41-45 — D packs 4 codes per byte and fits the 64 code bytes."""
    if D % VALUES_PER_BYTE:
        raise ValueError(f"D={D} must be a multiple of {VALUES_PER_BYTE} (INT2 packing)")
    if D // VALUES_PER_BYTE > K_SLOT_BYTES - META_BYTES - PAD_BYTES:
        raise ValueError(f"D={D} exceeds the slot capacity")
