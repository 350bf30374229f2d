"""Oracle: paged-slot scatter write and gather/dequant.

Restates oscar_ascend/kernels/store_kernel.py (torch paths only).  Test
infrastructure only.

Caches are engine-owned ``(pages, bs, Hk, W)`` tensors of any element type;
they are addressed through their uint8 view, with byte strides.  A slot id
``s >= 0`` means page ``s // bs``, row ``s % bs``; ``s < 0`` is skipped.
"""
from __future__ import annotations

import torch

from . import format as fmt


def slot_bases(slots: torch.Tensor, bs: int, hk: int, k8: torch.Tensor, v8: torch.Tensor):
    """store_kernel.py:35-48 — byte offsets [N, H] of each (token, head) slot."""
    page = slots // bs
    row = slots % bs
    h = torch.arange(hk)
    k_off = (page * k8.stride(0) + row * k8.stride(1)).unsqueeze(-1) + h * k8.stride(2)
    v_off = (page * v8.stride(0) + row * v8.stride(1)).unsqueeze(-1) + h * v8.stride(2)
    return k_off, v_off


def store_ref(k_rot: torch.Tensor, v_rot: torch.Tensor, k_cache: torch.Tensor,
              v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """store_kernel.py:54-102 — quantize rotated K/V [N, H, D] and scatter.

    Writes the 8 meta bytes and the K codes into the K slot, the V codes into
    the V slot; pad bytes and bytes past the code width are left untouched.
    Negative slots are dropped before anything is computed.
    """
    k8, v8 = k_cache.view(torch.uint8), v_cache.view(torch.uint8)
    if not (k8.is_contiguous() and v8.is_contiguous()):
        raise ValueError("caches must be contiguous")
    N, H, D = k_rot.shape
    fmt.check_d(D)
    nb = D // fmt.VALUES_PER_BYTE
    bs = k8.shape[1]
    slots = slot_mapping.to(torch.int64)
    keep = slots >= 0
    slots, k_rot, v_rot = slots[keep], k_rot[keep], v_rot[keep]
    if slots.numel() == 0:
        return
    n = slots.numel()
    k_off, v_off = slot_bases(slots, bs, H, k8, v8)
    kp, ks, kz = fmt.quantize(k_rot.float().reshape(n, H, D))
    vp, vs, vz = fmt.quantize(v_rot.float().reshape(n, H, D))
    flat_k, flat_v = k8.view(-1), v8.view(-1)
    for j, value in enumerate((ks, kz, vs, vz)):
        lo, hi = fmt.f16_le(value)
        flat_k[k_off + 2 * j] = lo[..., 0]
        flat_k[k_off + 2 * j + 1] = hi[..., 0]
    cols = torch.arange(nb)
    flat_k[(k_off.unsqueeze(-1) + fmt.K_IDX_OFF) + cols] = kp
    flat_v[v_off.unsqueeze(-1) + cols] = vp


def dequant_split_ref(k8: torch.Tensor, v8: torch.Tensor, pages: torch.Tensor,
                      rows: torch.Tensor, hk: int, D: int):
    """store_kernel.py:105-133 — (k, v) fp32 [T, H, D] for slots (pages, rows)."""
    fmt.check_d(D)
    nb = D // fmt.VALUES_PER_BYTE
    pages, rows = pages.to(torch.int64), rows.to(torch.int64)
    h = torch.arange(hk)
    k_off = ((pages * k8.stride(0) + rows * k8.stride(1)).unsqueeze(-1) + h * k8.stride(2)).unsqueeze(-1)
    v_off = ((pages * v8.stride(0) + rows * v8.stride(1)).unsqueeze(-1) + h * v8.stride(2)).unsqueeze(-1)
    flat_k, flat_v = k8.reshape(-1), v8.reshape(-1)
    meta = flat_k[k_off + torch.arange(fmt.META_BYTES)]
    scales = [fmt.f16_from_le(meta[..., 2 * j:2 * j + 1], meta[..., 2 * j + 1:2 * j + 2]) for j in range(4)]
    cols = torch.arange(nb)
    k = fmt.dequant(flat_k[k_off + fmt.K_IDX_OFF + cols], scales[0], scales[1], D)
    v = fmt.dequant(flat_v[v_off + cols], scales[2], scales[3], D)
    return k, v


def gather_kv_ref(k_cache, v_cache, block_table, seq_lens, hk: int, D: int):
    """store_kernel.py:136-154 — per-sequence dequantized history lists."""
    k8, v8 = k_cache.view(torch.uint8), v_cache.view(torch.uint8)
    bs = k8.shape[1]
    ks, vs = [], []
    for b in range(block_table.shape[0]):
        pos = torch.arange(int(seq_lens[b]))
        k, v = dequant_split_ref(k8, v8, block_table[b][pos // bs], pos % bs, hk, D)
        ks.append(k)
        vs.append(v)
    return ks, vs


def full_dequant_ref(k_cache, v_cache, bt_row, cached_len: int, hk: int, D: int):
    """decode_kernel.py:120-134 — dequantized history [C, Hk, D] of one request."""
    k8, v8 = k_cache.view(torch.uint8), v_cache.view(torch.uint8)
    bs = k8.shape[1]
    pos = torch.arange(cached_len)
    return dequant_split_ref(k8, v8, bt_row[pos // bs], pos % bs, hk, D)


def logical_slots(k_cache, v_cache, slots: torch.Tensor, hk: int, D: int) -> torch.Tensor:
    """Read back logical 160-byte slots [N, H, 160] from the split physical slots.

    Mirrors the byte reassembly of the reference test
    tests/test_numeric.py:82-103 (pad bytes reported as zero).
    """
    k8, v8 = k_cache.view(torch.uint8), v_cache.view(torch.uint8)
    bs = k8.shape[1]
    nb = D // fmt.VALUES_PER_BYTE
    k_off, v_off = slot_bases(slots.to(torch.int64), bs, hk, k8, v8)
    flat_k, flat_v = k8.reshape(-1), v8.reshape(-1)
    out = torch.zeros(slots.numel(), hk, fmt.SLOT_SIZE, dtype=torch.uint8)
    out[..., :fmt.META_BYTES] = flat_k[k_off.unsqueeze(-1) + torch.arange(fmt.META_BYTES)]
    out[..., fmt.K_IDX_OFF:fmt.K_IDX_OFF + nb] = flat_k[k_off.unsqueeze(-1) + fmt.K_IDX_OFF + torch.arange(nb)]
    out[..., fmt.V_IDX_OFF:fmt.V_IDX_OFF + nb] = flat_v[v_off.unsqueeze(-1) + torch.arange(nb)]
    return out
