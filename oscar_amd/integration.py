"""Memory budgeting of the persistent OSCAR buffers (MI355X, 288 GB HBM3E).

Mirrors oscar_ascend/integration.py:17-44, 89-114: the KV-cache budget the
engine may allocate is what remains after the fixed per-layer buffers, in
whole cache blocks.  Per OSCAR layer the fixed buffers here are
  * R_k, R_v and their transposes, fp32       4 * D^2 * 4
  * the two MFMA rotation operands             2 * oscar_rotation_operand_bytes(D)
  * the FP32 window arena                      rows * bs * (2 * Hk * D * 4 + 8)
  * its fp16 MFMA operand images (K and V)     rows * bs * 2 * Hk * D * 2
  * the arena's seat-winner scratch            rows * bs * 4
and, once per device, the split-decode workspace of the largest batch.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

MI355X_HBM_BYTES = 288 * 10 ** 9
ROTATION_OPERAND_BYTES = 262144        # oscar_rotation_operand_bytes(256)


def memory_budget(available: int, native_per_block: int, shadow_per_block: int, fixed_bytes: int) -> int:
    """integration.py:17-23 — KV bytes = whole blocks that fit after the fixed buffers."""
    if native_per_block <= 0 or available <= fixed_bytes:
        raise ValueError("Insufficient memory for OSCAR persistent buffers")
    blocks = (available - fixed_bytes) // (native_per_block + shadow_per_block)
    if blocks < 1:
        raise ValueError("OSCAR memory budget cannot hold one cache block")
    return blocks * native_per_block


def arena_rows(block_size: int, sink: int, recent: int, staging: int) -> int:
    """integration.py:99-113 — rows reserved at the engine page size."""
    return max((staging + block_size - 1) // block_size,
               sink // block_size + (recent + block_size - 1) // block_size + 3)


def fixed_bytes_per_layer(head_dim: int, num_kv_heads: int, block_size: int, sink: int, recent: int,
                          staging: int, window: bool) -> int:
    fixed = 4 * head_dim * head_dim * 4 + 2 * ROTATION_OPERAND_BYTES
    if window:
        rows = arena_rows(block_size, sink, recent, staging)
        fixed += rows * block_size * (2 * num_kv_heads * head_dim * 4 + 2 * num_kv_heads * head_dim * 2 + 8 + 4)
    return fixed


DECODE_TILE = 32                       # history tokens per decode tile
DECODE_ROWS = 32                       # (query, head) rows per partial
DECODE_PARTIAL_FLOATS = DECODE_ROWS * 256 + 2 * DECODE_ROWS
DECODE_LAUNCH_ITEMS = 128              # (request, kv head) items carried in one launch's kernel arguments
DECODE_MAX_SPLITS = 1023               # history splits per item (the fresh-token partial makes 1024)
DECODE_MAX_TILES_PER_SPLIT = 256


def decode_tiles_per_split(max_requests: int, num_kv_heads: int, max_history: int) -> int:
    """The library's default split length (in tiles) for this batch shape."""
    tiles = -(-max_history // DECODE_TILE) if max_history > 0 else 0
    work = tiles * max_requests * num_kv_heads
    tps = 4
    while tps < 64 and work // tps > 512:
        tps *= 2
    while tps < DECODE_MAX_TILES_PER_SPLIT and -(-tiles // tps) > DECODE_MAX_SPLITS:
        tps *= 2
    return tps


def decode_workspace_bytes(max_requests: int, num_kv_heads: int, num_heads: int, max_query_len: int,
                           max_history: int, tiles_per_split: int = 0) -> int:
    """Same value as oscar_paged_decode_workspace_bytes (no library needed):
    one fp32 partial (32 rows x 256 + max + sum) per (request, kv head,
    history split or the fresh-token split, row tile)."""
    tps = tiles_per_split or decode_tiles_per_split(max_requests, num_kv_heads, max_history)
    tiles = -(-max_history // DECODE_TILE) if max_history > 0 else 0
    splits = -(-tiles // tps)
    row_tiles = -(-(max_query_len * (num_heads // num_kv_heads)) // DECODE_ROWS)
    per_launch = DECODE_LAUNCH_ITEMS // num_kv_heads         # requests per launch share one workspace
    chunk = min(max_requests, per_launch)
    return chunk * num_kv_heads * (splits + 1) * row_tiles * DECODE_PARTIAL_FLOATS * 4


def kv_block_bytes(block_size: int, num_kv_heads: int, slot_width: int, layers: int) -> int:
    """Native bytes of one cache block across the OSCAR layers (K and V caches)."""
    return 2 * block_size * num_kv_heads * slot_width * layers


def plan_capacity(available: int, layers: int, head_dim: int = 256, num_kv_heads: int = 1,
                  num_heads: int = 6, block_size: int = 128, slot_width: int = 256, sink: int = 128,
                  recent: int = 256, staging: int = 8192, window: bool = True, max_requests: int = 256,
                  max_query_len: int = 4, max_history: int = 262144) -> dict:
    """Budget one GPU: how many cache blocks (and INT2 tokens) fit."""
    fixed = layers * fixed_bytes_per_layer(head_dim, num_kv_heads, block_size, sink, recent, staging, window)
    fixed += decode_workspace_bytes(max_requests, num_kv_heads, num_heads, max_query_len, max_history)
    native = kv_block_bytes(block_size, num_kv_heads, slot_width, layers)
    budget = memory_budget(available, native, 0, fixed)
    blocks = budget // native
    return {"available": available, "fixed": fixed, "native_per_block": native, "budget": budget,
            "blocks": blocks, "tokens": blocks * block_size}


def source_fingerprint() -> str:
    """integration.py:26-32 — sha256 over the package's Python and HIP sources."""
    root = Path(__file__).parent
    digest = hashlib.sha256()
    for path in sorted(list(root.rglob("*.py")) + list(root.rglob("*.hip")) + list(root.rglob("*.h"))):
        digest.update(str(path.relative_to(root)).encode())
        digest.update(path.read_bytes())
    return digest.hexdigest()


def verify_layers(layer_types, actual_ids) -> None:
    """integration.py:35-44 — every full-attention layer must run OSCAR."""
    expected = {i for i, kind in enumerate(layer_types) if kind in ("full_attention", "attention")}
    if not expected or set(actual_ids) != expected or len(actual_ids) != len(expected):
        raise RuntimeError(f"Incomplete OSCAR layers: expected={sorted(expected)}, actual={sorted(actual_ids)}")


def install_runner_hooks() -> None:
    """Engine worker seams (reference integration.py:47-195) are engine-build
    specific; the vLLM-ROCm worker hooks are not wired in this build."""
    return None
