"""Per-layer orthogonal K/V rotations.

Same checkpoint formats and lookup rules as the reference loader
(oscar_ascend/rotation.py:18-129):
  * ``{"layers": {id: {"rotation": R_k, "rotation_v": R_v, ...}}}``
    (ids may be ints, numeric strings or module names),
  * ``{id: R}`` or ``{id: {"rotation": ...}}``,
  * a stacked ``[num_layers, D, D]`` tensor.
An empty path gives the identity; a missing layer gives the identity unless
``strict`` (then ValueError); strict mode also rejects non-finite or
non-orthogonal matrices.  Files are read with ``weights_only=True``.
"""
from __future__ import annotations

import re
from functools import lru_cache

import torch

_LAYER_RE = re.compile(r"\.layers\.(\d+)\.")


def layer_index_from_name(layer_name: str) -> int | None:
    """rotation.py:18-24 — '.layers.<i>.' first, else the last integer in the name."""
    m = _LAYER_RE.search(layer_name)
    if m is not None:
        return int(m.group(1))
    ints = re.findall(r"\d+", layer_name)
    return int(ints[-1]) if ints else None


def _resolve_key(key) -> int | None:
    """rotation.py:28-41 — int, numeric string or module-name keys."""
    if isinstance(key, int):
        return key
    if isinstance(key, str):
        try:
            return int(key)
        except ValueError:
            return layer_index_from_name(key)
    return None


def _tensors(entry: dict) -> dict:
    return {k: v.float().contiguous() for k, v in entry.items() if isinstance(v, torch.Tensor)}


@lru_cache(maxsize=8)
def load_checkpoint(path: str) -> dict:
    """rotation.py:44-90 — {layer id: {"rotation": R_k, ["rotation_v": R_v]}}."""
    obj = torch.load(path, map_location="cpu", weights_only=True)
    if not (isinstance(obj, dict) and obj.get("format_version", 0) >= 2
            and "r_h_pbr" in str(obj.get("objective", ""))):
        print(f"[oscar-amd] rotation checkpoint {path!r} is not a v2 (U@H@P_br) recipe; "
              "per-vector INT2 accuracy will suffer")
    table: dict[int, dict] = {}
    if isinstance(obj, dict) and "layers" in obj:
        for key, entry in obj["layers"].items():
            lid = _resolve_key(key)
            if lid is None:
                continue
            if isinstance(entry, dict) and "rotation" in entry:
                table[lid] = _tensors(entry)
            else:
                table[lid] = {"rotation": entry.float().contiguous()}
    elif isinstance(obj, dict):
        for key, entry in obj.items():
            lid = _resolve_key(key)
            if lid is None:
                continue
            if isinstance(entry, dict) and "rotation" in entry:
                table[lid] = _tensors(entry)
            elif isinstance(entry, torch.Tensor):
                table[lid] = {"rotation": entry.float().contiguous()}
    elif torch.is_tensor(obj) and obj.dim() == 3:
        for lid in range(obj.shape[0]):
            table[lid] = {"rotation": obj[lid].float().contiguous()}
    else:
        raise ValueError(f"Unrecognized OSCAR rotation checkpoint structure at {path!r}: {type(obj)}")
    return table


def get_layer_rotation(path: str, layer_name: str, head_dim: int, device, dtype=torch.float32,
                       mode: str = "k", strict: bool = False) -> torch.Tensor:
    """rotation.py:93-129 — this layer's [D, D] rotation (mode 'v' prefers rotation_v)."""
    if not path:
        return torch.eye(head_dim, device=device, dtype=dtype)
    table = load_checkpoint(path)
    lid = layer_index_from_name(layer_name)
    entry = table.get(lid) if lid is not None else None
    if entry is None:
        if strict:
            raise ValueError(f"Rotation checkpoint {path!r} is missing layer {layer_name}")
        return torch.eye(head_dim, device=device, dtype=dtype)
    rot = entry.get("rotation_v") if mode == "v" else entry.get("rotation")
    if rot is None:
        rot = entry.get("rotation")
    if rot is None:
        return torch.eye(head_dim, device=device, dtype=dtype)
    if rot.shape != (head_dim, head_dim):
        raise ValueError(f"OSCAR rotation for layer {lid} has shape {tuple(rot.shape)}, "
                         f"expected ({head_dim}, {head_dim}).")
    if strict:
        eye = torch.eye(head_dim)
        if not torch.isfinite(rot).all() or not torch.allclose(rot @ rot.t(), eye, atol=1e-3, rtol=1e-3):
            raise ValueError(f"Rotation checkpoint {path!r} layer {lid} is not finite/orthogonal")
    return rot.to(device=device, dtype=dtype).contiguous()
