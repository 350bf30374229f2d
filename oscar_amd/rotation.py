"""Per-layer orthogonal K/V rotations read from a checkpoint file.

Checkpoint layouts accepted (the on-disk formats of the reference's loader,
oscar_ascend/rotation.py:44-90, and of the calibration tool's output):

  1. {"layers": {layer_id: entry}, ...}      calibration output (format v2
     adds "format_version": 2 and an "objective" naming "r_h_pbr");
  2. {layer_id: entry}                       a bare mapping;
  3. a tensor [num_layers, D, D]             layer i is slice i.

An entry is a [D, D] tensor (the K rotation) or a dict holding "rotation"
(and optionally "rotation_v" and other tensors).  A layer_id is an int, a
numeric string or a module name; module names and vLLM layer names map to an
index by their ".layers.<i>." component, else by their last integer.

Lookup: an empty path or an absent layer gives the identity (strict mode:
ValueError for an absent layer, and for a matrix that is not finite or not
orthogonal within 1e-3).  The V rotation is "rotation_v" when the entry has
one, else "rotation".  Files are read with ``weights_only=True``: a
checkpoint that needs unpickling of arbitrary objects is refused.
"""
from __future__ import annotations

import re
import warnings
from functools import lru_cache

import torch

_DECODER_INDEX = re.compile(r"\.layers\.(\d+)\.")
_DIGITS = re.compile(r"\d+")


def layer_index_from_name(name: str) -> int | None:
    """Decoder-layer index of a module or layer name (None if it has no digits)."""
    found = _DECODER_INDEX.search(name)
    if found:
        return int(found.group(1))
    runs = _DIGITS.findall(name)
    return int(runs[-1]) if runs else None


def _layer_id(key) -> int | None:
    if isinstance(key, int):
        return key
    if isinstance(key, str):
        return int(key) if key.strip().lstrip("+-").isdigit() else layer_index_from_name(key)
    return None


def _as_entry(value, where: str) -> dict[str, torch.Tensor]:
    if isinstance(value, torch.Tensor):
        return {"rotation": value.float().contiguous()}
    if isinstance(value, dict) and isinstance(value.get("rotation"), torch.Tensor):
        return {k: t.float().contiguous() for k, t in value.items() if isinstance(t, torch.Tensor)}
    raise ValueError(f"{where}: a layer entry must be a matrix or hold a 'rotation' matrix")


def _is_v2_recipe(obj) -> bool:
    return isinstance(obj, dict) and obj.get("format_version", 0) >= 2 and "r_h_pbr" in str(obj.get("objective", ""))


@lru_cache(maxsize=8)
def load_checkpoint(path: str) -> dict[int, dict[str, torch.Tensor]]:
    """{layer index: {"rotation": R_k[, "rotation_v": R_v, ...]}} of one file (cached)."""
    obj = torch.load(path, map_location="cpu", weights_only=True)
    if not _is_v2_recipe(obj):
        warnings.warn(f"OSCAR rotations in {path} are not a format-v2 U@H@P_br calibration; "
                      "per-vector INT2 error will be higher than calibrated", stacklevel=2)
    if torch.is_tensor(obj):
        if obj.dim() != 3:
            raise ValueError(f"{path}: a stacked rotation tensor must be [layers, D, D], got {tuple(obj.shape)}")
        return {i: {"rotation": obj[i].float().contiguous()} for i in range(obj.shape[0])}
    if not isinstance(obj, dict):
        raise ValueError(f"{path}: expected a mapping or a stacked tensor of rotations, found {type(obj).__name__}")
    layers = obj["layers"] if "layers" in obj else obj
    table = {}
    for key, value in layers.items():
        lid = _layer_id(key)
        if lid is None:
            continue                 # metadata keys such as "format_version"
        if "layers" not in obj and not isinstance(value, (torch.Tensor, dict)):
            continue
        table[lid] = _as_entry(value, f"{path} [{key!r}]")
    return table


def _check_orthogonal(R: torch.Tensor, where: str) -> None:
    if not torch.isfinite(R).all():
        raise ValueError(f"{where}: rotation holds non-finite values")
    gram = R @ R.t()
    if not torch.allclose(gram, torch.eye(R.shape[0]), atol=1e-3, rtol=1e-3):
        dev = (gram - torch.eye(R.shape[0])).abs().max().item()
        raise ValueError(f"{where}: rotation is not orthogonal (max |R R^T - I| = {dev:.2e})")


def get_layer_rotation(path: str, layer_name: str, head_dim: int, device, dtype=torch.float32,
                       mode: str = "k", strict: bool = False) -> torch.Tensor:
    """The [D, D] rotation of one layer (x_rot = x @ R); mode "v" prefers rotation_v."""
    eye = lambda: torch.eye(head_dim, device=device, dtype=dtype)  # noqa: E731
    if not path:
        return eye()
    lid = layer_index_from_name(layer_name)
    entry = load_checkpoint(path).get(lid) if lid is not None else None
    if entry is None:
        if strict:
            raise ValueError(f"{path} has no rotation for layer {layer_name!r} (index {lid})")
        return eye()
    R = entry.get("rotation_v") if mode == "v" else None
    R = entry["rotation"] if R is None else R
    where = f"{path} layer {lid} ({mode})"
    if tuple(R.shape) != (head_dim, head_dim):
        raise ValueError(f"{where}: rotation shape {tuple(R.shape)} does not match head_dim {head_dim}")
    if strict:
        _check_orthogonal(R, where)
    return R.to(device=device, dtype=dtype).contiguous()
