"""Rotation calibration, worker side (oscar_ascend/calib.py:1-149).

With ``OSCAR_ASCEND_CALIB=1`` the plugin swaps no attention impl. Instead it
registers a forward pre-hook on every decoder full-attention module
(``register_attention_hook``). During the engine's own forward passes the hook
keeps the unquantized Q, K and V entering ``Attention.forward``, up to
``OSCAR_ASCEND_CALIB_TOKEN_CAP`` tokens per layer (default 512). The captures
stay on the device. After a calibration ``generate``, ``finalize_cov`` (run
in each worker through ``apply_model``) reduces each layer's captures to the
two matrices whose eigenvectors the rotations start from:

  Sigma_Q = (1/Hk) sum_h sym(Q_h^T Q_h / (n g))
      Q_h is the [n g, D] stack of the g query heads of kv head h. This is
      the K rotation's hessian (the qqt objective).
  Sigma_S = (1/Hk) sum_h sym((V_h sqrt(w))^T (V_h sqrt(w)) / n)
      w_i = k_i^T sym(Q_h^T Q_h / (n g)) k_i, rescaled so that sum_i w_i = n.
      This is the V rotation's score-weighted hessian (the sst objective).

sym(A) = (A + A^T) / 2.  Both are computed in fp32 on the capture device and
returned on the CPU with the token count n, as the reference returns them.
``oscar_amd.gen_rotations`` merges the workers' results and composes the
rotations.
"""
from __future__ import annotations

import os

import torch

_captures: dict[str, dict[str, list]] = {}
_TOKEN_CAP = int(os.environ.get("OSCAR_ASCEND_CALIB_TOKEN_CAP", "512"))
_REGISTERED: set[int] = set()


def _calibrated_layer(layer_name: str) -> bool:
    """calib.py:34-44 — decoder self-attention only: no linear-attention and
    no MTP draft layer (those keep native caches and need no rotation)."""
    if ".self_attn" not in layer_name or ".linear_attn" in layer_name:
        return False
    return not (".mtp." in layer_name or layer_name.startswith("mtp."))


def _heads(x: torch.Tensor, take: int, heads: int, D: int) -> torch.Tensor:
    x = x[:take].detach()
    return (x.reshape(-1, heads, D) if x.dim() == 2 else x).float()


def register_attention_hook(attn_module) -> None:
    """calib.py:31-86 — capture hook on one Attention module (once per module).

    ``Attention.forward(query, key, value, ...)`` receives [N, H*D] (or
    already [N, H, D]) tensors. The hook restores the head view from the
    module's ``num_heads`` / ``num_kv_heads`` / ``head_size`` and appends at
    most the tokens still missing to reach the cap."""
    layer_name = getattr(attn_module, "layer_name", "") or ""
    if not _calibrated_layer(layer_name) or id(attn_module) in _REGISTERED:
        return
    _REGISTERED.add(id(attn_module))

    def hook(module, args, kwargs=None):
        if not args or len(args) < 3 or any(t is None for t in args[:3]):
            return None
        q, k, v = args[0], args[1], args[2]
        hq = int(getattr(module, "num_heads", 0) or 0)
        hk = int(getattr(module, "num_kv_heads", 0) or 0)
        D = int(getattr(module, "head_size", 0) or 0)
        if hq <= 0 or hk <= 0 or D <= 0 or q.shape[-1] % (hq * D if q.dim() == 2 else D):
            print(f"[oscar-amd][calib] cannot restore the head view of {layer_name}; not captured")
            return None
        store = _captures.setdefault(layer_name, {"q": [], "k": [], "v": []})
        have = sum(t.shape[0] for t in store["k"])
        if have >= _TOKEN_CAP:
            return None
        take = min(k.shape[0], _TOKEN_CAP - have)
        store["q"].append(_heads(q, take, hq, D))
        store["k"].append(_heads(k, take, hk, D))
        store["v"].append(_heads(v, take, hk, D))
        return None

    attn_module.register_forward_pre_hook(hook)


def reset_captures(model=None) -> None:
    """calib.py:89-93 — drop every capture (``apply_model`` signature fn(model))."""
    _captures.clear()


def _sym(a: torch.Tensor) -> torch.Tensor:
    return (a + a.t()) / 2


def layer_hessians(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """calib.py:123-141 — (Sigma_Q, Sigma_S) of one layer's [n, H, D] captures, fp32."""
    n, hq, D = q.shape
    hk = k.shape[1]
    g = hq // hk
    sigma_q = torch.zeros(D, D, device=q.device, dtype=torch.float32)
    sigma_s = torch.zeros(D, D, device=q.device, dtype=torch.float32)
    for h in range(hk):
        qh = q[:, h * g:(h + 1) * g, :].float().reshape(-1, D)
        kh, vh = k[:, h, :].float(), v[:, h, :].float()
        qtq = _sym(qh.t() @ qh / qh.shape[0])
        sigma_q += qtq
        w = ((kh @ qtq) * kh).sum(1)
        w = w / w.sum().clamp(min=1e-12) * n
        vw = vh * w.unsqueeze(1).sqrt()
        sigma_s += _sym(vw.t() @ vw / n)
    return sigma_q / hk, sigma_s / hk


def finalize_cov(model=None) -> dict:
    """calib.py:96-149 — {layer: {"q": {"cov": Sigma_Q, "count": n}, "v": {"cov": Sigma_S, "count": n}}}.

    Layers whose captures are not [n, H, D] or whose head counts do not
    divide are skipped with a message. The matrices come back on the CPU."""
    out = {}
    for layer_name, store in _captures.items():
        if not store["k"] or not store["q"]:
            continue
        q, k, v = (torch.cat(store[key], dim=0) for key in ("q", "k", "v"))
        if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
            print(f"[oscar-amd][calib] {layer_name}: captures are not [n, H, D]; skipped")
            continue
        hq, hk = q.shape[1], k.shape[1]
        if hq < hk or hq % hk:
            print(f"[oscar-amd][calib] {layer_name}: Hq={hq} is not a multiple of Hk={hk}; skipped")
            continue
        sigma_q, sigma_s = layer_hessians(q, k, v)
        n = k.shape[0]
        out[layer_name] = {"q": {"cov": sigma_q.detach().cpu(), "count": n},
                           "v": {"cov": sigma_s.detach().cpu(), "count": n}}
    return out
