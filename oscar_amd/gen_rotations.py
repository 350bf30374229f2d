"""Offline per-layer rotation checkpoints (tools/gen_rotations.py:1-249).

``python -m oscar_amd.gen_rotations --model PATH --save oscar_rotations.pt``
builds a vLLM engine on the ROCm platform with ``OSCAR_ASCEND_CALIB=1``, so
the plugin registers capture hooks (``oscar_amd.calib``) instead of swapping
impls. It then clears the captures, runs one calibration prompt through the
engine's normal generate path, and collects each worker's per-layer
(Sigma_Q, Sigma_S). The workers' statistics are merged weighted by token
count, and each layer's rotations are composed as

    R = U @ H @ P_br

U holds the eigenvectors of the merged hessian (ascending eigenvalues, as
``torch.linalg.eigh`` returns them), H is the normalised Sylvester Hadamard
matrix, and P_br places the i-th largest eigen-direction at column
bitrev(i). The high-variance directions are spread evenly over the features,
so no outlier direction dominates a vector's INT2 min/max. R_k comes from
Sigma_Q and R_v from Sigma_S. The eigendecomposition and the composition run
on the CPU in fp64. The checkpoint is format v2:
``{"format_version": 2, "objective": "qqt_r_h_pbr_k / sst_r_h_pbr_v",
"source_grouping": "layer", "layers": {"<id>": {"layer_id", "rotation",
"rotation_v", "eigenvalues", "eigenvalues_v"}}}``, which
``oscar_amd.rotation.load_checkpoint`` reads.

On MI355X one GPU holds the whole model (288 GB), so the engine defaults to
tensor_parallel_size=1; ``OSCAR_ASCEND_GEN_LLM_ARGS`` (JSON) overrides any
``LLM`` argument.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
from pathlib import Path

import torch

FORMAT_VERSION = 2
OBJECTIVE = "qqt_r_h_pbr_k / sst_r_h_pbr_v"
_LAYER_ID = re.compile(r"\.layers\.(\d+)\.")
CALIBRATION_TEXT = (
    "Calibration text for the OSCAR rotations: attention keys and values of a long technical passage. "
    "A model should keep stable hidden states over long sequences and spend little quantization noise "
    "on the directions its attention scores depend on. "
)


def _power_of_two(n: int, what: str) -> None:
    if n < 1 or n & (n - 1):
        raise ValueError(f"{what} size must be a power of two, got {n}")


def hadamard(n: int) -> torch.Tensor:
    """gen_rotations.py:93-100 — normalised Sylvester Hadamard [n, n] in fp64:
    H_1 = [1], H_2m = [[H_m, H_m], [H_m, -H_m]] / sqrt(2)."""
    _power_of_two(n, "Hadamard")
    h = torch.ones(1, 1, dtype=torch.float64)
    while h.shape[0] < n:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0) / 2 ** 0.5
    return h


def bit_reversal_perm(d: int) -> torch.Tensor:
    """gen_rotations.py:103-107 — i -> i with its log2(d) bits reversed."""
    _power_of_two(d, "Bit-reversal")
    bits = d.bit_length() - 1
    idx = torch.arange(d)
    out = torch.zeros(d, dtype=torch.long)
    for b in range(bits):
        out |= ((idx >> b) & 1) << (bits - 1 - b)
    return out


def br_permutation(eigenvalues: torch.Tensor) -> torch.Tensor:
    """gen_rotations.py:110-118 — P_br [d, d] (fp64): column bitrev(i) of M @ P_br
    is column sorted[i] of M, where sorted orders the eigenvalues descending.
    Ties keep their index order."""
    d = eigenvalues.numel()
    order = torch.argsort(eigenvalues, descending=True, stable=True)
    perm = torch.empty(d, dtype=torch.long)
    perm[bit_reversal_perm(d)] = order
    return torch.eye(d, dtype=torch.float64)[:, perm]


def compose_rotation(eigenvectors: torch.Tensor, eigenvalues: torch.Tensor,
                     h: torch.Tensor | None = None) -> torch.Tensor:
    """gen_rotations.py:121-124 — U @ H @ P_br."""
    U = eigenvectors.double()
    if h is None:
        h = hadamard(U.shape[0])
    return U @ h.double() @ br_permutation(eigenvalues)


def rotation_from_stats(stats: dict, D: int) -> tuple[torch.Tensor, torch.Tensor]:
    """gen_rotations.py:127-146 — merged hessian -> (R = U H P_br fp32, eigenvalues fp32).

    The mean hessian is symmetrised in fp64 and regularised by 1e-6 I
    before ``eigh``."""
    count = max(1, int(stats["count"]))
    cov = (stats["cov_sum"] / count).double()
    cov = (cov + cov.t()) / 2 + 1e-6 * torch.eye(D, dtype=torch.float64)
    try:
        evals, evecs = torch.linalg.eigh(cov)
    except Exception as e:  # noqa: BLE001 - NaN/inf statistics
        raise RuntimeError(f"eigh failed (non-finite hessian?): {e}") from e
    rot = compose_rotation(evecs, evals)
    err = (rot @ rot.t() - torch.eye(D, dtype=torch.float64)).abs().max().item()
    if err > 1e-6:
        print(f"[gen-rotations] composed rotation is orthogonal only to {err:.2e}")
    return rot.float().contiguous(), evals.float().contiguous()


def merge_rank_stats(per_rank: list, D: int) -> dict:
    """gen_rotations.py:73-88 — {layer: {"q"|"v": {"cov_sum", "count"}}}: each rank's
    mean hessian weighted by its token count."""
    merged: dict = {}
    for rank_stats in per_rank:
        for layer, st in rank_stats.items():
            for kind in ("q", "v"):
                agg = merged.setdefault(layer, {}).setdefault(
                    kind, {"cov_sum": torch.zeros(D, D, dtype=torch.float32), "count": 0})
                agg["cov_sum"] = agg["cov_sum"] + st[kind]["cov"].float() * st[kind]["count"]
                agg["count"] += st[kind]["count"]
    return merged


def build_checkpoint(merged: dict, D: int) -> dict:
    """gen_rotations.py:208-239 — the format-v2 checkpoint of the merged statistics.
    Layer names without a ``.layers.<i>.`` index are skipped."""
    layers = {}
    for name, st in sorted(merged.items()):
        m = _LAYER_ID.search(name)
        if m is None:
            print(f"[gen-rotations] no layer index in {name!r}; skipped")
            continue
        lid = int(m.group(1))
        r_k, e_k = rotation_from_stats(st["q"], D)
        r_v, e_v = rotation_from_stats(st["v"], D)
        layers[str(lid)] = {"layer_id": lid, "rotation": r_k, "rotation_v": r_v,
                            "eigenvalues": e_k, "eigenvalues_v": e_v}
    if not layers:
        raise ValueError("no layer statistics to build rotations from")
    return {"format_version": FORMAT_VERSION, "objective": OBJECTIVE, "source_grouping": "layer",
            "layers": layers}


def calibrate(llm, D: int, max_len: int) -> dict:
    """gen_rotations.py:189-206 — clear the captures, run the calibration prompt,
    collect and merge every worker's statistics."""
    from vllm import SamplingParams

    from . import calib

    llm.llm_engine.apply_model(calib.reset_captures)
    prompt = (CALIBRATION_TEXT * 8)[:max(64, max_len - 8)]
    llm.generate(prompt, SamplingParams(max_tokens=4, temperature=0.0))
    per_rank = llm.llm_engine.apply_model(calib.finalize_cov)
    if not per_rank or not any(per_rank):
        raise RuntimeError("no K/V captured: check OSCAR_ASCEND_CALIB=1 and the model's attention layers")
    return merge_rank_stats(per_rank, D)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model", required=True)
    ap.add_argument("--save", default="oscar_rotations.pt")
    ap.add_argument("--max-len", type=int, default=128)
    ap.add_argument("--head-dim", type=int, default=256)
    args = ap.parse_args(argv)
    # Workers are spawned (a forked child cannot use the parent's HIP state);
    # apply_model sends module-level functions, which needs pickled RPC.
    os.environ.setdefault("VLLM_WORKER_MULTIPROC_METHOD", "spawn")
    os.environ.setdefault("VLLM_ALLOW_INSECURE_SERIALIZATION", "1")
    os.environ["OSCAR_ASCEND_CALIB"] = "1"
    os.environ.pop("OSCAR_ASCEND_ENABLE", None)
    torch.set_num_threads(min(4, max(1, torch.get_num_threads())))

    from vllm import LLM

    llm_args = json.loads(os.environ.get("OSCAR_ASCEND_GEN_LLM_ARGS", "{}"))
    llm_args.setdefault("tensor_parallel_size", 1)
    llm_args.setdefault("gpu_memory_utilization", 0.9)
    llm = LLM(model=args.model, enforce_eager=True, max_model_len=max(args.max_len + 16, 128),
              dtype="bfloat16", **llm_args)
    merged = calibrate(llm, args.head_dim, args.max_len)
    ckpt = build_checkpoint(merged, args.head_dim)
    Path(args.save).parent.mkdir(parents=True, exist_ok=True)
    torch.save(ckpt, args.save)
    print(f"[gen-rotations] saved {args.save} (layers={len(ckpt['layers'])}, D={args.head_dim}); serve with "
          f"OSCAR_ASCEND_K_ROTATION_PATH={args.save} OSCAR_ASCEND_V_ROTATION_PATH={args.save}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
