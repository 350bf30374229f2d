"""Build the gfx950 HIP library ``oscar_amd/_oscar_hip.so`` in-tree.

Every ``*.hip`` file here is compiled separately (the quantizer without FP
contraction, so its fp32 ops round exactly like the reference's) and linked
into one shared library exporting the C ABI declared in include/oscar_amd.h.

Usage: python -m oscar_amd.csrc.build   (or __graft_entry__.build()).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
OUT = PKG / "_oscar_hip.so"
BUILD_DIR = PKG / "_build"

ARCH = "gfx950"
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed FP32 VALU forms stay off (they have given wrong results on this
    # pool); hipcc's host pass warns that it does not know the feature.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
PER_FILE = {
    "quant_write.hip": ["-ffp-contract=off"],
    "step_write.hip": ["-ffp-contract=off"],
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the OSCAR HIP library cannot be built")
    return path


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, *PER_FILE.get(src.name, []), "-I", str(HERE), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(HERE.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(len(sources), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT.relative_to(PKG.parent)} from {[s.name for s in sources]}")
    return OUT


if __name__ == "__main__":
    build()
