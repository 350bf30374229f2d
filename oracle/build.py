"""Build the C restatement of the quantizer into ``oracle/_build/`` (test infra).

gcc -O2 -ffp-contract=off (no fast-math): every fp32 operation rounds once.
The reference itself is Python (no compiled path), so there is no
``oracle/_ref`` build.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT_DIR = HERE / "_build"
LIB = OUT_DIR / "libquant_ref.so"


def build() -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-std=c11", "-shared", "-fPIC",
           str(HERE / "quant_ref.c"), "-o", str(LIB), "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle C build failed:\n{res.stderr}")
    return LIB


if __name__ == "__main__":
    print(build())
