"""Build the oracle's C restatement (TEST INFRASTRUCTURE) into oracle/_build/.

    python oracle/build_oracle.py

gcc, plain IEEE fp32 (no -ffast-math), so the host bisection arithmetic
matches the reference's host code.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build"
LIB = OUT / "liboracle_topk.so"


def build() -> Path:
    OUT.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fno-fast-math", "-ffp-contract=off",
           str(HERE / "topk_literal.c"), "-o", str(LIB), "-lm"]
    subprocess.run(cmd, check=True)
    return LIB


if __name__ == "__main__":
    print(build())
