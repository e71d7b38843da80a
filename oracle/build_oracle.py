"""Compile the C restatement of the oracle into oracle/_build/libfp8_oracle.so.

Test infrastructure only.  Called by ``__graft_entry__.build()``.  Plain gcc,
OpenMP, no fast-math and no FP contraction so every fp32 operation rounds the
way the restated torch/Triton code rounds it.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "c" / "fp8_oracle.c"
OUT_DIR = HERE / "_build"
LIB = OUT_DIR / "libfp8_oracle.so"


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [
        "gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
        "-fno-fast-math", "-std=c11", "-Wall", "-Wextra",
        str(SRC), "-o", str(tmp), "-lm",
    ]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
