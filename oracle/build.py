"""Build the oracle's C part: oracle/liboracle.so (gcc, CPU only).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  The reference has no native
code for this path (it has no MoE at all), so there is no oracle/_ref build:
nothing under /root/reference compiles into a checker.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "g5moe_oracle.c"
LIB = HERE / "liboracle.so"


def build(verbose: bool = False) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-Wall",
           str(SRC), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
