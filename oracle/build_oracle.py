"""Build recipe of the CPU oracle (test infrastructure only).

Compiles oracle/mb_oracle.c with gcc into oracle/libmb_oracle.so.  No fast-math and no FP
contraction, so the fp64 sums and the round-half-even helpers follow the C semantics
exactly.

The reference (Isalia20/metalBLAS) is Python + Metal Shading Language: its kernels need
Apple's Metal compiler and runtime, so there is no ``oracle/_ref`` build of it here; the
oracle is pinned against torch's CPU matmul, brute force and closed forms instead.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "mb_oracle.c")
LIB = os.path.join(HERE, "libmb_oracle.so")


def build(verbose: bool = False) -> str:
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-Wall", "-o", tmp, SRC, "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
