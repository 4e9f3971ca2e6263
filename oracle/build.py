"""Builds the C restatement (oracle/moe_cpu.c) as oracle/libmoe_cpu.so.

Test infrastructure only: the tests cross-check it against the numpy oracle and
``bench.py`` times it as the CPU baseline.  x86-64-v3 (AVX2/FMA) keeps the
library portable between this container and the benchmark host; contraction
into FMA is disabled so the rounding points stay those of the numpy oracle.
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "moe_cpu.c")
LIB = os.path.join(HERE, "libmoe_cpu.so")
CFLAGS = ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared",
          "-std=c11", "-Wall"]


def build(verbose: bool = False) -> str:
    tmp = LIB + ".tmp"
    cmd = ["gcc", *CFLAGS, SRC, "-o", tmp, "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("gcc failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
