"""Builds the CPU oracle (oracle/lokal_oracle.c) into oracle/liblokal_oracle.so.

TEST INFRASTRUCTURE: the oracle is the parity checker and the reported CPU
baseline, never part of the product path.  -ffp-contract=off keeps every
a*b+c as two roundings, as the Rust reference computes it; OpenMP threads the
row loop of matvec as rayon does (src/math.rs:14-16).
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "lokal_oracle.c"
LIB = HERE / "liblokal_oracle.so"

CFLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-Wall"]


def build(verbose: bool = False) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", *CFLAGS, str(SRC), "-o", str(tmp), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stderr}")
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
