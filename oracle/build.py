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
# The CPU-baseline build: the same source at -O3 with AVX2, so the 8
# independent lanes of math::dot (src/math.rs:20-24) become one 256-bit
# multiply and add as rustc's release build vectorises them.  Still no
# contraction and no fast-math: every lane rounds exactly as at -O2, and
# tests/test_oracle.py checks the two builds' logits are bit-identical.
LIB_O3 = HERE / "liblokal_oracle_o3.so"
CFLAGS_O3 = ["-O3", "-mavx2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
             "-Wall"]


def _gcc(flags: list[str], out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = ["gcc", *flags, str(SRC), "-o", str(tmp), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stderr}")
    tmp.replace(out)


def build(verbose: bool = False) -> Path:
    """Builds the parity oracle (-O2) and the CPU-baseline build (-O3 -mavx2)."""
    _gcc(CFLAGS, LIB)
    _gcc(CFLAGS_O3, LIB_O3)
    if verbose:
        print(f"built {LIB} and {LIB_O3.name}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
