"""Build recipe of the CPU oracle (test infrastructure, see nsr_oracle.c).

Compiles oracle/nsr_oracle.c into oracle/_build/libnsr_oracle.so with
gcc -O2 -ffp-contract=off -fopenmp (generic x86-64, no FMA contraction, no
fast-math), so the restated f32 op sequences round as the reference's Rust
code does.

The reference's own CPU path (Rust on a git-fork Candle with no Cargo.lock
and no vendored sources) cannot be compiled in this image, so there is no
oracle/_ref build.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT_DIR = HERE / "_build"
LIB = OUT_DIR / "libnsr_oracle.so"


def build() -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    tmp = OUT_DIR / "libnsr_oracle.so.tmp"
    cmd = [
        "gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
        "-fopenmp", "-Wall", "-Wextra", "-Wno-unused-parameter",
        str(HERE / "nsr_oracle.c"), "-lm", "-o", str(tmp),
    ]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("oracle build failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
