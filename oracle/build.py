"""Builds the C part of the oracle (raster_seq.c) with gcc. TEST INFRASTRUCTURE.

Output: oracle/_build/libraster_seq.so. No FP contraction beyond the explicit
fmaf calls (-ffp-contract=off), no fast-math: the file relies on IEEE fp32.

The reference itself (Metal shaders + an ObjC++ torch extension) needs the
Metal framework and cannot be built here, so there is no oracle/_ref build.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "libraster_seq.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-std=c11",
           "-Wall", "-o", str(tmp), str(HERE / "raster_seq.c"), "-lm"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{p.stdout}\n{p.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
