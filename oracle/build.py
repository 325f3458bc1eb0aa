"""Build the oracle's C restatement (test infrastructure only).

liboracle_f64.so  REAL=double, no FP contraction: the parity oracle.
liboracle_f32.so  REAL=float, OpenMP + AVX2/FMA: the timed CPU baseline.
"""
from __future__ import annotations

import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
OUT = HERE / "_build"


def build(verbose: bool = False) -> None:
    OUT.mkdir(exist_ok=True)
    src = str(HERE / "ltx_oracle.c")
    cmds = [
        ["gcc", "-O3", "-fopenmp", "-fPIC", "-shared", "-march=x86-64-v3", "-ffp-contract=off", "-DREAL=double", src,
         "-o", str(OUT / "liboracle_f64.so"), "-lm"],
        ["gcc", "-O3", "-fopenmp", "-fPIC", "-shared", "-march=x86-64-v3", "-DREAL=float", "-DREAL_F32", src,
         "-o", str(OUT / "liboracle_f32.so"), "-lm"],
    ]
    for c in cmds:
        if verbose:
            print(" ".join(c))
        r = subprocess.run(c, capture_output=True, text=True)
        if r.returncode:
            sys.stderr.write(r.stderr)
            raise RuntimeError("oracle build failed")


if __name__ == "__main__":
    build(verbose=True)
