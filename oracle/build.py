"""Compile the oracle's C restatement into ``oracle/liboracle.so``.

Test infrastructure only (see oracle/__init__.py).  gcc -O2 with
-ffp-contract=off and no fast-math, so each float operation in oracle.c
rounds once in program order.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "oracle.c")
OUT = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = False) -> str:
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-o", OUT + ".tmp", SRC, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(OUT + ".tmp", OUT)
    if verbose:
        print(f"[oracle.build] -> {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
