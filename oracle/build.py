"""Builds the oracle's C restatement (oracle/oracle.c) into oracle/_build/liboracle.so with gcc.

Test infrastructure only (the checker and the CPU baseline). The reference itself is Elixir
on Nx/EXLA and has no C sources to compile, so there is no oracle/_ref build.
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(BUILD, "liboracle.so")


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fPIC", "-shared", "-Wall", "-fopenmp",
           "-o", tmp, os.path.join(HERE, "oracle.c"), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"gcc failed on oracle.c:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
