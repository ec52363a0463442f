"""Build oracle/liboracle.so from oracle/c/oracle.c with gcc (test oracle)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = True) -> str:
    src = os.path.join(HERE, "c", "oracle.c")
    cmd = ["gcc", "-O2", "-std=c99", "-shared", "-fPIC", "-o", LIB, src, "-lm"]
    subprocess.run(cmd, check=True)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
