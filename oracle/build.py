"""Build recipe of the oracle's C restatement (oracle/cmoe.c -> oracle/libcmoe.so).

TEST INFRASTRUCTURE ONLY.  The reference has no C or C++ source on this path
(it is Python on MLX with Metal kernels in strings), so there is no
``oracle/_ref`` build.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, "cmoe.c")
LIB = os.path.join(HERE, "libcmoe.so")


def build(verbose: bool = False) -> str:
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-std=c11", SOURCE, "-o", tmp, "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"gcc failed for {SOURCE}:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB
