"""Compile the CPU restatement (oracle/hipo_ref.c) -- test infrastructure.

    python oracle/build.py

Produces oracle/_build/libhipo_ref.so with gcc -O2 -fopenmp (no fast-math,
no -march: plain IEEE double/float arithmetic).  The reference itself is
Python-only, so there is nothing to build into oracle/_ref/.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SRC = ORACLE_DIR / "hipo_ref.c"
BUILD_DIR = ORACLE_DIR / "_build"
LIB_PATH = BUILD_DIR / "libhipo_ref.so"


def build(verbose: bool = False) -> Path:
    cc = os.environ.get("CC") or shutil.which("gcc") or "gcc"
    BUILD_DIR.mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, "-O2", "-fopenmp", "-fPIC", "-shared", "-std=c11",
           "-Wall", "-Wextra", "-o", str(tmp), str(SRC), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stdout}{proc.stderr}")
    if verbose and (proc.stdout or proc.stderr):
        print(proc.stdout + proc.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
