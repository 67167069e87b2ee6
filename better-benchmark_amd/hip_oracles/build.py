"""Build libhip_oracles.so for gfx950 with hipcc (in-tree, no CMake).

    python better-benchmark_amd/hip_oracles/build.py [--verbose]

Each csrc/*.hip file is compiled to an object under hip_oracles/_build/ and
the objects are linked into hip_oracles/libhip_oracles.so, which the ctypes
loader in hip_oracles/__init__.py opens.  Every call recompiles everything
(the build is the "does it compile" check and takes seconds).
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
REPO_ROOT = PKG_DIR.parents[1]
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libhip_oracles.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = "gfx950"
SOURCES = [
    "hipo_abi.hip",
    "row_mean.hip",
    "bias_gelu_nhwc.hip",
    "masked_softmax.hip",
    "row_norms.hip",
    "batchnorm.hip",
    "batchnorm_fused.hip",
    "spatial_mean.hip",
    "batchnorm_bf16.hip",
    "flat_copy.hip",
    "gelu_flat.hip",
    "transpose.hip",
    "gelu_bwd.hip",
]

# Packed-FP32 VALU forms are disabled for all device code (the compiler
# otherwise emits v_pk_{add,mul,fma}_f32 from plain float code).  The host
# pass prints a harmless "not a recognized feature" warning for this flag.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every source and link the shared library; returns its path."""
    cc = hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([cc, *DEVICE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}",
                     "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=8)
    args = ap.parse_args(argv)
    path = build(verbose=args.verbose, jobs=args.jobs)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
