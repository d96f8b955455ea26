"""Build libascq.so (the gfx950 library) in-tree with hipcc.

Usage: python asc-devkit_clone_amd/build.py [--jobs N]

Each translation unit is compiled separately (in parallel) and then linked.  Flags:
  -ffp-contract=off                       every fp32 mul/add stays a separate IEEE op (bit parity)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                          no packed fp32 VALU instructions are generated
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libascq.so"
SOURCES = ["api.cpp", "quant.hip", "gemm_i8.hip", "gemm_f8.hip", "gemv_antiquant.hip", "aq_gemm.hip", "mx_gemm.hip",
           "transpose.hip", "layout.hip"]
ARCH = os.environ.get("ASCQ_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def _compile(src: str) -> Path:
    out = BUILD / (Path(src).stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return out


def build(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    args = ap.parse_args()
    print(build(args.jobs))
    return 0


if __name__ == "__main__":
    sys.exit(main())
