"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only, no GPU needed).

- The C ABI's host layer (csrc/api.cpp) is rebuilt with the sanitizers on its host side only (hipcc
  -Xarch_host -fsanitize=...; the device code is the normal build's) and linked with the other objects of the
  normal build into tests/cpp/sanitize_abi.cpp, which drives every entry point's argument checks.
- The oracle (oracle/ascq_oracle.c) is built with gcc -fsanitize=address,undefined and driven by
  tests/cpp/sanitize_oracle.c over its codecs, matmuls, epilogues and the enAtomic combine."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BUILD = ROOT / "asc-devkit_clone_amd" / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CLANGXX = "/opt/rocm/lib/llvm/bin/clang++"
SAN_ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1",
               OMP_NUM_THREADS="2")


def test_c_abi_host_checks_under_sanitizers(tmp_path):
    objs = sorted(p for p in BUILD.glob("*.o") if p.name != "api.o")
    if not objs or not Path(HIPCC).exists() or not Path(CLANGXX).exists():
        pytest.skip("needs the normal build's objects (asc-devkit_clone_amd/build.py) and the ROCm compilers")
    api = tmp_path / "api_san.o"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-ffp-contract=off",
                    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                    "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
                    "-x", "hip", "-c", str(ROOT / "asc-devkit_clone_amd" / "csrc" / "api.cpp"), "-o", str(api)],
                   check=True, capture_output=True)
    exe = tmp_path / "sanitize_abi"
    subprocess.run([CLANGXX, "-g", "-fsanitize=address,undefined", "-I", str(ROOT / "include"),
                    str(ROOT / "tests" / "cpp" / "sanitize_abi.cpp"), str(api), *map(str, objs),
                    "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=SAN_ENV)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ok: 0 failure(s)" in r.stdout


def test_oracle_under_sanitizers(tmp_path):
    exe = tmp_path / "sanitize_oracle"
    subprocess.run(["gcc", "-O1", "-g", "-std=c11", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-fno-omit-frame-pointer", "-fopenmp", "-I", str(ROOT / "oracle"),
                    str(ROOT / "tests" / "cpp" / "sanitize_oracle.c"), str(ROOT / "oracle" / "ascq_oracle.c"),
                    "-lm", "-o", str(exe)], check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120,
                       env=dict(SAN_ENV, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1"))
    assert r.returncode == 0, r.stdout + r.stderr
