"""Every reference path cited in the tracked sources and documents exists in the reference tree.

Citations such as `docs/zh/api/appendix/mmad_mx_interface_boundary_value_summary.md:11` or
`impl/adv_api/detail/quantization/dequant/ascend_dequant_3510_impl.h:345-598` are how a reader checks a pin; a path
that does not exist pins nothing.  Bare file names (`ascend_quant.h:64`) are not checked.  Skipped where the
reference tree is not mounted."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference")
PREFIXES = ("docs/", "impl/", "examples/", "include/adv_api/", "include/basic_api/", "include/simt_api/",
            "include/c_api/", "include/tensor_api/", "cmake/")
PAT = re.compile(r"(?<![\w/.])((?:" + "|".join(re.escape(p) for p in PREFIXES)
                 + r")[A-Za-z0-9_./\-]*[A-Za-z0-9_]\.(?:md|h|hpp|cpp|asc|py|txt|cmake))")


def _tracked():
    out = subprocess.run(["git", "ls-files"], cwd=ROOT, capture_output=True, text=True, check=True).stdout.split()
    skip = ("SURVEY.md", "BASELINE.md", "VERDICT.md", "ADVICE.md")
    return [ROOT / f for f in out if f.endswith((".h", ".hpp", ".c", ".cpp", ".hip", ".py", ".md")) and f not in skip]


def test_cited_reference_paths_exist():
    if not REF.is_dir():
        pytest.skip("reference tree not mounted")
    missing = {}
    for f in _tracked():
        for m in PAT.finditer(f.read_text(errors="replace")):
            p = m.group(1)
            if not (REF / p).exists():
                missing.setdefault(p, []).append(str(f.relative_to(ROOT)))
    assert not missing, "cited reference paths that do not exist: " + "; ".join(
        f"{p} (in {', '.join(sorted(set(fs))[:3])})" for p, fs in sorted(missing.items()))
