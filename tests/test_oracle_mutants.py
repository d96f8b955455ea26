"""The oracle's pins must catch plausible mistakes.

oracle/ascq_oracle.c carries planted-mistake switches (OQ_MUTANT = n): a dropped 13-bit truncation of the
QUANT_PRE multiplier, half-away instead of half-even rounding, a swapped int4 nibble order, a dropped bias, a
reordered group-matmul epilogue, a transposed MX scale index, offset/scale applied in the wrong order, a
double-rounded multiplier, a wrong E2M1 code, a ties-away f16 cast, an unrounded half add, a per-channel
dequant indexed by row, a requant offset added before the clamp, a ties-away fp8 cast, an ignored requant
sign flag, a FasterGelu with the wrong sign, and policy-form quant mistakes (arithmetic type, bf16 step, group
axis, offset rounding, directed E2M1 modes) and dequant layout mistakes (int32 rounding, the single-row
reshape, padded dst rows, group axis) and HiFloat8 / arch-3510 legacy quant mistakes, MX E1M2 / bias and enAtomic
mistakes, and the newer Quantize / AntiQuantize interface's channel index and fp32 arithmetic.  Each mutant is compiled on the CPU into a temporary library and the pinning tests of
tests/test_oracle.py are run against it; every mutant must fail at least one of them.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "oracle" / "ascq_oracle.c"

MUTANTS = {
    1: "QUANT_PRE M1 not truncated to (1,8,10) bits",
    2: "rint replaced by round-half-away",
    3: "int4 nibble order swapped",
    4: "int32 bias dropped",
    5: "group epilogue multiplies the per-token scale first",
    6: "MX [sK/2, N, 2] scale layout read as [N, sK]",
    7: "antiquant multiplies before adding the offset",
    8: "dynamic quant multiplier 1/(absmax/127) (double rounding)",
    9: "E2M1 code 5 decoded as 2.5",
    10: "f32->f16 ties rounded away from zero",
    11: "legacy quant: product not rounded to half before the offset add",
    12: "per-channel dequant indexed by row",
    13: "requant offset added before the [-256, 255] clamp",
    14: "f32->fp8 ties rounded away from zero",
    15: "requant sign flag ignored (always int8 saturation)",
    16: "FasterGelu coefficient with the wrong sign",
    17: "int4 requant without the 9-bit offset",
    18: "int4 requant output nibbles swapped",
    19: "per-group antiquant scales indexed along the wrong axis",
    20: "fp8 antiquant computed in the scale type instead of fp32",
    21: "fp8 quant computed in the scale type instead of fp32",
    22: "E2M1 quant cast without the bf16 rounding step",
    23: "per-group quant scales indexed along the wrong axis",
    24: "quant product not rounded to the scale type before the offset add",
    25: "E2M1 floor / ceil applied to the magnitude regardless of sign",
    26: "E1M2 rint ties resolved toward zero instead of to the even code",
    27: "dequant int32 -> fp32 rounded to nearest even instead of ties away",
    28: "legacy dequant without the DEQUANT_WITH_SINGLE_ROW reshape",
    29: "legacy dequant dst rows not padded to 32 bytes",
    30: "per-group dequant scales indexed along the wrong axis",
    31: "HiFloat8 encoder writes the 2-bit exponent field for every |E| >= 2",
    32: "legacy quant to fp8 computed in half arithmetic instead of fp32",
    33: "HiFloat8 ties rounded toward zero instead of away",
    34: "HiFloat8 decoder reads the 1-bit exponent field's sign inverted",
    35: "MX E1M2 elements decoded as E2M1",
    36: "MX bias dropped",
    37: "enAtomic max / min swapped",
    38: "group epilogue int32 -> fp32 rounded to nearest even instead of ties away",
    39: "hifloat8 Matmul operands decoded as fp8 e4m3",
    40: "Quantize / AntiQuantize PER_CHANNEL scales indexed by row",
    41: "Quantize computed in the scale type instead of fp32",
    42: "AntiQuantize computed in the scale type instead of fp32",
}


@pytest.fixture(scope="module")
def mutant_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("oracle_mutants")


def _build(n: int, d: Path) -> Path:
    so = d / f"liboracle_m{n}.so"
    cmd = ["gcc", "-O2", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-ffp-contract=off", "-std=c11", "-shared",
           f"-DOQ_MUTANT={n}", "-o", str(so), str(SRC), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True)
    return so


@pytest.mark.parametrize("n", sorted(MUTANTS))
def test_pins_reject_mutant(n, mutant_dir):
    so = _build(n, mutant_dir)
    env = dict(os.environ, ASCQ_ORACLE_SO=str(so), OMP_NUM_THREADS="4")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-W", "ignore",
                        str(ROOT / "tests" / "test_oracle.py")], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=600)
    assert r.returncode != 0, f"mutant {n} ({MUTANTS[n]}) passed every pin:\n{r.stdout[-2000:]}"


def test_unmutated_oracle_passes(mutant_dir):
    so = _build(0, mutant_dir)
    env = dict(os.environ, ASCQ_ORACLE_SO=str(so), OMP_NUM_THREADS="4")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-W", "ignore",
                        str(ROOT / "tests" / "test_oracle.py")], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stdout[-3000:]
