"""Pins of the oracle (CPU, no GPU).

Every oracle function is checked against something other than its own formula:
  * the reference examples' golden procedures (tests/golden/*.npz, see make_golden.py) with the reference's
    verification tolerances where its golden is itself approximate;
  * trusted IEEE implementations: numpy float16 casts, torch bfloat16 / float8 casts, numpy float32 arithmetic;
  * closed forms and brute force on small inputs (exact rationals, nearest-neighbour search over a codebook).
"""
from __future__ import annotations

import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle_lib as O

GOLD = Path(__file__).resolve().parent / "golden"
rng0 = np.random.default_rng(12345)


def ref_verify(out, golden, rtol=1e-3, atol=1e-3, err_tol=1e-3):
    """verify_result.py of the reference examples: np.isclose with rtol/atol, error ratio <= err_tol."""
    bad = ~np.isclose(out.astype(np.float64), golden.astype(np.float64), rtol=rtol, atol=atol, equal_nan=True)
    return bad.mean() <= err_tol


# --------------------------------------------------------------------------- scalar codecs
def _random_f32(n):
    bits = rng0.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0, 0x80000000, 0x33000000, 0x33000001, 0x387FE000, 0x387FF000, 0x38800000, 0x477FE000,
                         0x477FEFFF, 0x477FF000, 0x477FF001, 0x7F800000, 0xFF800000, 0x7FC00000, 0x3F801000,
                         0x3F803000, 0x3F800FFF, 0x00000001], np.uint32)
    # values in the f16 range with exact ties at the 13 discarded bits
    ties = (rng0.integers(0x33000000, 0x47800000, n // 4, dtype=np.uint64).astype(np.uint32) & ~np.uint32(0x1FFF)) | 0x1000
    return np.concatenate([bits, specials, ties]).view(np.float32)


def test_f32_to_f16_matches_numpy():
    x = _random_f32(40000)
    got = O.f32_to_f16(x, sat=False)
    exp = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert (got[~nan] == exp[~nan]).all()
    assert np.isnan(got[nan].view(np.float16)).all()


def test_f32_to_f16_saturating():
    x = _random_f32(20000)
    got = O.f32_to_f16(x, sat=True).view(np.float16).astype(np.float32)
    fin = ~np.isnan(x)
    exp = np.clip(x[fin], -65504, 65504).astype(np.float16).astype(np.float32)
    assert (got[fin] == exp).all()


def test_f16_to_f32_all_codes():
    L = O.lib()
    codes = np.arange(65536, dtype=np.uint16)
    got = np.array([L.oq_f16_to_f32(int(c)) for c in codes], np.float32)
    exp = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(exp)
    assert (got[~nan].view(np.uint32) == exp[~nan].view(np.uint32)).all() and np.isnan(got[nan]).all()


def test_f32_to_bf16_matches_torch():
    L = O.lib()
    x = _random_f32(30000)
    x = x[np.isfinite(x) & (np.abs(x) < 3.38e38)]
    got = np.array([L.oq_f32_to_bf16(float(v), 0) for v in x], np.uint16)
    exp = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (got == exp).all()
    assert L.oq_f32_to_bf16(3.4e38, 1) == 0x7F7F and L.oq_f32_to_bf16(float("inf"), 1) == 0x7F7F
    assert L.oq_f32_to_bf16(-float("inf"), 1) == 0xFF7F


def test_f64_to_f16_matches_numpy():
    L = O.lib()
    d = np.concatenate([rng0.standard_normal(20000) * 10.0 ** rng0.integers(-8, 5, 20000),
                        np.array([1 + 2.0 ** -11, 1 + 2.0 ** -11 + 2.0 ** -40, 2.0 ** -25, 3 * 2.0 ** -26, 65519.99,
                                  65520.0, 2049.0, 2051.0])])
    got = np.array([L.oq_f64_to_f16(float(v), 0) for v in d], np.uint16)
    exp = d.astype(np.float16).view(np.uint16)
    assert (got == exp).all()


def _nearest_even(d, grid):
    """brute-force round-to-nearest-even of d onto a sorted grid of (value, code) pairs"""
    vals = grid[0]
    i = np.searchsorted(vals, d)
    cands = [j for j in (i - 1, i) if 0 <= j < len(vals)]
    best = min(cands, key=lambda j: (abs(vals[j] - d), grid[1][j] & 1))
    return grid[1][best]


def test_f64_to_bf16_brute_force():
    L = O.lib()
    codes = np.arange(0, 0x7F80, dtype=np.uint16)
    vals = (codes.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    grid = (vals, codes)
    for d in np.concatenate([np.abs(rng0.standard_normal(3000)) * 10.0 ** rng0.integers(-30, 30, 3000),
                             vals[1000:1010] + (vals[1001:1011] - vals[1000:1010]) / 2]):
        assert L.oq_f64_to_bf16(float(d), 0) == _nearest_even(d, grid)
        assert L.oq_f64_to_bf16(float(-d), 0) == (_nearest_even(d, grid) | 0x8000)


def test_quant_pre_m1_matches_gen_data_decode():
    """accompanying_quantization.md table 1 / gen_data_s322f16.py extract_quant_params: M1 = (-1)^s (1+m/1024)
    2^(e-127) from bits [31:13]; offset bits [45:37]; sign flag bit 46."""
    L = O.lib()
    for f in [0.1, 1.0, -0.5, 3.14159, 2.0 ** -12, 1e-30, 65504.0, -7.7e10]:
        w = L.oq_pack_quant_pre(f, 0, 0)
        bits = (w >> 13) & 0xFFFFF
        s, e, m = (bits >> 18) & 1, (bits >> 10) & 0xFF, bits & 0x3FF
        ref = (-1) ** s * (1 + m / 1024) * 2.0 ** (e - 127)
        assert L.oq_quant_pre_m1(w) == np.float32(ref)
    w = L.oq_pack_quant_pre(1.0, -5, 1)
    assert (w >> 37) & 0x1FF == (-5) & 0x1FF and (w >> 46) & 1 == 1
    assert L.oq_quant_pre_m1(np.float32(0.1).view(np.uint32)) == np.float32(0.0999755859375)


@pytest.mark.parametrize("mode,fn", [(O.ROUND_RINT, np.rint), (O.ROUND_FLOOR, np.floor), (O.ROUND_CEIL, np.ceil),
                                     (O.ROUND_TRUNC, np.trunc),
                                     (O.ROUND_ROUND, lambda v: np.sign(v) * np.floor(np.abs(v) + 0.5))])
def test_round_modes(mode, fn):
    L = O.lib()
    v = np.concatenate([np.arange(-40, 41) / 4.0, rng0.uniform(-300, 300, 500)]).astype(np.float32)
    got = np.array([L.oq_round_to_int(float(x), mode) for x in v])
    assert (got == fn(v.astype(np.float64)).astype(np.int64)).all()
    assert L.oq_round_to_int(float("nan"), mode) == 0


# --------------------------------------------------------------------------- MX / fp8 codecs
E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]  # OCP MX v1.0 table of E2M1 magnitudes


def test_e2m1_decode_table():
    L = O.lib()
    for c in range(16):
        v = E2M1[c & 7] * (-1 if c & 8 else 1)
        assert L.oq_e2m1_decode(c) == v


def test_e2m1_encode_nearest_even():
    L = O.lib()
    pos = [(E2M1[c], c) for c in range(8)]
    xs = np.concatenate([rng0.uniform(-8, 8, 4000), [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0, -0.25, -5.0]])
    for x in xs:
        a = abs(float(x))
        best = min(pos, key=lambda p: (abs(p[0] - a), p[1] & 1))[1]
        exp = best | (8 if x < 0 else 0)
        got = L.oq_e2m1_encode_rne(float(x))
        assert got == exp or (best == 0 and got & 7 == 0), (x, got, exp)


def test_e8m0_and_shared_exp():
    L = O.lib()
    for e in range(255):
        assert L.oq_e8m0_decode(e) == np.float32(2.0 ** (e - 127))
    assert math.isnan(L.oq_e8m0_decode(255))
    for a in list(rng0.uniform(1e-6, 1e6, 500)) + [1.0, 4.0, 0.75, 6.0, 6.01]:
        assert L.oq_mx_shared_exp(float(np.float32(a))) == math.floor(math.log2(float(np.float32(a)))) - 2 + 127


@pytest.mark.parametrize("fmt,tdt", [(O.FP8_E4M3, torch.float8_e4m3fn), (O.FP8_E5M2, torch.float8_e5m2)])
def test_fp8_decode_matches_torch(fmt, tdt):
    L = O.lib()
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    exp = codes.view(tdt).to(torch.float32).numpy()
    got = np.array([L.oq_fp8_decode(int(c), fmt) for c in range(256)], np.float32)
    nan = np.isnan(exp)
    assert np.isnan(got[nan]).all() and (got[~nan] == exp[~nan]).all()


# --------------------------------------------------------------------------- ops vs golden fixtures
def test_deqf16_seed9_golden_exact():
    f = np.load(GOLD / "deqf16_seed9.npz")
    acc = O.matmul_i8(f["x1"], f["x2"])
    out = O.mm_dequant(acc, O.F16, qscalar=int(f["quant_word"][0]))
    assert (out == f["golden"].view(np.uint16)).all()


def test_matmul_quant_vector_golden_within_reference_tolerance():
    f = np.load(GOLD / "matmul_quant_vector.npz")
    acc = O.matmul_i8(f["x1"], f["x2"], f["bias"])
    out = O.mm_dequant(acc, O.F16, qvec=f["quant_words"]).view(np.float16)
    g = f["golden"]
    assert ref_verify(out, g)
    # the golden rounds acc to f16 before the multiply; the fixpipe multiplies the exact acc: identical
    # whenever acc is exactly representable in f16
    small = np.abs(acc) <= 2048
    assert (out[small] == g[small]).all()


def test_quant_example_golden_exact():
    f = np.load(GOLD / "quant_example.npz")
    q = O.quant_legacy_f16(f["src"].view(np.uint16), O.F16, scale_scalar=0x4000,
                           offset_scalar=int(np.float16(0.9).view(np.uint16)))
    assert (q == f["golden"]).all()


def test_dequant_example_golden_exact():
    f = np.load(GOLD / "dequant_example.npz")
    y = O.dequant_legacy(f["inp"], O.INT32, f["scale"], O.F32, dst_type=O.F32, cal_count=32)
    assert (y.view(np.uint32) == f["golden"].view(np.uint32)).all()


# --------------------------------------------------------------------------- AscendDequant layout contract
def _rna_exact(v: int) -> int:
    """nearest binary32 value to the integer v, ties away from zero (exact integer arithmetic)"""
    a = abs(v)
    if a < (1 << 24):
        return v
    s = a.bit_length() - 24
    lo = (a >> s) << s
    rem = a - lo
    r = lo + (1 << s) if 2 * rem >= (1 << s) else lo
    return -r if v < 0 else r


def test_i32_to_f32_ties_away():
    """MrgZRndA = CAST_ROUND (half away from zero): 2^24 + 1 -> 2^24 + 2 (nearest-even would give 2^24),
    2^24 + 5 -> 2^24 + 6 (nearest-even: 2^24 + 4); non-ties round to nearest; INT_MIN / INT_MAX -> -+2^31"""
    L = O.lib()
    kat = {(1 << 24) + 1: (1 << 24) + 2, -((1 << 24) + 1): -((1 << 24) + 2), (1 << 24) + 5: (1 << 24) + 6,
           (1 << 24) + 3: (1 << 24) + 4, (1 << 25) + 2: (1 << 25) + 4, (1 << 25) + 1: 1 << 25,
           2 ** 31 - 1: 2 ** 31, -(2 ** 31): -(2 ** 31), (1 << 24) - 1: (1 << 24) - 1, 0: 0, 7: 7, -5: -5}
    for v, want in kat.items():
        assert int(L.oq_i32_to_f32_rna(v)) == want, v
    vals = np.concatenate([rng0.integers(-(2 ** 31), 2 ** 31, 20000, dtype=np.int64),
                           ((rng0.integers(1 << 24, 2 ** 31 - 512, 5000, dtype=np.int64) >> 3) << 3) | 4,
                           ((rng0.integers(1 << 24, 1 << 25, 2000, dtype=np.int64) >> 1) << 1) | 1])
    for v in vals.tolist():
        assert int(L.oq_i32_to_f32_rna(int(v))) == _rna_exact(int(v)), v


def _f16_sat(v32):
    return np.clip(v32, -65504, 65504).astype(np.float16).view(np.uint16)


def _bf16_sat(v32):
    big = float(torch.finfo(torch.bfloat16).max)
    t = torch.from_numpy(np.clip(v32, -big, big).astype(np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def _cast(v32, dst_type):
    return {O.F16: _f16_sat, O.BF16: _bf16_sat, O.F32: lambda v: v.astype(np.float32)}[dst_type](v32)


@pytest.mark.parametrize("dst_type", [O.F16, O.BF16, O.F32])
def test_dequant_single_row_worked_examples(dst_type):
    """UpdateDequantParams' own examples (ascend_dequant_common_impl.h:214-216): int32 {1, 16, 8} is processed as
    {2, 8, 8} for an f32 dst (8 fp32 fill a 32-byte block) but stays {1, 16, 8} for a bf16 dst, so only 8 of the
    16 elements are dequantised; MULTI_ROW never reshapes."""
    src = np.arange(-7, 9, dtype=np.int32) * 3
    scale = np.linspace(0.5, 4.0, 8).astype(np.float32)
    sentinel = 0x7777 if dst_type != O.F32 else np.float32(-1.25)
    for mode in (O.SINGLE_ROW, O.MULTI_ROW):
        init = np.full((2, 16), sentinel, np.float32 if dst_type == O.F32 else np.uint16)
        rows, cols, ldd = O.dequant_legacy_shape(dst_type, 1, 16, 8, mode)
        out = O.dequant_legacy(src, O.INT32, scale, O.F32, dst_type=dst_type, cal_count=8, mode=mode, m=1, n=16,
                               dst=init)
        flat = out.reshape(-1)
        exp = _cast(src[:8].astype(np.float32) * scale, dst_type)
        assert (flat[:8] == exp).all()
        reshaped = mode == O.SINGLE_ROW and dst_type == O.F32
        assert (rows, cols, ldd) == ((2, 8, 8) if reshaped else (1, 16, 16))
        if reshaped:
            assert (flat[8:16] == _cast(src[8:].astype(np.float32) * scale, dst_type)).all()
        else:
            assert (flat[8:] == init.reshape(-1)[8:]).all()


@pytest.mark.parametrize("n,cal", [(8, 8), (24, 24), (40, 40), (24, 16), (40, 8)])
@pytest.mark.parametrize("dst_type", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("per_tensor", [False, True])
def test_dequant_padded_dst_rows(n, cal, dst_type, per_tensor):
    """dst rows start every ceil(n / block) * block elements (dstInner, ascend_dequant_3510_impl.h:44, 99), block =
    32 bytes of dst; columns >= calCount and the padding stay unwritten; with m = 1 the SINGLE_ROW rule may first
    reshape {1, n, cal} into {n / cal, cal, cal}"""
    rng = np.random.default_rng(n * 131 + cal)
    for m in (1, 3):
        src = rng.integers(-(1 << 20), 1 << 20, (m, n), dtype=np.int32)
        scale = rng.uniform(-3, 3, n).astype(np.float32)
        ss = np.float32(0.0371)
        blk = 8 if dst_type == O.F32 else 16
        mm, nn = m, n
        if m == 1 and cal % blk == 0 and n % cal == 0:
            mm, nn = n // cal, cal
        ldd = -(-nn // blk) * blk
        init = np.full((mm, ldd), 0x5555 if dst_type != O.F32 else np.float32(3.5),
                       np.float32 if dst_type == O.F32 else np.uint16)
        out = O.dequant_legacy(src, O.INT32, scale, O.F32, per_tensor=per_tensor, dst_type=dst_type, cal_count=cal,
                               scale_scalar=ss, dst=init.copy())
        assert out.shape == (mm, ldd)
        s2 = src.reshape(mm, nn)
        sc = ss if per_tensor else scale[:cal]
        exp = _cast(s2[:, :cal].astype(np.float32) * sc, dst_type)
        assert (out[:, :cal] == exp).all()
        assert (out[:, cal:] == init[:, cal:]).all()


@pytest.mark.parametrize("src_type", [O.INT32, O.F32])
@pytest.mark.parametrize("scale_type", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("k_dim", [0, 1])
def test_dequant_policy_per_group_axes(src_type, scale_type, k_dim):
    """PER_GROUP: kDim 1 scales [rows][ceil(n/g)] along each row, kDim 0 scales [ceil(rows/g)][n] down the columns
    (ascend_dequant_3510_impl.h:367-598); checked against numpy's repeat of the scale table, with ragged row and
    column counts (tail groups)"""
    rng = np.random.default_rng(7 + k_dim + 3 * scale_type + 11 * src_type)
    rows, n, g = 70, 200, 64
    if src_type == O.INT32:
        src = rng.integers(-(1 << 23), 1 << 23, (rows, n), dtype=np.int32)
        s32 = src.astype(np.float32)
    else:
        src = (rng.standard_normal((rows, n)) * 1000).astype(np.float32)
        s32 = src
    shape = (rows, -(-n // g)) if k_dim == 1 else (-(-rows // g), n)
    sf = rng.uniform(-2, 2, shape).astype(np.float32)
    if scale_type == O.F16:
        sf = sf.astype(np.float16)
        sw, sv = sf, sf.astype(np.float32)
    elif scale_type == O.BF16:
        bt = torch.from_numpy(sf).to(torch.bfloat16)
        sw, sv = bt.view(torch.int16).numpy().view(np.uint16), bt.float().numpy()
    else:
        sw, sv = sf, sf
    full = np.repeat(sv, g, axis=1)[:, :n] if k_dim == 1 else np.repeat(sv, g, axis=0)[:rows]
    for dst_type in (O.F16, O.BF16, O.F32):
        out = O.dequant_policy(src, src_type, sw, scale_type, O.PER_GROUP, dst_type, k_dim=k_dim, group=g)
        assert (out == _cast(s32 * full, dst_type)).all()


def test_dequant_policy_per_token_and_cal_count():
    """PER_TOKEN: scale[r] along row r; rows = calCount / n (a partial last row is not processed)"""
    rng = np.random.default_rng(99)
    src = rng.integers(-(1 << 22), 1 << 22, (9, 48), dtype=np.int32)
    sc = rng.uniform(0.001, 0.1, 9).astype(np.float32)
    init = np.full((9, 48), 0x4242, np.uint16)
    out = O.dequant_policy(src, O.INT32, sc, O.F32, O.PER_TOKEN, O.F16, cal_count=8 * 48 + 5, dst=init.copy())
    assert (out[:8] == _f16_sat(src[:8].astype(np.float32) * sc[:8, None])).all()
    assert (out[8] == init[8]).all()


def test_dequant_int32_sources_round_ties_away():
    """large int32 accumulators convert with ties away before the multiply (scale 1 keeps the conversion visible)"""
    src = np.array([[(1 << 24) + 1, (1 << 24) + 5, -((1 << 24) + 1), (1 << 25) + 2] * 2], np.int32)
    want = np.array([_rna_exact(int(v)) for v in src[0]], np.float32)
    one = np.ones(8, np.float32)
    y = O.dequant_legacy(src, O.INT32, one, O.F32, dst_type=O.F32, cal_count=8)
    assert (y[0] == want).all()
    yp = O.dequant_policy(src, O.INT32, np.ones(1, np.float32), O.F32, O.PER_TOKEN, O.F32)
    assert (yp[0] == want).all()


@pytest.mark.parametrize("arch,arith", [("2201", O.ARITH_F16), ("3510", O.ARITH_F32)])
def test_antiquant_seed10_golden_exact(arch, arith):
    f = np.load(GOLD / "antiquant_seed10.npz")
    y = O.antiquant(f["src"], O.INT8, f["scale"].view(np.uint16), f["offset"].view(np.uint16), 8, 128, 8, False,
                    O.F16, arith)
    assert (y == f[f"golden_{arch}"].view(np.uint16)).all()


def test_group_matmul_golden_within_reference_tolerance():
    f = np.load(GOLD / "group_matmul_example.npz")
    G, (m, k), n = 4, f["x"].shape, f["weight"].shape[2]
    y = O.group_matmul(f["x"], f["pts"], f["weight"], f["scale"], f["group_list"], 1, G, m, k, n, O.F16)
    # verify_result.py of that example: rtol = atol = 1e-3, error ratio <= 1e-4
    assert ref_verify(y.view(np.float16), f["golden"], err_tol=1e-4)


def test_mx_example_golden_exact():
    f = np.load(GOLD / "mx_example.npz")
    M = N = K = 256
    Bt = np.ascontiguousarray(f["b_packed"])
    C, Ce, _ = O.mx_matmul(f["a_packed"], Bt, f["scale_a"], f["scale_b_pairs"], M, N, K, trans_b=False,
                           sa_layout=0, sb_layout=0)
    assert (C == f["golden_bf16"]).all()


# --------------------------------------------------------------------------- ops vs independent numpy / exact
def test_matmul_i8_vs_numpy():
    A = rng0.integers(-128, 128, (37, 300), dtype=np.int8)
    B = rng0.integers(-128, 128, (300, 45), dtype=np.int8)
    bias = rng0.integers(-(2 ** 31), 2 ** 31 - 1, 45, dtype=np.int64).astype(np.int32)
    exp = (A.astype(np.int64) @ B.astype(np.int64) + bias).astype(np.int64)
    exp = ((exp + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)  # two's-complement wrap
    assert (O.matmul_i8(A, B, bias) == exp).all()
    assert (O.matmul_i8(A, np.ascontiguousarray(B.T), bias, trans_b=True) == exp).all()
    assert (O.matmul_i8(np.ascontiguousarray(A.T), B, bias, trans_a=True) == exp).all()


def test_mm_dequant_vs_numpy_f32():
    acc = rng0.integers(-(2 ** 26), 2 ** 26, (64, 48)).astype(np.int32)
    s = (np.exp(rng0.uniform(-20, 5, 48)) * np.where(rng0.random(48) < 0.2, -1, 1)).astype(np.float32)
    words = s.view(np.uint32).astype(np.uint64)
    m1 = (s.view(np.uint32) & np.uint32(0xFFFFE000)).view(np.float32)
    exp16 = np.clip(acc.astype(np.float32) * m1, -65504, 65504).astype(np.float16).view(np.uint16)
    assert (O.mm_dequant(acc, O.F16, qvec=words) == exp16).all()
    expb = torch.from_numpy(acc.astype(np.float32) * m1).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (O.mm_dequant(acc, O.BF16, qvec=words) == expb).all()


def test_quant_per_token_vs_numpy():
    x = (rng0.standard_normal((20, 300)) * 30).astype(np.float32)
    s = rng0.uniform(0.1, 3, 20).astype(np.float32)
    o = rng0.uniform(-4, 4, 20).astype(np.float32)
    v = x * s[:, None] + o[:, None]
    exp = np.clip(np.rint(v), -128, 127).astype(np.int8)
    assert (O.quant_per_token(x, O.F32, s, o) == exp).all()
    exp_floor = np.clip(np.floor(x * s[:, None]), -128, 127).astype(np.int8)
    assert (O.quant_per_token(x, O.F32, s, None, O.ROUND_FLOOR) == exp_floor).all()


def test_dynamic_quant_invariants_and_numpy():
    x = rng0.standard_normal((50, 1024)).astype(np.float32)
    x[rng0.random(x.shape) < 0.001] *= 50
    x16 = x.astype(np.float16)
    q, s = O.quant_dynamic_per_token(x16.view(np.uint16), O.F16)
    xf = x16.astype(np.float32)
    amax = np.abs(xf).max(1)
    mult = np.float32(127.0) / amax
    assert (q == np.clip(np.rint(xf * mult[:, None]), -128, 127).astype(np.int8)).all()
    assert (s == (amax / np.float32(127.0)).astype(np.float32)).all()
    assert np.abs(q.astype(np.int32)).max() <= 127
    # the row maximum maps to +-127 exactly
    rows = np.arange(50)
    assert (np.abs(q[rows, np.abs(xf).argmax(1)]) == 127).all()


def test_dynamic_quant_exhaustive_half_rows():
    """Each row holds every non-negative binary16 value up to its absmax, so all rounding boundaries of
    x * (127 / absmax) are visited; the multiplier is one fp32 division (not 1 / (absmax / 127))."""
    codes = np.arange(0, 0x7C00, dtype=np.uint16)
    allh = codes.view(np.float16).astype(np.float32)
    amaxes = [0.50048828125, 0.83203125, 1.1376953125, 1.5166015625, 1.990234375, 2.169921875, 13.140625]
    n = int((allh <= max(amaxes)).sum())
    x = np.zeros((len(amaxes), n), np.float16)
    for i, a in enumerate(amaxes):
        v = allh[allh <= a].astype(np.float16)
        x[i, :v.size] = v
        x[i, v.size:] = -v[: n - v.size] if v.size else 0
    q, s = O.quant_dynamic_per_token(x.view(np.uint16), O.F16)
    xf = x.astype(np.float32)
    mult = (np.float32(127.0) / np.abs(xf).max(1)).astype(np.float32)
    assert (q == np.clip(np.rint(xf * mult[:, None]), -128, 127).astype(np.int8)).all()


def _half_round_exact(fr: Fraction) -> np.float16:
    """round an exact rational to binary16 (nearest, ties to even) by brute force over neighbouring codes"""
    f = float(fr)
    h = np.float16(f)
    cands = [h, np.nextafter(h, np.float16(np.inf)), np.nextafter(h, np.float16(-np.inf))]
    return min(cands, key=lambda c: (abs(Fraction(float(c)) - fr), int(c.view(np.uint16)) & 1))


def test_legacy_quant_half_ops_exact_rationals():
    x = rng0.uniform(-8, 8, 600).astype(np.float16)
    sc = rng0.uniform(0.01, 30, 8).astype(np.float16)
    of = (rng0.uniform(-3, 3, 8) * 10.0 ** rng0.integers(-6, 1, 8)).astype(np.float16)
    q = O.quant_legacy_f16(x.view(np.uint16), O.F16, scale_vec=sc.view(np.uint16), offset_vec=of.view(np.uint16),
                           scale_count=8)
    for i in range(600):
        t = _half_round_exact(Fraction(float(x[i])) * Fraction(float(sc[i % 8])))
        t = _half_round_exact(Fraction(float(t)) + Fraction(float(of[i % 8])))
        exp = int(np.clip(np.rint(np.float64(t)), -128, 127))
        assert q[i] == exp


def test_antiquant_f16_ops_exact_rationals_int4_groups():
    K, N, g = 64, 6, 32
    nib = rng0.integers(0, 16, K * N, dtype=np.uint8)
    packed = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    qv = np.where(nib >= 8, nib.astype(np.int32) - 16, nib.astype(np.int32)).reshape(K, N)
    sc = np.exp(rng0.uniform(-7, -2, (K // g, N))).astype(np.float16)
    of = (rng0.uniform(-8, 8, (K // g, N)) * 10.0 ** rng0.integers(-5, 1, (K // g, N))).astype(np.float16)
    y = O.antiquant(packed, O.INT4, sc.view(np.uint16), of.view(np.uint16), K, N, g).view(np.float16)
    for k in range(K):
        for n in range(N):
            t = _half_round_exact(Fraction(int(qv[k, n])) + Fraction(float(of[k // g, n])))
            t = _half_round_exact(Fraction(float(t)) * Fraction(float(sc[k // g, n])))
            assert y[k, n] == t


def test_antiquant_matmul_vs_numpy():
    M, K, N, g = 3, 256, 32, 128
    w = rng0.integers(-128, 128, (K, N), dtype=np.int8)
    sc = np.exp(rng0.uniform(np.log(1e-3), np.log(1e-1), (K // g, N))).astype(np.float16)
    of = rng0.uniform(-8, 8, (K // g, N)).astype(np.float16)
    x = rng0.standard_normal((M, K)).astype(np.float16)
    y, ye, ya = O.antiquant_matmul(x.view(np.uint16), w, O.INT8, sc.view(np.uint16), of.view(np.uint16), g, M, N, K)
    wf = O.antiquant(w, O.INT8, sc.view(np.uint16), of.view(np.uint16), K, N, g).view(np.float16)
    exact = x.astype(np.float64) @ wf.astype(np.float64)
    assert np.allclose(ye, exact, rtol=1e-12, atol=1e-12)
    assert (y.view(np.float16) == ye.astype(np.float16)).all()
    assert np.allclose(ya, np.abs(x.astype(np.float64)) @ np.abs(wf.astype(np.float64)), rtol=1e-12)


def test_group_matmul_vs_numpy_exact():
    G, K, N = 3, 200, 40
    counts = np.array([5, 0, 11], np.int64)
    M = 20
    x = rng0.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng0.integers(-127, 128, (G, K, N), dtype=np.int8)
    pts = rng0.uniform(1e-3, 1e-1, M).astype(np.float32)
    sc = rng0.uniform(1e-4, 1e-2, (G, N)).astype(np.float32)
    y = O.group_matmul(x, pts, w, sc, counts, 1, G, M, K, N, O.BF16)
    off = np.concatenate([[0], np.cumsum(counts)])
    for g in range(G):
        s, e = off[g], off[g + 1]
        acc = (x[s:e].astype(np.int64) @ w[g].astype(np.int64)).astype(np.float32)
        v = (acc * sc[g]) * pts[s:e, None]
        exp = torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert (y[s:e] == exp).all()
    assert (y[16:] == 0).all()


def test_group_matmul_f32_epilogue_order():
    """fp32 output exposes the epilogue's rounding order: (acc * scale[g, n]) first, then * pts[m]
    (quant_group_matmul_custom.asc's dequant of the int32 tile, then the per-token multiply)."""
    G, K, N, M = 2, 64, 48, 24
    counts = np.array([10, 14], np.int64)
    x = rng0.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng0.integers(-127, 128, (G, K, N), dtype=np.int8)
    pts = rng0.uniform(1e-3, 1e-1, M).astype(np.float32)
    sc = rng0.uniform(1e-4, 1e-2, (G, N)).astype(np.float32)
    y = O.group_matmul(x, pts, w, sc, counts, 1, G, M, K, N, O.F32, y=np.zeros((M, N), np.float32))
    off = np.concatenate([[0], np.cumsum(counts)])
    for g in range(G):
        s, e = off[g], off[g + 1]
        acc = (x[s:e].astype(np.int64) @ w[g].astype(np.int64)).astype(np.float32)
        first = (acc * sc[g][None, :]).astype(np.float32)
        exp = (first * pts[s:e, None]).astype(np.float32)
        assert np.array_equal(y[s:e], exp)
        other = ((acc * pts[s:e, None]).astype(np.float32) * sc[g][None, :]).astype(np.float32)
        assert not np.array_equal(other, exp)  # the two orders differ on these inputs


def test_group_matmul_ties_above_2_24_round_away():
    """Accumulators on fp32 ties in [2^24, 2^26): the group epilogue's AscendDequant converts int32 -> fp32 with ties
    away from zero (ascend_dequant_3510_impl.h:61), checked against the numpy restatement of group_cases.py; the
    nearest-even conversion changes more than 50 of these bf16 outputs."""
    import group_cases as GC

    x, w, pts, sc, counts = GC.tie_case(7)
    M, K = x.shape
    G, _, N = w.shape
    y = O.group_matmul(x, pts, w, sc, counts, 1, G, M, K, N, O.BF16)
    assert np.array_equal(y, GC.group_reference(x, w, pts, sc, counts))
    assert GC.rne_differs(x, w, pts, sc, counts) > 50


def test_mx_matmul_vs_numpy_decode():
    M, N, K = 8, 12, 128
    A = rng0.integers(0, 256, (M, K // 2), dtype=np.uint8)
    Bt = rng0.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sA = rng0.integers(110, 140, (M, K // 32), dtype=np.uint8)
    sB = rng0.integers(110, 140, (N, K // 32), dtype=np.uint8)
    table = np.array([E2M1[c & 7] * (-1 if c & 8 else 1) for c in range(16)])

    def dec(p, s):
        v = table[np.stack([p & 0xF, p >> 4], -1).reshape(p.shape[0], -1)]
        return v * 2.0 ** (np.repeat(s.astype(np.float64), 32, axis=1) - 127)

    exact = dec(A, sA) @ dec(Bt, sB).T
    _, Ce, _ = O.mx_matmul(A, Bt, sA, sB, M, N, K, trans_b=True, sa_layout=0, sb_layout=1)
    assert np.allclose(Ce, exact, rtol=1e-13, atol=1e-13)


def test_mx_quantize_fp4_roundtrip():
    x = rng0.standard_normal((16, 256)).astype(np.float32)
    p, s = O.mx_quantize_fp4(x)
    table = np.array([E2M1[c & 7] * (-1 if c & 8 else 1) for c in range(16)])
    v = table[np.stack([p & 0xF, p >> 4], -1).reshape(16, 256)] * 2.0 ** (np.repeat(s, 32, 1).astype(np.float64) - 127)
    # the shared exponent puts every block max at 4 <= |x| / scale < 8; E2M1 spacing is at most 2 (between 4
    # and 6), so an element inside the E2M1 range is off by at most one scale unit, and one clamped from
    # [6, 8) to 6 by less than two
    scale = 2.0 ** (np.repeat(s, 32, 1).astype(np.float64) - 127)
    blk = np.abs(x.reshape(16, 8, 32)).max(-1) / 2.0 ** (s.astype(np.float64) - 127)
    assert ((blk >= 4) & (blk < 8)).all()
    err = np.abs(v - x)
    inside = np.abs(x) / scale <= 6
    assert (err[inside] <= scale[inside]).all()
    assert (err < 2 * scale).all()


# --------------------------------------------------------------------------- fp8 operand Matmul / MX-FP8
_T8 = {O.FP8_E4M3: torch.float8_e4m3fn, O.FP8_E5M2: torch.float8_e5m2}


def fp8_bytes(rng, shape, fmt, lo=0, hi=256):
    """random fp8 codes without NaN / inf (e4m3fn: S.1111.111 is NaN; e5m2: exponent 31 is inf / NaN)"""
    c = rng.integers(lo, hi, shape, dtype=np.int64).astype(np.uint8)
    bad = (c & 0x7F) == 0x7F if fmt == O.FP8_E4M3 else (c & 0x7C) == 0x7C
    return np.where(bad, c & 0x80, c).astype(np.uint8)


def torch_decode(codes, fmt):
    return torch.from_numpy(np.ascontiguousarray(codes)).view(_T8[fmt]).to(torch.float64).numpy()


@pytest.mark.parametrize("fa,fb", [(O.FP8_E4M3, O.FP8_E4M3), (O.FP8_E5M2, O.FP8_E5M2), (O.FP8_E4M3, O.FP8_E5M2),
                                   (O.FP8_E5M2, O.FP8_E4M3)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, True), (False, True)])
def test_matmul_fp8_vs_torch_decode(fa, fb, ta, tb):
    """exact sum vs torch's float8 decode and a float64 matmul; bias enters once, in the fp64 sum"""
    M, N, K = 9, 13, 70
    rng = np.random.default_rng(801)
    A = fp8_bytes(rng, (K, M) if ta else (M, K), fa)
    B = fp8_bytes(rng, (N, K) if tb else (K, N), fb)
    bias = rng.standard_normal(N).astype(np.float32)
    _, exact, absd, bmax = O.matmul_fp8(A, B, fa, fb, bias=bias, trans_a=ta, trans_b=tb)
    a = torch_decode(A, fa)
    b = torch_decode(B, fb)
    a = a.T if ta else a
    b = b.T if tb else b
    ref = a @ b
    assert np.allclose(exact, ref + bias.astype(np.float64), rtol=0, atol=1e-12 * np.abs(a) @ np.abs(b) + 1e-30)
    assert np.allclose(absd, np.abs(a) @ np.abs(b), rtol=1e-13, atol=0)
    P = np.abs(a[:, :, None] * b[None, :, :])  # [M, K, N]
    ref_bmax = sum(P[:, h:h + 16, :].max(1) for h in range(0, K, 16))  # K = 70: groups of 16 x 4, 6
    assert np.allclose(bmax, ref_bmax, rtol=1e-15, atol=0)


@pytest.mark.parametrize("out_type,tdt", [(O.F16, torch.float16), (O.BF16, torch.bfloat16), (O.F32, torch.float32)])
def test_matmul_fp8_epilogue_vs_torch(out_type, tdt):
    """QF322{F16,BF16,F32}_PRE: fp32(acc + bias) * M1 (M1 = the word's bits 13..31) then torch's rne cast;
    without a quant word the plain cast; per-channel words pick column n"""
    M, N, K = 6, 20, 64
    rng = np.random.default_rng(802)
    A = fp8_bytes(rng, (M, K), O.FP8_E4M3, 0, 120)
    B = fp8_bytes(rng, (K, N), O.FP8_E4M3, 0, 120)
    bias = rng.standard_normal(N).astype(np.float32)
    words = np.array([O.lib().oq_pack_quant_pre(float(v), 0, 0) | 0x1FFF for v in rng.uniform(0.01, 2.0, N)],
                     np.uint64)
    m1 = (words.astype(np.uint64) & np.uint64(0xFFFFE000)).astype(np.uint32).view(np.float32)

    def as_f64(out):
        if out_type == O.F32:
            return out.astype(np.float64)
        return torch.from_numpy(out.view(np.int16)).view(tdt).to(torch.float64).numpy()

    for use_q, qvec in [(False, None), (True, words)]:
        out, exact, _, _ = O.matmul_fp8(A, B, O.FP8_E4M3, O.FP8_E4M3, bias=bias, out_type=out_type, use_q=use_q,
                                     qvec=qvec)
        v = exact.astype(np.float32)
        if use_q:
            v = (v * m1[None, :]).astype(np.float32)
        exp = torch.from_numpy(v).to(tdt).to(torch.float64).numpy()
        if out_type == O.F16:
            exp = np.clip(exp, -65504.0, 65504.0)  # the fixpipe cast saturates
        assert np.array_equal(as_f64(out), exp)
    # scalar word: column-independent M1
    out, exact, _, _ = O.matmul_fp8(A, B, O.FP8_E4M3, O.FP8_E4M3, out_type=O.F32, use_q=True, qscalar=int(words[3]))
    assert np.array_equal(out, (exact.astype(np.float32) * m1[3]).astype(np.float32))


@pytest.mark.parametrize("fa,fb", [(O.FP8_E4M3, O.FP8_E4M3), (O.FP8_E5M2, O.FP8_E4M3)])
def test_mx_matmul_fp8_vs_torch_decode(fa, fb):
    """MX-FP8: elements decoded by torch, scales 2^(e-127) per 32 K, both scale layouts of the sample"""
    M, N, K = 5, 7, 128
    rng = np.random.default_rng(803)
    A = fp8_bytes(rng, (M, K), fa)
    B = fp8_bytes(rng, (K, N), fb)
    sK = K // 32
    sA = rng.integers(115, 135, (M, sK), dtype=np.uint8)
    sB = rng.integers(115, 135, (N, sK), dtype=np.uint8)
    a = torch_decode(A, fa) * 2.0 ** (np.repeat(sA.astype(np.float64), 32, 1) - 127)
    b = torch_decode(B, fb) * 2.0 ** (np.repeat(sB.astype(np.float64), 32, 1).T - 127)
    sB_pairs = np.ascontiguousarray(sB.T.reshape(sK // 2, 2, N).transpose(0, 2, 1))  # [sK/2, N, 2]
    _, Ce, Ca, Cb = O.mx_matmul(A, B, sA, sB_pairs, M, N, K, trans_b=False, sa_layout=0, sb_layout=0, elem_fmt=fa,
                                fmt_b=fb, blockmax=True)
    assert np.allclose(Ce, a @ b, rtol=0, atol=1e-12 * (np.abs(a) @ np.abs(b)))
    assert np.allclose(Ca, np.abs(a) @ np.abs(b), rtol=1e-13, atol=0)
    P = np.abs(a[:, :, None] * b[None, :, :])
    assert np.allclose(Cb, sum(P[:, h:h + 16, :].max(1) for h in range(0, K, 16)), rtol=1e-15, atol=0)


# --------------------------------------------------------------------------- requant epilogues (REQ8 / QF322B8 / QF322FP8)
def _word(m1, offset=0, sign=1):
    return int(O.lib().oq_pack_quant_pre(float(m1), int(offset), int(sign)))


def test_req8_seed9_golden_exact():
    """(V)REQ8 golden of asc_copy_l0c2gm (gen_data_s322s8.py, seed 9): scalar and per-channel forms"""
    f = np.load(GOLD / "req8_seed9.npz")
    acc = O.matmul_i8(f["x1"], f["x2"])
    w = int(f["quant_word"][0])
    assert np.array_equal(O.mm_requant(acc, qscalar=w).view(np.int8), f["golden"])
    qv = np.full(acc.shape[1], w, np.uint64)
    assert np.array_equal(O.mm_requant(acc, qvec=qv).view(np.int8), f["golden"])


def test_qf322b8_seed9_golden_exact():
    """(V)QF322B8_PRE golden of asc_copy_l0c2gm scenario 4 / 5 (gen_data.py, seed 9), on its fp32 accumulators"""
    f = np.load(GOLD / "qf322b8_seed9.npz")
    w = int(f["quant_word"][0])
    L = O.lib()
    acc = f["acc_f32"]
    m1 = float(np.uint32(w & 0xFFFFE000).view(np.float32))
    got = np.array([L.oq_requant8(float(np.float32(v) * np.float32(m1)), w) for v in acc.ravel()], np.uint8)
    assert np.array_equal(got.view(np.int8).reshape(acc.shape), f["golden"])


def test_prequant_doc_example():
    """asc_set_l0c_copy_prequant.md example: identity x identity, scale 2, offset 3, signed -> 5 on the
    diagonal, 3 elsewhere (the offset is added after the multiply, zeros included)"""
    L = O.lib()
    w = _word(2.0, 3, 1)
    acc = np.eye(16, dtype=np.float32)
    got = np.array([[L.oq_requant8(float(v * 2.0), w) for v in row] for row in acc], np.uint8).view(np.int8)
    exp = np.full((16, 16), 3, np.int8)
    np.fill_diagonal(exp, 5)
    assert np.array_equal(got, exp)
    # the fp8 Matmul path with the same word: e4m3 identity (0x38 = 1.0)
    A = np.zeros((16, 16), np.uint8)
    np.fill_diagonal(A, 0x38)
    out, _, _, _ = O.matmul_fp8(A, A, O.FP8_E4M3, O.FP8_E4M3, out_type=O.INT8, use_q=True, qscalar=w)
    assert np.array_equal(out.view(np.int8), exp)


def test_requant8_boundaries_and_offsets():
    """closed form over random values, offsets 0..511 and both sign flags; NaN -> 0, +-inf saturate
    (matrix_compute_move_out_interface_boundary_value_summary.md:74-79, 106-109)"""
    L = O.lib()
    rng = np.random.default_rng(804)
    v = np.concatenate([rng.uniform(-700, 700, 3000), np.arange(-260, 260) + 0.5, [255.4, 255.5, -256.5]])
    v = v.astype(np.float32)
    for _ in range(6):
        off, sign = int(rng.integers(0, 512)), int(rng.integers(0, 2))
        w = _word(1.0, off, sign) | (0x1F << 32)  # bits 32-36 (shift, MCB) are ignored
        got = np.array([L.oq_requant8(float(x), w) for x in v], np.uint8)
        t = np.round(np.clip(v.astype(np.float64), -256, 255)) + off
        exp = np.clip(t, -128, 127).astype(np.int8).view(np.uint8) if sign else np.clip(t, 0, 255).astype(np.uint8)
        assert np.array_equal(got, exp), (off, sign)
    ws, wu = _word(1.0, 0, 1), _word(1.0, 0, 0)
    assert L.oq_requant8(float("nan"), ws) == 0 and L.oq_requant8(float("nan"), wu) == 0
    assert L.oq_requant8(float("inf"), ws) == 127 and L.oq_requant8(float("-inf"), ws) == 0x80
    assert L.oq_requant8(float("inf"), wu) == 255 and L.oq_requant8(float("-inf"), wu) == 0


def test_requant4_saturation_offset_and_packing():
    """(V)REQ4 / QF322S4_PRE: saturation to 7 / -8 (matrix_compute_move_out_interface_boundary_value_summary.md:
    110-111), the 9-bit offset applies after rounding and the sign flag does not (asc_set_l0c_copy_prequant.md:106,
    117); codes packed two per byte with the even column in the low nibble (the int4b_t layout of
    matmul_int4/scripts/gen_data.py: (x[j+1] << 4) + (x[j] & 0xF))"""
    L = O.lib()
    w = _word(1.0, 0, 1)
    nan, inf = float("nan"), float("inf")
    for v, e in [(0.0, 0), (7.4, 7), (7.5, 7), (6.5, 6), (2.5, 2), (-2.5, -2), (-7.5, -8), (-8.5, -8), (-9.0, -8),
                 (1e6, 7), (-1e6, -8), (nan, 0), (inf, 7), (-inf, -8)]:
        assert L.oq_requant4(v, w) == e & 0xF, v
    w3 = _word(1.0, 3, 0)
    assert L.oq_requant4(2.0, w3) == 5 and L.oq_requant4(5.0, w3) == 7 and L.oq_requant4(-12.0, w3) == 0x8
    assert L.oq_requant4(-20.0, _word(1.0, 15, 1)) == (-5 & 0xF) == L.oq_requant4(-20.0, _word(1.0, 15, 0))
    assert L.oq_requant4(-1e6, _word(1.0, 300, 1)) == 7  # clamped to -256 before the offset: 44 -> 7
    assert O.mm_requant4(np.array([[12, -13]], np.int32), qscalar=_word(0.5, 0, 1)).tolist() == [[0xA6]]  # x M1 first
    acc = np.array([[1, -2, 7, -8, 100, -100, 3, 0]], np.int32)
    assert O.mm_requant4(acc, qscalar=w).tolist() == [[0xE1, 0x87, 0x87, 0x03]]
    assert np.array_equal(O.unpack_int4(O.mm_requant4(acc, qscalar=w), 8), [[1, -2, 7, -8, 7, -8, 3, 0]])
    f = np.array([[0.25, -0.75, 6.5, 7.5]], np.float32)  # fp32 path: rint ties to even
    assert O.unpack_int4(O.requant4_f32(f, qscalar=w), 4).tolist() == [[0, -1, 6, 7]]


@pytest.mark.parametrize("fmt", [O.FP8_E4M3, O.FP8_E5M2])
def test_f32_to_fp8_vs_torch(fmt):
    """in-range values (including exact ties between neighbouring codes and subnormals) vs torch's rne cast;
    e4m3 saturates to +-448 with NaN -> 0 (fixpipe default), e5m2 overflows to inf (NaN stays NaN)"""
    L = O.lib()
    tdt = _T8[fmt]
    top = 448.0 if fmt == O.FP8_E4M3 else 57344.0
    rng = np.random.default_rng(805)
    vals = np.exp(rng.uniform(np.log(2.0 ** -20), np.log(top), 4000)) * rng.choice([-1, 1], 4000)
    codes = np.arange(256, dtype=np.uint8)
    dec = torch_decode(codes, fmt)
    fin = np.sort(np.unique(np.abs(dec[np.isfinite(dec)])))
    mids = (fin[1:] + fin[:-1]) / 2  # exact ties
    vals = np.concatenate([vals, mids, -mids, fin, [0.0, -0.0]]).astype(np.float32)
    vals = vals[np.abs(vals) <= top]
    got = np.array([L.oq_f32_to_fp8(float(x), fmt) for x in vals], np.uint8)
    exp = torch.from_numpy(vals).to(tdt).view(torch.uint8).numpy()
    assert np.array_equal(got, exp)
    if fmt == O.FP8_E4M3:
        for x, c in [(449.0, 0x7E), (1e6, 0x7E), (-1e6, 0xFE), (float("inf"), 0x7E), (float("-inf"), 0xFE),
                     (float("nan"), 0x00)]:
            assert L.oq_f32_to_fp8(x, fmt) == c
    else:
        for x, c in [(61439.0, 0x7B), (61440.0, 0x7C), (-1e9, 0xFC), (float("inf"), 0x7C)]:
            assert L.oq_f32_to_fp8(x, fmt) == c
        assert L.oq_f32_to_fp8(float("nan"), fmt) == 0x7F


def test_matmul_fp8_requant_outputs_compose():
    """QF322B8 / QF322FP8 outputs of oq_matmul_fp8 equal requant8 / f32_to_fp8 of fp32((s + bias)) * M1"""
    L = O.lib()
    rng = np.random.default_rng(806)
    M, N, K = 7, 9, 64
    A = fp8_bytes(rng, (M, K), O.FP8_E4M3, 0, 100)
    B = fp8_bytes(rng, (K, N), O.FP8_E5M2, 0, 100)
    bias = rng.standard_normal(N).astype(np.float32)
    words = np.array([_word(x, int(o), int(sg)) for x, o, sg in
                      zip(rng.uniform(0.05, 3.0, N), rng.integers(0, 512, N), rng.integers(0, 2, N))], np.uint64)
    m1 = (words & np.uint64(0xFFFFE000)).astype(np.uint32).view(np.float32)
    for ot in (O.INT8, O.FP8_E4M3, O.FP8_E5M2):
        out, exact, _, _ = O.matmul_fp8(A, B, O.FP8_E4M3, O.FP8_E5M2, bias=bias, out_type=ot, use_q=True, qvec=words)
        v = (exact.astype(np.float32) * m1[None, :]).astype(np.float32)
        if ot == O.INT8:
            exp = np.array([[L.oq_requant8(float(v[i, j]), int(words[j])) for j in range(N)] for i in range(M)])
        else:
            exp = np.array([[L.oq_f32_to_fp8(float(v[i, j]), ot) for j in range(N)] for i in range(M)])
        assert np.array_equal(out.view(np.uint8), exp.astype(np.uint8))


# --------------------------------------------------------------------------- group matmul FasterGelu
def test_faster_gelu_vs_sample_formula():
    """oq_faster_gelu (fp32 ops x / (1 + exp(-1.702 x))) against the sample's algebraically different form
    x * exp(0.851 (x - |x|)) / (1 + exp(-1.702 |x|)) (gen_data.py:19-23) in float64: within the fp32 rounding
    errors of the op sequence, and -0 where the fp32 exp overflows (x below ~-52.1; the float64 form gives a value below 1e-36)"""
    L = O.lib()
    x = np.concatenate([np.linspace(-60, 60, 2001), np.random.default_rng(807).normal(0, 3, 2000),
                        [-1e30, -90.0, -1e-30, 0.0, 1e-30, 90.0, 1e30]]).astype(np.float32)
    c = float(np.float32(1.702))
    xd = x.astype(np.float64)
    ref = xd * np.exp(c / 2 * (xd - np.abs(xd))) / (1 + np.exp(-c * np.abs(xd)))
    got = np.array([L.oq_faster_gelu(float(v)) for v in x], np.float64)
    # the fp32 product -1.702 x carries a relative error 2^-24, which exp turns into |1.702 x| 2^-24 relative
    rtol = (4 + c * np.abs(xd)) * 2.0 ** -24
    assert (np.abs(got - ref) <= rtol * np.abs(ref) + 1e-36).all()
    tail = x < -52.2
    assert (got[tail] == 0).all() and np.signbit(got[tail]).all()


def test_group_matmul_gelu_golden_within_reference_tolerance():
    """the sample's verify_result.py criterion (isclose rtol = atol = 1e-3, error ratio <= 1e-4) against the
    restated golden with FastGelu, and the bare epilogue (act = 0) does not pass it"""
    f = np.load(GOLD / "group_matmul_gelu_example.npz")
    m, k = f["x"].shape
    G, _, n = f["weight"].shape
    y = O.group_matmul(f["x"], f["pts"], f["weight"], f["scale"], f["group_list"], 1, G, m, k, n, O.F16, act=1)
    assert ref_verify(y.view(np.float16), f["golden"], err_tol=1e-4)
    y0 = O.group_matmul(f["x"], f["pts"], f["weight"], f["scale"], f["group_list"], 1, G, m, k, n, O.F16, act=0)
    assert not ref_verify(y0.view(np.float16), f["golden"], err_tol=1e-4)


# --------------------------------------------------------------------------- NZ fractal layout
@pytest.mark.parametrize("G,K,N", [(3, 64, 96), (1, 16, 32)])
def test_nz_to_nd_matches_generator_layout(G, K, N):
    """the group-matmul generator's NZ weights, weight.reshape([G, K/16, 16, N/32, 32]).transpose(0, 3, 1, 2, 4)
    (gen_data.py:62), back to ND [G, K, N] and to K-contiguous [G, N, K]; and ND -> NZ reproduces them"""
    rng = np.random.default_rng(808)
    w = rng.integers(-128, 128, (G, K, N)).astype(np.int8)
    nz = np.ascontiguousarray(w.reshape(G, K // 16, 16, N // 32, 32).transpose(0, 3, 1, 2, 4))
    assert np.array_equal(O.nz_to_nd(nz, 1, G, K, N).view(np.int8), w)
    assert np.array_equal(O.nz_to_nd(nz, 1, G, K, N, transpose_out=True).view(np.int8), w.transpose(0, 2, 1))
    assert np.array_equal(O.nd_to_nz(w, 1, G, K, N), nz.reshape(-1).view(np.uint8))


@pytest.mark.parametrize("dt,esize", [(np.int8, 1), (np.float16, 2), (np.float32, 4)])
def test_nz_padding_and_element_sizes(dt, esize):
    """ragged rows / columns: NZ pads to 16 rows and 32-byte column blocks (zeros), C0 = 32 / element bytes"""
    rng = np.random.default_rng(809)
    B, R, C = 2, 37, 45
    nd = rng.integers(-100, 100, (B, R, C)).astype(dt)
    c0 = 32 // esize
    Rp, Cp = -(-R // 16) * 16, -(-C // c0) * c0
    pad = np.zeros((B, Rp, Cp), dt)
    pad[:, :R, :C] = nd
    ref = np.ascontiguousarray(pad.reshape(B, Rp // 16, 16, Cp // c0, c0).transpose(0, 3, 1, 2, 4))
    nz = O.nd_to_nz(nd, esize, B, R, C)
    assert np.array_equal(nz, ref.reshape(-1).view(np.uint8))
    assert np.array_equal(O.nz_to_nd(nz, esize, B, R, C).view(dt).reshape(B, R, C), nd)


# --------------------------------------------------------------------------- AscendAntiQuant policy form (3510)
def _bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _bf16_vals(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16).float().numpy()


def test_antiquant_policy_int8_half_and_bf16_arithmetic():
    """int8 source: + offset and * scale each rounded in scaleT -- numpy float16 arithmetic for half, torch bfloat16
    arithmetic for bf16 (ascend_antiquant_3510_impl.h:1386-1412, 1965-2011)"""
    rng = np.random.default_rng(901)
    m, n, g = 64, 48, 32
    q = rng.integers(-128, 128, (m, n)).astype(np.int8)
    sc = rng.uniform(0.001, 3.0, ((m + g - 1) // g, n))
    of = rng.uniform(-20.0, 20.0, ((m + g - 1) // g, n))
    rows = np.arange(m) // g
    sh, oh = sc.astype(np.float16), of.astype(np.float16)
    got = O.antiquant_policy(q, O.INT8, sh.view(np.uint16), O.F16, O.F16, O.PER_GROUP, m, n, g, oh.view(np.uint16))
    exp = (q.astype(np.float16) + oh[rows]) * sh[rows]
    assert np.array_equal(got, exp.view(np.uint16))
    sb, ob = _bf16_bits(sc), _bf16_bits(of)
    got = O.antiquant_policy(q, O.INT8, sb, O.BF16, O.BF16, O.PER_GROUP, m, n, g, ob)
    tq = torch.from_numpy(q.astype(np.float32)).to(torch.bfloat16)
    ts = torch.from_numpy(_bf16_vals(sb)[rows]).to(torch.bfloat16)
    to = torch.from_numpy(_bf16_vals(ob)[rows]).to(torch.bfloat16)
    exp = ((tq + to) * ts).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, exp)


def test_antiquant_policy_fp32_scale_and_fp8_source():
    """fp32 scaleT (and every fp8 source) compute in fp32 and cast once (rne, saturating) to the output; an fp8
    source with half scales still computes in fp32 (the half product would round twice)"""
    rng = np.random.default_rng(902)
    m, n = 16, 64
    q = rng.integers(-128, 128, (m, n)).astype(np.int8)
    sc = rng.uniform(0.001, 3.0, m).astype(np.float32)
    of = rng.uniform(-5.0, 5.0, m).astype(np.float32)
    got = O.antiquant_policy(q, O.INT8, sc, O.F32, O.F32, O.PER_TOKEN, m, n, offset=of)
    exp = (q.astype(np.float32) + of[:, None]) * sc[:, None]
    assert np.array_equal(got, exp)
    got16 = O.antiquant_policy(q, O.INT8, sc, O.F32, O.F16, O.PER_TOKEN, m, n, offset=of)
    assert np.array_equal(got16, exp.astype(np.float16).view(np.uint16))
    codes = rng.integers(0, 256, (m, n)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C  # no e4m3 NaN codes
    sh = rng.uniform(0.5, 1.5, n).astype(np.float16)
    oh = rng.uniform(-3.0, 3.0, n).astype(np.float16)
    got = O.antiquant_policy(codes, O.FP8_E4M3, sh.view(np.uint16), O.F16, O.F16, O.PER_TOKEN, m, n,
                             offset=oh.view(np.uint16), is_transpose=True)  # transposed: one scale per column
    v = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    exp = ((v + oh.astype(np.float32)[None, :]) * sh.astype(np.float32)[None, :]).astype(np.float16)
    assert np.array_equal(got, exp.view(np.uint16))


@pytest.mark.parametrize("k_dim,transpose", [(0, False), (1, False), (0, True), (1, True)])
def test_antiquant_policy_group_axis(k_dim, transpose):
    """PER_GROUP scale layout: along the columns ([m][ceil(n/g)]) when (kDim 1, not transposed) or (kDim 0,
    transposed), else along the rows ([ceil(m/g)][n]) (ascend_antiquant_3510_impl.h:2205-2212); scales 2^j make
    every index visible in the output"""
    m, n, g = 64, 96, 32
    q = np.ones((m, n), np.int8)
    col = (k_dim == 1 and not transpose) or (k_dim == 0 and transpose)
    shape = (m, (n + g - 1) // g) if col else ((m + g - 1) // g, n)
    sc = np.exp2(np.arange(shape[0] * shape[1]) % 24 - 12).astype(np.float32).reshape(shape)
    got = O.antiquant_policy(q, O.INT8, sc, O.F32, O.F32, O.PER_GROUP, m, n, g, k_dim=k_dim, is_transpose=transpose)
    r, c = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
    exp = sc[r, c // g] if col else sc[r // g, c]
    assert np.array_equal(got, exp)


def test_antiquant_policy_fp4_e8m0():
    """fp4 E2M1 with E8M0 group scales: bf16(v) * bf16(2^(e-127)) rounded once to bf16; e = 0 is 2^-127 (bf16
    0x0040), e = 255 NaN; half output is a saturating cast of that bf16 (ascend_antiquant_3510_impl.h:1724-1828)"""
    m, n, g = 4, 64, 32
    nib = np.tile(np.arange(16, dtype=np.uint8), (m, n // 16))
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    e = np.array([[127, 130], [0, 1], [254, 120], [255, 127]], np.uint8)
    got = O.antiquant_policy(packed, O.FP4_E2M1, e, O.E8M0, O.BF16, O.PER_GROUP, m, n, g, k_dim=1)
    mag = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)
    vals = np.concatenate([mag, -mag])[nib]
    scale = np.where(e == 0, 2.0 ** -127, np.exp2(e.astype(np.float64) - 127))[:, np.arange(n) // g]
    prod = vals * scale
    exp = _bf16_bits(prod.astype(np.float32))  # products of <= 2 significant bits: exact unless they overflow
    exp[3, :32] = 0x7FFF                       # e = 255 -> NaN (the NaN pattern of the scale)
    assert np.array_equal(got[:3], exp[:3]) and np.isnan(_bf16_vals(got[3, :32])).all()
    assert np.array_equal(got[3, 32:], exp[3, 32:])
    assert got[1, 2] == 0x0040 and got[2, 15] == 0xFF80  # 1 * 2^-127 (bf16 subnormal); -6 * 2^127 overflows to -inf
    h = O.antiquant_policy(packed, O.FP4_E2M1, e, O.E8M0, O.F16, O.PER_GROUP, m, n, g, k_dim=1)
    assert h[0, 15] == np.float16(-6.0).view(np.uint16) and h[2, 7] == 0x7BFF  # 6 * 2^127 saturates to 65504


# --------------------------------------------------------------------------- AscendQuant policy form
def _round_mode_np(y, mode):
    """float64 round modes of docs/zh/api/SIMD-API/tensor_api/reg_vector_compute/type_conversion/rounding_mode.md:17-25"""
    if mode == O.ROUND_FLOOR:
        return np.floor(y)
    if mode == O.ROUND_CEIL:
        return np.ceil(y)
    if mode == O.ROUND_TRUNC:
        return np.trunc(y)
    if mode == O.ROUND_ROUND:
        return np.sign(y) * np.floor(np.abs(y) + 0.5)
    return np.rint(y)


def _sat_s8(y, mode):
    with np.errstate(invalid="ignore"):
        r = np.clip(_round_mode_np(np.nan_to_num(y, nan=0.0, posinf=1e9, neginf=-1e9), mode), -128, 127)
    return r.astype(np.int8)


def test_quant_policy_int8_round_mode_table():
    """float -> integer round modes, the table of rounding_mode.md:40-47 (1.4, 1.5, 2.5, -1.4, -1.5, -2.5); 257
    saturates to 127 and NaN gives 0 under SAT (type_conversion/cast.md:108)"""
    x = np.array([[1.4, 1.5, 2.5, -1.4, -1.5, -2.5, 257.0, -300.0, np.nan, np.inf, -np.inf, 0.0]], np.float32)
    one = np.ones(1, np.float32)
    table = {O.ROUND_RINT: [1, 2, 2, -1, -2, -2], O.ROUND_ROUND: [1, 2, 3, -1, -2, -3],
             O.ROUND_FLOOR: [1, 1, 2, -2, -2, -3], O.ROUND_CEIL: [2, 2, 3, -1, -1, -2],
             O.ROUND_TRUNC: [1, 1, 2, -1, -1, -2], O.ROUND_NONE: [1, 2, 2, -1, -2, -2]}
    for mode, exp in table.items():
        got = O.quant_policy(x, O.F32, one, O.F32, O.INT8, O.PER_TOKEN, 1, x.shape[1], round_mode=mode)
        assert got[0].tolist() == exp + [127, -128, 0, 127, -128, 0], mode


@pytest.mark.parametrize("mode", [O.ROUND_RINT, O.ROUND_FLOOR, O.ROUND_CEIL, O.ROUND_ROUND, O.ROUND_TRUNC])
def test_quant_policy_int8_scale_type_arithmetic(mode):
    """int8 dst: x * s (+ o) with each op rounded in scaleT -- numpy float16 arithmetic for half, torch bfloat16 for
    bf16, numpy float32 for an f32 scale met by a half source -- then the round mode and saturation
    (ascend_quant_per_group_3510_impl.h:499-540, 1001-1046; TransRegForS8 ascend_quant_3510_impl.h:934-992)"""
    rng = np.random.default_rng(950 + mode)
    m, n, g = 64, 96, 32
    x = rng.uniform(-160.0, 160.0, (m, n))
    x[0, :8] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.5]  # exact ties with s = 1, o = 0
    sc = rng.uniform(0.05, 2.0, (m, (n + g - 1) // g))
    of = rng.uniform(-8.0, 8.0, sc.shape)
    sc[0, 0], of[0, 0] = 1.0, 0.0
    col = np.arange(n) // g
    xh, sh, oh = x.astype(np.float16), sc.astype(np.float16), of.astype(np.float16)
    got = O.quant_policy(xh.view(np.uint16), O.F16, sh.view(np.uint16), O.F16, O.INT8, O.PER_GROUP, m, n, g,
                         offset=oh.view(np.uint16), k_dim=1, round_mode=mode)
    y = (xh * sh[:, col]) + oh[:, col]
    assert np.array_equal(got, _sat_s8(y.astype(np.float64), mode))
    xb, sb, ob = _bf16_bits(x), _bf16_bits(sc), _bf16_bits(of)
    got = O.quant_policy(xb, O.BF16, sb, O.BF16, O.INT8, O.PER_GROUP, m, n, g, offset=ob, k_dim=1, round_mode=mode)
    t = lambda b: torch.from_numpy(_bf16_vals(b)).to(torch.bfloat16)
    yb = (t(xb) * t(sb)[:, col] + t(ob)[:, col]).double().numpy()
    assert np.array_equal(got, _sat_s8(yb, mode))
    s32, o32 = sc.astype(np.float32), of.astype(np.float32)
    got = O.quant_policy(xh.view(np.uint16), O.F16, s32, O.F32, O.INT8, O.PER_GROUP, m, n, g, offset=o32, k_dim=1,
                         round_mode=mode)
    y32 = xh.astype(np.float32) * s32[:, col] + o32[:, col]
    assert np.array_equal(got, _sat_s8(y32.astype(np.float64), mode))


def test_quant_policy_per_token_matches_fp32_per_token():
    """PER_TOKEN with an f32 scale and offset is the per-token quant already restated (quant_per_token); the two
    restatements agree element for element"""
    rng = np.random.default_rng(960)
    m, n = 32, 200
    x = rng.uniform(-300.0, 300.0, (m, n)).astype(np.float16)
    sc = rng.uniform(0.01, 1.5, m).astype(np.float32)
    of = rng.uniform(-4.0, 4.0, m).astype(np.float32)
    for mode in (O.ROUND_RINT, O.ROUND_FLOOR, O.ROUND_ROUND):
        a = O.quant_policy(x.view(np.uint16), O.F16, sc, O.F32, O.INT8, O.PER_TOKEN, m, n, offset=of, round_mode=mode)
        b = O.quant_per_token(x.view(np.uint16), O.F16, sc, of, round_mode=mode)
        assert np.array_equal(a, b)


@pytest.mark.parametrize("fmt", [O.FP8_E4M3, O.FP8_E5M2])
def test_quant_policy_fp8_in_fp32(fmt):
    """fp8 dst: x * s + o in fp32 whatever scaleT, then rint with saturation (ascend_quant_per_group_3510_impl.h:
    33-79, 393-431; TransRegForFp8 ascend_quant_3510_impl.h:888-896): torch's float8 casts (rne) after a clamp to
    the largest finite value; NaN -> 0 (cast.md:109)"""
    rng = np.random.default_rng(970 + fmt)
    m, n = 48, 128
    mx = 448.0 if fmt == O.FP8_E4M3 else 57344.0
    x = (rng.standard_normal((m, n)) * np.exp2(rng.integers(-12, 14, (m, n)))).astype(np.float16)
    x[0, :6] = [np.nan, np.inf, -np.inf, 65504.0, -65504.0, 0.0]
    sh = rng.uniform(0.5, 2.0, m).astype(np.float16)
    oh = rng.uniform(-1.0, 1.0, m).astype(np.float16)
    got = O.quant_policy(x.view(np.uint16), O.F16, sh.view(np.uint16), O.F16, fmt, O.PER_TOKEN, m, n,
                         offset=oh.view(np.uint16))
    with np.errstate(invalid="ignore", over="ignore"):
        v = x.astype(np.float32) * sh.astype(np.float32)[:, None] + oh.astype(np.float32)[:, None]
    v = np.where(np.isnan(v), 0.0, np.clip(v, -mx, mx)).astype(np.float32)
    dt = torch.float8_e4m3fn if fmt == O.FP8_E4M3 else torch.float8_e5m2
    exp = torch.from_numpy(v).to(dt).view(torch.uint8).numpy()
    assert np.array_equal(got, exp)
    assert got[0, 0] == 0 and got[0, 1] == (0x7E if fmt == O.FP8_E4M3 else 0x7B)
    # an f32 scale with a bf16 source: still one f32 product
    xb = _bf16_bits(rng.uniform(-30.0, 30.0, (m, n)))
    s32 = rng.uniform(0.5, 4.0, m).astype(np.float32)
    got = O.quant_policy(xb, O.BF16, s32, O.F32, fmt, O.PER_TOKEN, m, n)
    v = np.clip(_bf16_vals(xb) * s32[:, None], -mx, mx).astype(np.float32)
    assert np.array_equal(got, torch.from_numpy(v).to(dt).view(torch.uint8).numpy())


# E2M1 casts of a bf16 value, worked by hand from the mode definitions (rounding_mode.md:17-25) on the code table
# {0, 0.5, 1, 1.5, 2, 3, 4, 6}: the seven tie points, both signs, inside-interval values and saturation
_E2M1_X = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -2.5, 0.3, -0.3, 5.5, 7.0, -100.0, 6.0, -1.0]
_E2M1_KAT = {
    O.ROUND_RINT: [0x0, 0x2, 0x2, 0x4, 0x4, 0x6, 0x6, 0x8, 0xC, 0x1, 0x9, 0x7, 0x7, 0xF, 0x7, 0xA],
    O.ROUND_ROUND: [0x1, 0x2, 0x3, 0x4, 0x5, 0x6, 0x7, 0x9, 0xD, 0x1, 0x9, 0x7, 0x7, 0xF, 0x7, 0xA],
    O.ROUND_FLOOR: [0x0, 0x1, 0x2, 0x3, 0x4, 0x5, 0x6, 0x9, 0xD, 0x0, 0x9, 0x6, 0x7, 0xF, 0x7, 0xA],
    O.ROUND_CEIL: [0x1, 0x2, 0x3, 0x4, 0x5, 0x6, 0x7, 0x8, 0xC, 0x1, 0x8, 0x7, 0x7, 0xF, 0x7, 0xA],
    O.ROUND_TRUNC: [0x0, 0x1, 0x2, 0x3, 0x4, 0x5, 0x6, 0x8, 0xC, 0x0, 0x8, 0x6, 0x7, 0xF, 0x7, 0xA],
}


@pytest.mark.parametrize("mode", sorted(_E2M1_KAT))
def test_quant_policy_e2m1_round_modes(mode):
    """E2M1 dst (PER_GROUP): the bf16 -> E2M1 cast in each round mode with saturation (cast.md:96;
    TransRegForFp4 ascend_quant_3510_impl.h:995-1036), against the hand-worked table; packed two a byte, even
    element in the low nibble"""
    x = np.array([_E2M1_X], np.float32)
    n = x.shape[1]
    assert [O.lib().oq_e2m1_encode(float(v), mode) for v in _E2M1_X] == _E2M1_KAT[mode]
    one = _bf16_bits(np.ones((1, 1), np.float32))
    got = O.quant_policy(_bf16_bits(x), O.BF16, one, O.BF16, O.FP4_E2M1, O.PER_GROUP, 1, n, 32, k_dim=1,
                         round_mode=mode)
    k = np.array(_E2M1_KAT[mode], np.uint8)
    assert np.array_equal(got[0], k[0::2] | (k[1::2] << 4))


def test_quant_policy_e2m1_rint_matches_mx_encoder():
    """rint E2M1 agrees with the MX quantiser's nearest-even encoder (pinned by the MX golden) on a sweep of bf16
    values"""
    v = _bf16_vals(np.arange(0, 0x10000, 7, dtype=np.uint32).astype(np.uint16))
    v = v[np.isfinite(v) & (np.abs(v) < 64)]
    L = O.lib()
    assert all(L.oq_e2m1_encode(float(a), O.ROUND_RINT) == L.oq_e2m1_encode_rne(float(a)) for a in v)


def test_quant_policy_e2m1_through_bf16():
    """a half or f32 product is first rounded to bf16 (rne, saturating; NaN -> 0), then cast to E2M1: 0.7495 rounds to
    bf16 0.75, a tie that rint sends to 1.0 (code 2), where a direct cast would give 0.5 (code 1); an offset is
    ignored for E2M1 (ascend_quant_per_group_3510_impl.h:1385)"""
    xh = np.array([[0.74951171875, 2.49, -5.01, 70000.0 / 2, np.nan, 0.74951171875]], np.float16)
    xh = np.concatenate([xh, np.zeros((1, 26), np.float16)], axis=1)
    sh = np.ones((1, 1), np.float16)
    got = O.quant_policy(xh.view(np.uint16), O.F16, sh.view(np.uint16), O.F16, O.FP4_E2M1, O.PER_GROUP, 1, 32, 32,
                         offset=np.full((1, 1), 9.0, np.float16).view(np.uint16), k_dim=1)
    # 2.49 -> bf16 2.484375 -> 2 (code 4); -5.01 -> bf16 -5.0 -> tie -> -4 (code 0xE); 35000 -> 6; NaN -> 0
    assert got[0, :3].tolist() == [0x2 | (0x4 << 4), 0xE | (0x7 << 4), 0x0 | (0x2 << 4)]
    x32 = np.zeros((1, 32), np.float32)
    x32[0, :2] = [0.7499, 0.7499]
    got = O.quant_policy(x32, O.F32, np.ones((1, 1), np.float32), O.F32, O.FP4_E2M1, O.PER_GROUP, 1, 32, 32,
                         k_dim=1)
    assert got[0, 0] == 0x22  # f32 0.7499 -> bf16 0.75 -> rint 1.0


def test_e1m2_decode_table():
    """fp4x2_e1m2_t decode: sign | 1-bit exponent (bias 1) | 2-bit mantissa gives the magnitudes k / 4, k = 0..7; the
    largest finite value is 1.75 (mmad_mx_interface_boundary_value_summary.md:11) and every code is exact in bf16
    (precision_conversion.md:112-115)"""
    L = O.lib()
    got = [L.oq_e1m2_decode(c) for c in range(16)]
    assert got[:8] == [k / 4 for k in range(8)]
    assert got[8:] == [-k / 4 for k in range(8)] and math.copysign(1.0, got[8]) < 0
    assert all(_bf16_vals(_bf16_bits(np.array([v], np.float32)))[0] == v for v in got)


def test_e1m2_encode_published_cases():
    """bf16 -> fp4x2_e1m2_t worked example (precision_conversion.md:345-354): 1.375 -> CAST_RINT 1.5, CAST_FLOOR
    1.25, CAST_CEIL 1.5, CAST_ROUND 1.5, CAST_TRUNC 1.25; boundary table (mmad_mx_interface_boundary_value_summary.md:11):
    +inf -> 1.75, -inf -> -1.75, NaN -> 0"""
    L = O.lib()
    want = {O.ROUND_RINT: 1.5, O.ROUND_FLOOR: 1.25, O.ROUND_CEIL: 1.5, O.ROUND_ROUND: 1.5, O.ROUND_TRUNC: 1.25}
    for mode, v in want.items():
        assert L.oq_e1m2_decode(L.oq_e1m2_encode(1.375, mode)) == v
    for mode in want:
        assert L.oq_e1m2_encode(math.inf, mode) == 0x7
        assert L.oq_e1m2_encode(-math.inf, mode) == 0xF
        assert L.oq_e1m2_encode(math.nan, mode) == 0x0


def test_e1m2_encode_closed_form():
    """the E1M2 grid is uniform (step 0.25), so each round mode is numpy's integer rounding of 4 x on the signed value
    (rint ties to even, round ties away), magnitude clamped to 7, sign kept; checked on a sweep of bf16 values"""
    v = _bf16_vals(np.arange(0, 0x10000, 3, dtype=np.uint32).astype(np.uint16))
    v = v[np.isfinite(v)].astype(np.float64)
    away = lambda t: np.sign(t) * np.floor(np.abs(t) + 0.5)
    fns = {O.ROUND_RINT: np.rint, O.ROUND_FLOOR: np.floor, O.ROUND_CEIL: np.ceil, O.ROUND_ROUND: away,
           O.ROUND_TRUNC: np.trunc}
    L = O.lib()
    for mode, f in fns.items():
        with np.errstate(over="ignore", invalid="ignore"):
            k = np.minimum(np.abs(f(4.0 * v)), 7).astype(np.uint8)
        want = k | np.where(np.signbit(v), 8, 0).astype(np.uint8)
        got = np.array([L.oq_e1m2_encode(float(a), mode) for a in v], np.uint8)
        assert np.array_equal(got, want), mode


def test_quant_policy_e1m2_through_bf16():
    """E1M2 dst takes the same path as E2M1 (ascend_quant_per_group_3510_impl.h:1383-1440): an f32 product is rounded
    to bf16 first, so 0.3749 becomes 0.375, a tie (4 x = 1.5) that rint sends to code 2, where a direct cast would
    give code 1; saturation at 1.75 and NaN -> 0"""
    x = np.zeros((1, 32), np.float32)
    x[0, :6] = [0.3749, -0.3749, 3.0, -1e30, np.nan, 1.375]
    got = O.quant_policy(x, O.F32, np.ones((1, 1), np.float32), O.F32, O.FP4_E1M2, O.PER_GROUP, 1, 32, 32, k_dim=1)
    assert got[0, :3].tolist() == [0x2 | (0xA << 4), 0x7 | (0xF << 4), 0x0 | (0x6 << 4)]


def test_antiquant_policy_e1m2():
    """fp4 E1M2 source (PER_GROUP, E8M0 scales; ascend_antiquant_3510_impl.h:2144-2159 route both fp4 types alike):
    every code times 2^(e - 127), exact in bf16, equals the decoded value scaled by a power of two"""
    m, n, g = 4, 32, 32
    codes = np.arange(m * n, dtype=np.uint8).reshape(m, n) % 16
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    e = np.array([[127], [120], [130], [0]], np.uint8)
    got = O.antiquant_policy(packed, O.FP4_E1M2, e, O.E8M0, O.BF16, O.PER_GROUP, m, n, g, k_dim=1)
    L = O.lib()
    dec = np.array([[L.oq_e1m2_decode(int(c)) for c in row] for row in codes], np.float64)
    want = dec * np.ldexp(1.0, e.astype(np.int64) - 127)
    assert np.array_equal(_bf16_vals(got).astype(np.float64), want)


@pytest.mark.parametrize("k_dim", [0, 1])
def test_quant_policy_group_axis(k_dim):
    """PER_GROUP scale layout: kDim 1 groups along a row, scale [m][ceil(n/g)]; kDim 0 groups down a column,
    scale [ceil(m/g)][n] (ascend_quant_per_group_3510_impl.h:347-380, 727-760, 1001-1046); with x = 1 and integer
    scales the int8 output is the scale each element read, compared with numpy's repeat of the scale table"""
    m, n, g = 80, 96, 32
    shape = (m, (n + g - 1) // g) if k_dim == 1 else ((m + g - 1) // g, n)
    sc = ((np.arange(shape[0] * shape[1]) % 251) - 125).astype(np.float32).reshape(shape)
    got = O.quant_policy(np.ones((m, n), np.float32), O.F32, sc, O.F32, O.INT8, O.PER_GROUP, m, n, g, k_dim=k_dim)
    exp = np.repeat(sc, g, axis=1)[:, :n] if k_dim == 1 else np.repeat(sc, g, axis=0)[:m]
    assert np.array_equal(got, exp.astype(np.int8))


def test_quant_policy_scalar_offset():
    """the scalar-offset overloads take a scaleT value (ascend_quant_per_group_3510_impl.h:192-235, 297-333): a
    scalar 0.1 with half scales acts as the half 0.0999755859375 everywhere, like a tensor filled with it"""
    rng = np.random.default_rng(980)
    m, n, g = 8, 64, 32
    x = rng.uniform(-50.0, 50.0, (m, n)).astype(np.float16)
    sh = rng.uniform(0.5, 2.0, (m, 2)).astype(np.float16)
    full = np.full(sh.shape, np.float16(0.1), np.float16)
    for dst in (O.INT8, O.FP8_E5M2):
        a = O.quant_policy(x.view(np.uint16), O.F16, sh.view(np.uint16), O.F16, dst, O.PER_GROUP, m, n, g,
                           offset_scalar=0.1, k_dim=1)
        b = O.quant_policy(x.view(np.uint16), O.F16, sh.view(np.uint16), O.F16, dst, O.PER_GROUP, m, n, g,
                           offset=full.view(np.uint16), k_dim=1)
        c = O.quant_policy(x.view(np.uint16), O.F16, sh.view(np.uint16), O.F16, dst, O.PER_GROUP, m, n, g, k_dim=1)
        assert np.array_equal(a, b) and not np.array_equal(a, c)


# --------------------------------------------------------------------------- HiFloat8
def _hif8_nearest(x, table):
    """brute-force HiFloat8 code of each x: the nearest finite table value, ties to the larger magnitude, |x| >= 2^15
    saturating to +-32768, NaN -> 0, results of magnitude 0 coded 0x00 (exact rationals: every value involved is a
    float32)"""
    fin = [c for c in range(256) if np.isfinite(table[c]) and c != 0x80]
    vals = [(Fraction(float(table[c])), c) for c in fin]
    out = []
    for v in np.asarray(x, np.float32).reshape(-1):
        if np.isnan(v):
            out.append(0)
            continue
        if np.isinf(v) or abs(float(v)) >= 32768.0:
            out.append(0x6E if v > 0 else 0xEE)
            continue
        fv = Fraction(float(v))
        best = None
        for tv, c in vals:
            if (tv < 0) != (fv < 0) and tv != 0:
                continue
            d = abs(tv - fv)
            key = (d, -abs(tv))  # ties go to the larger magnitude (away from zero)
            if best is None or key < best[0]:
                best = (key, c, tv)
        out.append(0x00 if best[2] == 0 else best[1])
    return np.array(out, np.uint8)


def test_hif8_decode_published_points():
    """0x00 zero, 0x80 NaN, 0x6F / 0xEF +-inf, 0x6E the saturation value 32768 (__half22hif82_rna_sat.md table),
    0x01 the smallest subnormal 2^-22 that Ev = -23 rounds to (Cast.md:263-266), the documented example D = 01,
    E = 3, M = 2^-1 + 2^-2 -> 14 (fp8_data_type_intro.md:36), and the 1-bit exponent field's sign"""
    t = O.hif8_table()
    assert t[0x00] == 0 and np.isnan(t[0x80]) and t[0x6F] == np.inf and t[0xEF] == -np.inf
    assert t[0x6E] == 32768.0 and t[0xEE] == -32768.0
    assert t[0x01] == 2.0 ** -22 and t[0x81] == -(2.0 ** -22)
    assert t[0b0_01_01_110] == 14.0
    assert t[0b0_001_0_000] == 2.0 and t[0b0_001_1_000] == 0.5 and t[0b0_0001_000] == 1.0
    fin = t[np.isfinite(t)]
    assert np.abs(fin).max() == 32768.0 and np.abs(fin[fin != 0]).min() == 2.0 ** -22
    assert (fin.astype(np.float16).astype(np.float32) == fin).all()  # every code is an f16 value
    pos = np.unique(fin[fin > 0])
    assert len(pos) == 126  # 0x01..0x7F without the inf code 0x6F, each a distinct value
    assert (t[0x81:0x100][np.isfinite(t[0x81:0x100])] == -t[0x01:0x80][np.isfinite(t[0x01:0x80])]).all()


def test_hif8_encode_inverts_decode():
    """the encoder (Cast.md's rules) and the decoder (the layout of asc_type_conversion_utils.h) are independent
    restatements: encoding every finite code's value gives the code back"""
    t = O.hif8_table()
    for c in range(256):
        if c in (0x80, 0x6F, 0xEF) or (c == 0x00):
            continue
        assert O.lib().oq_hif8_encode(float(t[c]), 0) == c, hex(c)


def test_hif8_encode_saturation_table():
    """__half22hif82_rna_sat.md: +-0 -> 0, nan -> 0, +-inf -> +-32768, +-65504 -> +-32768, 2^-24 -> 0; without
    saturation nan is 0x80 and overflow +-inf"""
    L = O.lib()
    kat = {0.0: 0x00, -0.0: 0x00, float("nan"): 0x00, float("inf"): 0x6E, float("-inf"): 0xEE, 65504.0: 0x6E,
           -65504.0: 0xEE, 2.0 ** -24: 0x00, 40960.0: 0x6E, 32768.0: 0x6E}
    for x, c in kat.items():
        assert L.oq_hif8_encode(x, 1) == c, x
    assert L.oq_hif8_encode(float("nan"), 0) == 0x80
    assert L.oq_hif8_encode(65504.0, 0) == 0x6F and L.oq_hif8_encode(-1e30, 0) == 0xEF
    assert L.oq_hif8_encode(36000.0, 0) == 0x6E  # below 1.25 * 2^15: still 32768


def test_hif8_encode_matches_nearest_ties_away_on_every_f16():
    """every f16 bit pattern (the half -> hifloat8 cast of the legacy quant) against the brute-force nearest code"""
    t = O.hif8_table()
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    got = O.hif8_encode(x, sat=True)
    sel = rng0.choice(65536, 6000, replace=False)
    np.testing.assert_array_equal(got[sel], _hif8_nearest(x[sel], t))
    # exact ties between neighbouring codes round away from zero
    pos = np.unique(t[np.isfinite(t) & (t > 0)]).astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    assert (mids.astype(np.float64) == (pos[:-1] + pos[1:]) / 2).all()
    np.testing.assert_array_equal(O.hif8_encode(mids), _hif8_nearest(mids, t))
    np.testing.assert_array_equal(O.hif8_encode(-mids), _hif8_nearest(-mids, t))


def test_hif8_encode_random_f32():
    t = O.hif8_table()
    x = (rng0.standard_normal(4000) * np.exp2(rng0.uniform(-26, 17, 4000))).astype(np.float32)
    np.testing.assert_array_equal(O.hif8_encode(x), _hif8_nearest(x, t))


def hif8_codes(rng, shape, lo=None, hi=None):
    """random finite HiFloat8 codes (no NaN 0x80, no +-inf 0x6F / 0xEF); with lo / hi, the codes of the integers
    lo .. hi (the sample's data class: uniform(0, 5) cast to integers, then encoded)"""
    if lo is not None:
        ints = rng.integers(lo, hi + 1, shape).astype(np.float32)
        return O.hif8_encode(ints.reshape(-1)).reshape(shape)
    c = rng.integers(0, 256, shape, dtype=np.int64).astype(np.uint8)
    bad = (c == 0x80) | ((c & 0x7F) == 0x6F)
    return np.where(bad, np.uint8(0x08), c).astype(np.uint8)


def test_hif8_matmul_vs_numpy_decode():
    """hifloat8 x hifloat8 Matmul (matmul_fp8.asc:229): the oracle's exact sums against a numpy fp64 matmul of the
    HiFloat8 table's values (the table pinned above), with f32 bias, both transposes, and f32 / f16 / bf16 outputs
    as the casts of (sum + bias) * M1"""
    t = O.hif8_table().astype(np.float64)
    M, N, K = 24, 40, 96
    A = hif8_codes(rng0, (M, K))
    B = hif8_codes(rng0, (K, N))
    bias = rng0.standard_normal(N).astype(np.float32)
    exact_np = t[A] @ t[B] + bias.astype(np.float64)[None, :]
    for ta, tb in [(False, False), (True, True)]:
        Ain = np.ascontiguousarray(A.T) if ta else A
        Bin = np.ascontiguousarray(B.T) if tb else B
        out, exact, absd, bmax = O.matmul_fp8(Ain, Bin, O.HIF8, O.HIF8, bias=bias, out_type=O.F32, trans_a=ta,
                                              trans_b=tb)
        assert np.allclose(exact, exact_np, rtol=1e-12, atol=0)
        assert np.allclose(absd, np.abs(t[A]) @ np.abs(t[B]), rtol=1e-12, atol=0)
        assert np.array_equal(out, exact.astype(np.float32))
    m1 = np.float32(2.0 ** -9)
    word = int(m1.view(np.uint32))
    for ot, cast in [(O.F16, np.float16), (O.BF16, None)]:
        out, exact, _, _ = O.matmul_fp8(A, B, O.HIF8, O.HIF8, bias=bias, out_type=ot, use_q=True, qscalar=word)
        v = (exact.astype(np.float32) * m1).astype(np.float32)
        if cast is not None:
            exp = np.clip(v, -65504, 65504).astype(np.float16).view(np.uint16)
        else:
            exp = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(out, exp)


def test_hif8_matmul_sample_golden():
    """the sample's own data class and check (matmul_fp8/scripts/gen_data.py gen_golden_data_hif8: A [428, 158] and
    B [158, 479] from uniform(0, 5) cast to uint8, encoded to hifloat8, f32 bias uniform(-1, 1), golden = fp32
    matmul + bias; verify_result.py: rtol = atol = 1e-3, error ratio <= 1e-3): the sums are integers below 2^24, so
    the oracle matches the fp32 golden exactly"""
    rng = np.random.default_rng(229)
    M, N, K = 428, 479, 158
    a_int = rng.uniform(0, 5, (M, K)).astype(np.uint8)
    b_int = rng.uniform(0, 5, (K, N)).astype(np.uint8)
    bias = rng.uniform(-1, 1, N).astype(np.float32)
    A = O.hif8_encode(a_int.astype(np.float32).reshape(-1)).reshape(M, K)
    B = O.hif8_encode(b_int.astype(np.float32).reshape(-1)).reshape(K, N)
    golden = ((a_int.astype(np.float32) @ b_int.astype(np.float32)) + bias[None, :]).astype(np.float32)
    out, _, _, _ = O.matmul_fp8(A, B, O.HIF8, O.HIF8, bias=bias, out_type=O.F32)
    assert ref_verify(out, golden)
    assert np.array_equal(out, golden)


def test_hif8_matmul_hif8_output():
    """(V)QF322HIF8_PRE: (sum + bias) * M1 encoded with ties away and saturation (the encoder pinned above); the
    per-channel words reach the right columns, and sums past 32768 saturate"""
    M, N, K = 16, 24, 64
    A = hif8_codes(rng0, (M, K), -4, 4)
    B = hif8_codes(rng0, (K, N), -4, 4)
    t = O.hif8_table().astype(np.float64)
    m1 = np.exp2(rng0.integers(-4, 9, N)).astype(np.float32) * np.float32(1.375)
    words = m1.view(np.uint32).astype(np.uint64)
    out, exact, _, _ = O.matmul_fp8(A, B, O.HIF8, O.HIF8, out_type=O.HIF8, use_q=True, qvec=words)
    assert np.array_equal(exact, t[A] @ t[B])
    v = (exact.astype(np.float32) * m1[None, :]).astype(np.float32)
    assert np.array_equal(out, O.hif8_encode(v.reshape(-1)).reshape(M, N))
    assert (np.abs(v) >= 32768).any() and ((out & 0x7F) == 0x6E).any()


# --------------------------------------------------------------------------- legacy AscendQuant, arch-3510 form
def _h(v):
    return np.asarray(v, np.float64).astype(np.float16)  # one correctly rounded conversion


def _half_ops(x32, s32, o32, sat_x=True, sat_so=True):
    """t = half(x*s); t = half(t + o) with x, s, o first rounded to half (saturating where the reference saturates)"""
    def to_h(v, sat):
        v = np.asarray(v, np.float64)
        return (np.clip(v, -65504, 65504) if sat else v).astype(np.float16)
    xh, sh, oh = to_h(x32, sat_x), to_h(s32, sat_so), to_h(o32, sat_so)
    t = _h(xh.astype(np.float64) * sh.astype(np.float64))
    return _h(t.astype(np.float64) + oh.astype(np.float64))


def _bf16(v):
    t = torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16), t.float().numpy()


def test_quant_legacy_int8_f16_matches_the_half_form():
    """an f16 source with f16 scale / offset tensors is the 2201 half-arithmetic form (oq_quant_legacy_f16), and
    the quant example golden (scale 2.0, offset 0.9) is reproduced from float scalars"""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(4096) * 40).astype(np.float16)
    sc = rng.uniform(-3, 3, 64).astype(np.float16)
    of = rng.uniform(-20, 20, 64).astype(np.float16)
    a = O.quant_legacy(x.view(np.uint16), O.F16, O.INT8, sc.view(np.uint16), of.view(np.uint16), scale_count=64)
    b = O.quant_legacy_f16(x.view(np.uint16), O.F16, scale_vec=sc.view(np.uint16), offset_vec=of.view(np.uint16),
                           scale_count=64)
    np.testing.assert_array_equal(a, b)
    f = np.load(GOLD / "quant_example.npz")
    q = O.quant_legacy(f["src"].view(np.uint16), O.F16, O.INT8, scale_scalar=2.0, offset_scalar=0.9)
    assert (q == f["golden"]).all()


@pytest.mark.parametrize("src_type", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("dst_type", [O.INT8, O.HIF8, O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("kind", ["tensor", "scalar_offset", "per_tensor"])
def test_quant_legacy_3510_forms(src_type, dst_type, kind):
    """int8 / hifloat8: half arithmetic after saturating casts of the srcT tensors (plain rne for the float scalars),
    rint / ties-away with saturation; fp8: fp32 arithmetic, rint with saturation, NaN -> 0 -- checked with numpy /
    torch arithmetic, torch's fp8 casts and the brute-force HiFloat8 coder; sources beyond the f16 range included"""
    rng = np.random.default_rng(10 * src_type + dst_type + len(kind))
    n, sc_n = 2048, 32
    x = (rng.standard_normal(n) * np.exp2(rng.uniform(-6, 10, n))).astype(np.float32)
    x[:4] = [1e6, -7e4, 70000.0, np.nan]
    s = rng.uniform(-2, 2, sc_n).astype(np.float32) * np.float32(0.01 if dst_type == O.INT8 else 1.0)
    o = rng.uniform(-30, 30, sc_n).astype(np.float32)
    if src_type == O.F16:
        xs, s_, o_ = x.astype(np.float16), s.astype(np.float16), o.astype(np.float16)
        xw, sw, ow = xs.view(np.uint16), s_.view(np.uint16), o_.view(np.uint16)
        xv, sv, ov = xs.astype(np.float32), s_.astype(np.float32), o_.astype(np.float32)
    elif src_type == O.BF16:
        (xw, xv), (sw, sv), (ow, ov) = _bf16(x), _bf16(s), _bf16(o)
    else:
        xw, sw, ow, xv, sv, ov = x, s, o, x, s, o
    ss, osc = np.float32(0.0137), np.float32(2.71875)
    if kind == "tensor":
        q = O.quant_legacy(xw, src_type, dst_type, sw, ow, scale_count=sc_n)
        S, OFF, sat_so = np.tile(sv, n // sc_n), np.tile(ov, n // sc_n), True
    elif kind == "scalar_offset":
        q = O.quant_legacy(xw, src_type, dst_type, sw, None, offset_scalar=float(osc), scale_count=sc_n)
        o_src = {O.F16: np.float32(np.float16(osc)), O.BF16: _bf16(np.array([osc]))[1][0], O.F32: osc}[src_type]
        S, OFF, sat_so = np.tile(sv, n // sc_n), np.full(n, o_src, np.float32), True
    else:
        q = O.quant_legacy(xw, src_type, dst_type, scale_scalar=float(ss), offset_scalar=float(osc))
        S, OFF, sat_so = np.full(n, ss, np.float32), np.full(n, osc, np.float32), False
    if dst_type in (O.FP8_E4M3, O.FP8_E5M2):
        v = (xv * S).astype(np.float32) + OFF  # numpy float32 ops: one rounding each
        mx = 448.0 if dst_type == O.FP8_E4M3 else 57344.0
        fdt = torch.float8_e4m3fn if dst_type == O.FP8_E4M3 else torch.float8_e5m2
        c = torch.from_numpy(np.clip(np.nan_to_num(v, nan=0.0), -mx, mx).astype(np.float32)).to(fdt)
        np.testing.assert_array_equal(q, c.view(torch.uint8).numpy())
        return
    sat_x = src_type != O.F16
    t = _half_ops(xv, S, OFF, sat_x=sat_x, sat_so=sat_so)
    tv = t.astype(np.float32)
    if dst_type == O.INT8:
        exp = np.clip(np.rint(np.nan_to_num(tv, nan=0.0, posinf=127, neginf=-128)), -128, 127).astype(np.int8)
        np.testing.assert_array_equal(q, exp)
    else:
        sel = rng.choice(n, 300, replace=False)
        np.testing.assert_array_equal(q[sel], _hif8_nearest(tv[sel], O.hif8_table()))


def test_quant_policy_hif8():
    """PER_TOKEN / PER_GROUP to hifloat8: the int8 path's scaleT arithmetic, then ties away with saturation"""
    rng = np.random.default_rng(17)
    m, n = 16, 256
    x = (rng.standard_normal((m, n)) * 50).astype(np.float32)
    sc = np.exp2(rng.uniform(-3, 8, m)).astype(np.float32)
    of = rng.uniform(-4, 4, m).astype(np.float32)
    q = O.quant_policy(x, O.F32, sc, O.F32, O.HIF8, O.PER_TOKEN, m, n, offset=of)
    v = (x * sc[:, None]).astype(np.float32) + of[:, None]
    sel = rng.choice(m * n, 400, replace=False)
    np.testing.assert_array_equal(q.reshape(-1)[sel], _hif8_nearest(v.reshape(-1)[sel], O.hif8_table()))
    xh = x.astype(np.float16)
    sh = sc.astype(np.float16)
    q = O.quant_policy(xh.view(np.uint16), O.F16, sh.view(np.uint16), O.F16, O.HIF8, O.PER_TOKEN, m, n)
    v = _h(xh.astype(np.float64) * sh.astype(np.float64)[:, None]).astype(np.float32)
    np.testing.assert_array_equal(q.reshape(-1)[sel], _hif8_nearest(v.reshape(-1)[sel], O.hif8_table()))


def test_antiquant_hif8_and_fp8_sources():
    """legacy AscendAntiQuant of hifloat8 / fp8: fp8 in fp32 ops; hifloat8 to f16 in half ops; hifloat8 to bf16 in
    bf16 ops along rows and in fp32 ops when transposed; the policy form treats hifloat8 like int8 (scaleT ops)"""
    rng = np.random.default_rng(23)
    K, N = 64, 48
    t = O.hif8_table()
    codes = rng.integers(0, 256, (K, N), dtype=np.uint8)
    codes[np.isin(codes, [0x80, 0x6F, 0xEF])] = 0x21
    q = t[codes].astype(np.float64)
    s32 = rng.uniform(-0.5, 0.5, N).astype(np.float32)
    o32 = rng.uniform(-3, 3, N).astype(np.float32)
    # f16 dst: half ops
    sh, oh = s32.astype(np.float16), o32.astype(np.float16)
    y = O.antiquant(codes, O.HIF8, sh.view(np.uint16), oh.view(np.uint16), K, N, 0, False, O.F16, O.ARITH_F32)
    e = _h(_h(q + oh.astype(np.float64)).astype(np.float64) * sh.astype(np.float64))
    np.testing.assert_array_equal(y, e.view(np.uint16))
    # bf16 dst along rows: bf16 ops (torch bf16 add / mul, each correctly rounded)
    sbw, sbv = _bf16(s32)
    obw, obv = _bf16(o32)
    y = O.antiquant(codes, O.HIF8, sbw, obw, K, N, 0, False, O.BF16, O.ARITH_F32)
    qt = torch.from_numpy(q.astype(np.float32)).to(torch.bfloat16)
    e = (qt + torch.from_numpy(obv).to(torch.bfloat16)) * torch.from_numpy(sbv).to(torch.bfloat16)
    np.testing.assert_array_equal(y, e.view(torch.int16).numpy().view(np.uint16))
    # bf16 dst transposed ([N, K] source): fp32 ops, one rint cast
    ct = np.ascontiguousarray(codes.T)
    y = O.antiquant(ct, O.HIF8, sbw, obw, K, N, 0, True, O.BF16, O.ARITH_F16)
    e32 = ((t[ct] + obv[:, None]).astype(np.float32) * sbv[:, None]).astype(np.float32)
    np.testing.assert_array_equal(y, _bf16(e32)[0])
    # fp8 source, f16 dst: fp32 ops then one rne cast, whatever arith the caller passes
    f8 = rng.integers(0, 256, (K, N), dtype=np.uint8)
    f8[(f8 & 0x7F) == 0x7F] = 0x11
    fv = torch.from_numpy(f8).view(torch.float8_e4m3fn).float().numpy()
    y = O.antiquant(f8, O.FP8_E4M3, sh.view(np.uint16), oh.view(np.uint16), K, N, 0, False, O.F16, O.ARITH_F16)
    e32 = ((fv + oh.astype(np.float32)).astype(np.float32) * sh.astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(y, np.clip(e32, -65504, 65504).astype(np.float16).view(np.uint16))
    # per tensor: hifloat8 -> f16 half ops, -> bf16 fp32 ops; scale only
    ys = O.antiquant_scalar(codes, O.HIF8, int(oh[0].view(np.uint16)), int(sh[0].view(np.uint16)), O.F16)
    np.testing.assert_array_equal(ys, _h(_h(q + float(oh[0])).astype(np.float64) * float(sh[0])).view(np.uint16)
                                  .reshape(-1))
    ys = O.antiquant_scalar(codes, O.HIF8, int(obw[0]), int(sbw[0]), O.BF16, has_offset=False)
    np.testing.assert_array_equal(ys, _bf16((t[codes] * np.float32(sbv[0])).astype(np.float32))[0].reshape(-1))
    # policy form: hifloat8 like int8 in f16 scaleT ops
    yp = O.antiquant_policy(codes, O.HIF8, sh.view(np.uint16), O.F16, O.F16, O.PER_TOKEN, K, N, is_transpose=True,
                            offset=oh.view(np.uint16))
    np.testing.assert_array_equal(yp, _h(_h(q + oh.astype(np.float64)).astype(np.float64) * sh.astype(np.float64))
                                  .view(np.uint16))


# ---------------------------------------------------------------------------------------------------------------
# MX matmul with fp4x2_e1m2_t elements and an f32 bias
# ---------------------------------------------------------------------------------------------------------------
E1M2 = [k / 4 for k in range(8)]  # sign | 1-bit exponent (bias 1) | 2-bit mantissa: magnitudes k / 4


def _fp4_table(fmt):
    mags = E1M2 if fmt == O.FP4_E1M2 else E2M1
    return np.array([mags[c & 7] * (-1 if c & 8 else 1) for c in range(16)])


@pytest.mark.parametrize("fa,fb", [(O.FP4_E1M2, O.FP4_E1M2), (O.FP4_E1M2, O.FP4_E2M1), (O.FP4_E2M1, O.FP4_E1M2)])
def test_mx_matmul_e1m2_vs_numpy_decode(fa, fb):
    """the reference golden of the E1M2 sample (matmul_mxfp4_high_performance/scripts/gen_data.py:47-61): each
    element times 2^(scale - 127) of its 32-element K block, fp64 matmul; here against an independent numpy
    decode of the format tables, every code and a spread of block scales"""
    M, N, K = 8, 12, 256
    A = rng0.integers(0, 256, (M, K // 2), dtype=np.uint8)
    Bt = rng0.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sA = rng0.integers(110, 140, (M, K // 32), dtype=np.uint8)
    sB = rng0.integers(110, 140, (N, K // 32), dtype=np.uint8)

    def dec(p, s, fmt):
        v = _fp4_table(fmt)[np.stack([p & 0xF, p >> 4], -1).reshape(p.shape[0], -1)]
        return v * 2.0 ** (np.repeat(s.astype(np.float64), 32, axis=1) - 127)

    exact = dec(A, sA, fa) @ dec(Bt, sB, fb).T
    _, Ce, _ = O.mx_matmul(A, Bt, sA, sB, M, N, K, trans_b=True, sa_layout=0, sb_layout=1, elem_fmt=fa, fmt_b=fb)
    assert np.allclose(Ce, exact, rtol=1e-13, atol=1e-13)


def test_mx_matmul_e1m2_sample_data():
    """the sample's own data classes: elements randint(-1, 2) cast to e1m2 (codes for -1, 0, 1), scales
    randint(127, 130), B given [K, N] with scales [sK/2, N, 2]; the exact sums are integers times powers of two,
    so the bf16 golden of each is its rne cast"""
    M, N, K = 16, 24, 256
    a = rng0.integers(-1, 2, (M, K))
    b = rng0.integers(-1, 2, (K, N))
    code = {-1: 0xC, 0: 0x0, 1: 0x4}  # e1m2: 1.0 = exponent 1, mantissa 0
    ca = np.vectorize(code.get)(a).astype(np.uint8)
    cb = np.vectorize(code.get)(b).astype(np.uint8)
    A = (ca[:, 0::2] | (ca[:, 1::2] << 4)).astype(np.uint8)
    B = (cb[:, 0::2] | (cb[:, 1::2] << 4)).astype(np.uint8)  # [K, N/2], two per byte along N
    sK = K // 32
    sA = rng0.integers(127, 130, (M, sK), dtype=np.uint8)
    sB = rng0.integers(127, 130, (sK, N), dtype=np.uint8)
    sB_pairs = np.ascontiguousarray(sB.reshape(sK // 2, 2, N).transpose(0, 2, 1))
    exact = (a * 2.0 ** (np.repeat(sA.astype(np.float64), 32, 1) - 127)) @ (
        b * 2.0 ** (np.repeat(sB.astype(np.float64), 32, 0) - 127))
    C, Ce, _ = O.mx_matmul(A, B, sA, sB_pairs, M, N, K, trans_b=False, sa_layout=0, sb_layout=0,
                           elem_fmt=O.FP4_E1M2)
    assert np.array_equal(Ce, exact)
    assert np.array_equal(C, _bf16_bits(exact.astype(np.float32)))


def test_mx_matmul_bias():
    """SetBias on the MX matmul (matmul_mx/matmul_mx.asc:99-116,199-201): an f32 [N] bias joins the sum before the
    output cast, and its magnitude the absolute sum"""
    M, N, K = 4, 8, 128
    A = rng0.integers(0, 256, (M, K // 2), dtype=np.uint8)
    Bt = rng0.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sA = np.full((M, K // 32), 127, np.uint8)
    sB = np.full((N, K // 32), 127, np.uint8)
    bias = rng0.standard_normal(N).astype(np.float32)
    _, Ce0, Ca0 = O.mx_matmul(A, Bt, sA, sB, M, N, K, trans_b=True, sa_layout=0, sb_layout=1)
    C, Ce, Ca = O.mx_matmul(A, Bt, sA, sB, M, N, K, trans_b=True, sa_layout=0, sb_layout=1, bias=bias)
    assert np.array_equal(Ce, Ce0 + bias.astype(np.float64))
    assert np.array_equal(Ca, Ca0 + np.abs(bias.astype(np.float64)))
    assert np.array_equal(C, _bf16_bits(Ce.astype(np.float32))) or np.abs(
        _bf16_vals(C) - Ce).max() <= np.abs(Ce).max() * 2.0 ** -8


# ---------------------------------------------------------------------------------------------------------------
# IterateAll enAtomic: C = add / max / min (C, result) in C's type
# ---------------------------------------------------------------------------------------------------------------
def test_combine_int32():
    """int32 C: wrapping add (two's complement, as the int32 accumulators wrap), signed max / min"""
    c = rng0.integers(-2**31, 2**31, 4096).astype(np.int32)
    v = rng0.integers(-2**31, 2**31, 4096).astype(np.int32)
    add = ((c.astype(np.int64) + v) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
    assert np.array_equal(O.c_combine(c, v, O.INT32, 1), add)
    assert np.array_equal(O.c_combine(c, v, O.INT32, 2), np.maximum(c, v))
    assert np.array_equal(O.c_combine(c, v, O.INT32, 3), np.minimum(c, v))


def test_combine_float_add_known_answers():
    """single rounding to nearest even in C's type, overflow to inf (the IEEE sum)"""
    f32 = O.c_combine(np.array([1.0, 1.0, 3e38], np.float32), np.array([2.0 ** -24, 3 * 2.0 ** -24, 3e38], np.float32),
                      O.F32, 1)
    assert f32[0] == 1.0 and f32[1] == np.float32(1.0 + 2.0 ** -22) and np.isinf(f32[2])
    h = lambda xs: np.array(xs, np.float16).view(np.uint16)
    # 2048 + 1 = 2049: a tie between 2048 and 2050, even -> 2048; 2048 + 3 -> 2052; 65504 + 16 = 65520: a tie
    # between 65504 (odd) and 65536 -> inf; 1 + 2^-11 (a tie) -> 1; subnormal sum exact
    got = O.c_combine(h([2048, 2048, 65504, 1.0, 2.0 ** -24]), h([1, 3, 16, 2.0 ** -11, 2.0 ** -23]), O.F16, 1)
    assert np.array_equal(got.view(np.float16), np.array([2048, 2052, np.inf, 1.0, 3 * 2.0 ** -24], np.float16))
    # bf16: 1 + 2^-8 is a tie -> 1; 1 + 3 * 2^-8 -> 1 + 2^-6 (tie to even); 1.5 * 2^127 + 2^127 -> inf
    b = lambda xs: _bf16_bits(np.array(xs, np.float32))
    got = O.c_combine(b([1.0, 1.0, 1.5 * 2.0 ** 127]), b([2.0 ** -8, 3 * 2.0 ** -8, 2.0 ** 127]), O.BF16, 1)
    assert np.array_equal(_bf16_vals(got), np.array([1.0, 1.0 + 2.0 ** -6, np.inf]))


def test_combine_half_add_matches_torch():
    """random f16 / bf16 pairs over the whole finite range against torch's CPU add (fp32 sum, rne cast): the
    fp32 intermediate of p' = 24 >= 2p + 1 bits makes that the correctly rounded sum"""
    import torch
    for ct, tdt in ((O.F16, torch.float16), (O.BF16, torch.bfloat16)):
        bits = rng0.integers(0, 65536, (2, 20000)).astype(np.uint16)
        t = torch.from_numpy(bits.view(np.int16)).view(tdt)
        ok = torch.isfinite(t).all(0)
        a, v = t[0][ok], t[1][ok]
        want = (a + v).view(torch.int16).numpy().view(np.uint16)
        got = O.c_combine(a.view(torch.int16).numpy().view(np.uint16), v.view(torch.int16).numpy().view(np.uint16),
                          ct, 1)
        nan = torch.isnan(a + v).numpy()
        assert np.array_equal(got[~nan], want[~nan])


def test_combine_max_min_special_values():
    """max / min replace C only when the new value compares greater / smaller: a NaN never replaces and is never
    replaced, -0 does not replace +0 (nor the reverse)"""
    c = np.array([1.0, np.nan, 0.0, -0.0, -3.0, 2.0], np.float32)
    v = np.array([2.0, 5.0, -0.0, 0.0, np.nan, -7.0], np.float32)
    mx = O.c_combine(c, v, O.F32, 2)
    mn = O.c_combine(c, v, O.F32, 3)
    assert np.array_equal(mx.view(np.uint32), np.array([2.0, np.nan, 0.0, -0.0, -3.0, 2.0], np.float32).view(np.uint32))
    assert np.array_equal(mn.view(np.uint32), np.array([1.0, np.nan, 0.0, -0.0, -3.0, -7.0], np.float32).view(np.uint32))
    h16 = np.array([1.0, -2.0, 3.0], np.float16).view(np.uint16)
    w16 = np.array([0.5, -1.0, 3.0], np.float16).view(np.uint16)
    assert np.array_equal(O.c_combine(h16, w16, O.F16, 2).view(np.float16), np.array([1.0, -1.0, 3.0], np.float16))
    assert np.array_equal(O.c_combine(h16, w16, O.F16, 3).view(np.float16), np.array([0.5, -2.0, 3.0], np.float16))


# --------------------------------------------------------------------------- Quantize / Dequantize / AntiQuantize
def test_quantize_per_tensor_example_golden_exact():
    """the reference's quant example on arch 3510 (quant.asc: Quantize PER_TENSOR, scale 2.0, offset 0.9, CAST_RINT,
    float32 source) against its own golden np.round(src * 2.0 + 0.9)"""
    f = np.load(GOLD / "quant_example_3510.npz")
    src = f["src"].reshape(1, -1)
    got = O.quantize(src, O.F32, O.INT8, O.PER_TENSOR, 1, src.shape[1], scale_scalar=2.0, offset_scalar=0.9)
    assert np.array_equal(got[0], f["golden"])


def test_dequantize_per_channel_example_golden_exact():
    """the reference's dequant example on arch 3510 (dequant.asc: Dequantize PER_CHANNEL, int32 [128, 32], f32 scale
    [32]) against its golden inp * scale in float32"""
    f = np.load(GOLD / "dequant_example.npz")
    y = O.dequantize(f["inp"], O.INT32, O.F32, O.PER_CHANNEL, scale=f["scale"], scale_type=O.F32)
    assert (y.view(np.uint32) == f["golden"].view(np.uint32)).all()


def test_antiquantize_per_channel_example_golden_exact():
    """the reference's antiquant example on arch 3510 (antiquant.asc: AntiQuantize PER_CHANNEL with an offset, int8
    [8, 128], f16 offset / scale [1, 128]) against its golden: fp32 (src + offset) * scale, one cast to f16"""
    f = np.load(GOLD / "antiquant_seed10.npz")
    y = O.antiquantize(f["src"], O.INT8, O.F16, O.PER_CHANNEL, 8, 128, scale=f["scale"].view(np.uint16).reshape(-1),
                       scale_type=O.F16, offset=f["offset"].view(np.uint16).reshape(-1))
    assert np.array_equal(y, f["golden_3510"].view(np.uint16))
    assert not np.array_equal(y, f["golden_2201"].view(np.uint16))  # the half-arithmetic golden differs


def _policy_tables(rng, policy, m, n, g, lo, hi):
    """(scale argument, broadcast [m, n] view) for a policy: PER_TENSOR a scalar, PER_CHANNEL [n], PER_TOKEN [m],
    PER_GROUP kDim 0 [ceil(m / g)][n]"""
    if policy == O.PER_TENSOR:
        v = np.float32(rng.uniform(lo, hi))
        return v, np.full((m, n), v, np.float32)
    if policy == O.PER_CHANNEL:
        v = rng.uniform(lo, hi, n).astype(np.float32)
        return v, np.broadcast_to(v[None, :], (m, n))
    if policy == O.PER_TOKEN:
        v = rng.uniform(lo, hi, m).astype(np.float32)
        return v, np.broadcast_to(v[:, None], (m, n))
    v = rng.uniform(lo, hi, ((m + g - 1) // g, n)).astype(np.float32)
    return v, v[np.arange(m) // g]


@pytest.mark.parametrize("policy", [O.PER_TENSOR, O.PER_CHANNEL, O.PER_TOKEN, O.PER_GROUP])
@pytest.mark.parametrize("mode", [O.ROUND_RINT, O.ROUND_FLOOR, O.ROUND_ROUND])
def test_quantize_int8_vs_numpy(policy, mode):
    """int8 Quantize for every policy: numpy float32 x * s, then + o, the round mode and saturation; the scale and
    offset indexed per policy (PER_GROUP with kDim 0: one row of scales per group of rows)"""
    rng = np.random.default_rng(1300 + 10 * policy + mode)
    m, n, g = 70, 96, 32
    x = rng.uniform(-200.0, 200.0, (m, n)).astype(np.float32)
    s, S = _policy_tables(rng, policy, m, n, g, 0.05, 1.5)
    o, Of = _policy_tables(rng, policy, m, n, g, -6.0, 6.0)
    tensor = policy != O.PER_TENSOR
    got = O.quantize(x, O.F32, O.INT8, policy, m, n, scale=s if tensor else None, scale_type=O.F32,
                     offset=o if tensor else None, scale_scalar=float(s) if not tensor else 1.0,
                     offset_scalar=float(o) if not tensor else None, group=g, k_dim=0, round_mode=mode)
    y = (x * S) + Of
    assert np.array_equal(got, _sat_s8(y.astype(np.float64), mode))


@pytest.mark.parametrize("dst", [O.INT8, O.HIF8, O.FP8_E4M3, O.FP4_E2M1])
@pytest.mark.parametrize("st", [O.F16, O.BF16])
def test_quantize_16bit_scale_widened_to_fp32(dst, st):
    """Quantize with a half / bf16 source, scale and offset computes in fp32 (the scale and offset widened exactly,
    quantize_impl.h:262-294): it equals the AscendQuant policy form given the same scale and offset as f32 values (the
    form that computes in fp32), and for int8 differs from that form's own 16-bit arithmetic on this data"""
    rng = np.random.default_rng(1400 + dst + 7 * st)
    m, n, g = 64, 128, 32
    col = (n + g - 1) // g
    x = rng.uniform(-150.0, 150.0, (m, n))
    sc = rng.uniform(0.05, 1.9, (m, col))
    of = rng.uniform(-4.0, 4.0, (m, col))
    if dst == O.FP4_E2M1:
        x, sc = x / 40.0, sc
    bits = (lambda a: a.astype(np.float16).view(np.uint16)) if st == O.F16 else _bf16_bits
    vals = (lambda b: b.view(np.float16).astype(np.float32)) if st == O.F16 else _bf16_vals
    xb, sb, ob = bits(x), bits(sc), bits(of)
    got = O.quantize(xb, st, dst, O.PER_GROUP, m, n, scale=sb, scale_type=st, offset=ob, group=g, k_dim=1)
    ref = O.quant_policy(xb, st, vals(sb).astype(np.float32), O.F32, dst, O.PER_GROUP, m, n, g,
                         offset=vals(ob).astype(np.float32), k_dim=1)
    assert np.array_equal(got, ref)
    if dst == O.INT8:
        own = O.quant_policy(xb, st, sb, st, dst, O.PER_GROUP, m, n, g, offset=ob, k_dim=1)
        assert not np.array_equal(got, own)


def test_quantize_per_channel_is_one_group_of_rows():
    """PER_CHANNEL (scale[c]) is PER_GROUP with kDim 0 and a single group spanning every row; PER_TENSOR is PER_TOKEN
    with every row's scale equal -- both to hifloat8 and fp8 outputs as well"""
    rng = np.random.default_rng(1500)
    m, n = 40, 64
    x = rng.uniform(-3000.0, 3000.0, (m, n)).astype(np.float32)
    s = rng.uniform(0.01, 3.0, n).astype(np.float32)
    o = rng.uniform(-9.0, 9.0, n).astype(np.float32)
    for dst in (O.INT8, O.HIF8, O.FP8_E5M2):
        a = O.quantize(x, O.F32, dst, O.PER_CHANNEL, m, n, scale=s, offset=o)
        b = O.quant_policy(x, O.F32, s[None, :], O.F32, dst, O.PER_GROUP, m, n, 64, offset=o[None, :], k_dim=0)
        assert np.array_equal(a, b)
        t = O.quantize(x, O.F32, dst, O.PER_TENSOR, m, n, scale_scalar=0.75, offset_scalar=-1.25)
        u = O.quant_policy(x, O.F32, np.full(m, 0.75, np.float32), O.F32, dst, O.PER_TOKEN, m, n,
                           offset_scalar=-1.25)
        assert np.array_equal(t, u)


@pytest.mark.parametrize("policy", [O.PER_TENSOR, O.PER_CHANNEL, O.PER_TOKEN, O.PER_GROUP])
def test_dequantize_vs_numpy(policy):
    """Dequantize: f32(src) * scale, one cast: PER_TENSOR a bf16 scalar to bf16, PER_CHANNEL a bf16 tensor to f32,
    PER_TOKEN / PER_GROUP (kDim 1) f32 scales to f16 (int32 values below 2^24: the conversion is exact)"""
    rng = np.random.default_rng(1600 + policy)
    m, n, g = 48, 64, 32
    src = rng.integers(-(1 << 20), 1 << 20, (m, n)).astype(np.int32)
    if policy == O.PER_TENSOR:
        sv = _bf16_vals(_bf16_bits(np.array([0.0123], np.float32)))[0]
        y = O.dequantize(src, O.INT32, O.BF16, policy, scale_scalar=0.0123, scale_type=O.BF16)
        exp = _bf16_sat(src.astype(np.float32) * np.float32(sv))
    elif policy == O.PER_CHANNEL:
        sb = _bf16_bits(rng.uniform(-0.01, 0.01, n).astype(np.float32))
        y = O.dequantize(src, O.INT32, O.F32, policy, scale=sb, scale_type=O.BF16)
        exp = src.astype(np.float32) * _bf16_vals(sb)[None, :]
    else:
        shape = (m,) if policy == O.PER_TOKEN else (m, n // g)
        s = rng.uniform(-1e-3, 1e-3, shape).astype(np.float32)
        y = O.dequantize(src, O.INT32, O.F16, policy, scale=s, scale_type=O.F32, group=g, k_dim=1)
        S = s[:, None] if policy == O.PER_TOKEN else s[:, np.arange(n) // g]
        exp = _f16_sat(src.astype(np.float32) * S)
    assert np.array_equal(y.view(np.uint32) if y.dtype == np.float32 else y,
                          exp.view(np.uint32) if exp.dtype == np.float32 else exp)


@pytest.mark.parametrize("policy", [O.PER_TENSOR, O.PER_CHANNEL, O.PER_TOKEN, O.PER_GROUP])
@pytest.mark.parametrize("src_type", [O.INT8, O.FP8_E4M3])
def test_antiquantize_vs_numpy(policy, src_type):
    """AntiQuantize: fp32 (src + o) * s and one cast for every policy, also with half scales (PER_TENSOR /
    PER_CHANNEL take scales of the dst type; PER_TOKEN / PER_GROUP here f16 scales to f16 and f32 scales to bf16)"""
    rng = np.random.default_rng(1700 + 10 * policy + src_type)
    m, n, g = 40, 96, 32
    if src_type == O.INT8:
        q = rng.integers(-128, 128, (m, n)).astype(np.int8)
        xv = q.astype(np.float32)
    else:
        q = fp8_bytes(rng, (m, n), O.FP8_E4M3)
        xv = torch.from_numpy(q).view(torch.float8_e4m3fn).float().numpy()
    for st, dt in ((O.F16, O.F16), (O.F32, O.BF16)):
        if st == O.F32 and policy in (O.PER_TENSOR, O.PER_CHANNEL):
            st, dt = O.BF16, O.BF16
        s, S = _policy_tables(rng, policy, m, n, g, 0.01, 2.0)
        o, Of = _policy_tables(rng, policy, m, n, g, -30.0, 30.0)
        if st == O.F16:
            s, S, o, Of = [np.asarray(a).astype(np.float16) for a in (s, S, o, Of)]
            sa, oa = (np.asarray(s).view(np.uint16), np.asarray(o).view(np.uint16))
        elif st == O.BF16:
            sa, oa = _bf16_bits(np.atleast_1d(s)), _bf16_bits(np.atleast_1d(o))
            S = _bf16_vals(_bf16_bits(np.ascontiguousarray(S, np.float32)))
            Of = _bf16_vals(_bf16_bits(np.ascontiguousarray(Of, np.float32)))
        else:
            sa, oa = s, o
        tensor = policy != O.PER_TENSOR
        y = O.antiquantize(q, src_type, dt, policy, m, n, scale=sa if tensor else None, scale_type=st,
                           offset=oa if tensor else None,
                           scale_scalar=1.0 if tensor else float(np.asarray(S).reshape(-1)[0]),
                           offset_scalar=None if tensor else float(np.asarray(Of).reshape(-1)[0]), group=g, k_dim=0)
        v = (xv + np.asarray(Of, np.float32)) * np.asarray(S, np.float32)
        exp = _f16_sat(v) if dt == O.F16 else _bf16_sat(v)
        assert np.array_equal(y, exp), (policy, st)
