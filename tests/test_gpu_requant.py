"""GPU parity: the requant epilogues of the Matmul through the C ABI.

  * int8 A / B with int8 / uint8 C: (V)REQ8 -- bit-exact against the oracle (int32 sums are exact on both sides),
    and against the reference's golden (asc_copy_l0c2gm gen_data_s322s8.py, seed 9);
  * fp8 A / B with int8 / uint8 C: (V)QF322B8_PRE; fp8 C: (V)QF322FP8_PRE.  The fp32 accumulator carries the fp8
    MFMA's group-alignment error (test_gpu_fp8.py), so each output must lie between the epilogue applied to the
    low and the high end of the oracle's interval [s - d, s + d] (the epilogues are monotone), and outside those
    boundary cases it must equal the oracle's output (and overall at least 97 % do); the doc example
    (asc_set_l0c_copy_prequant.md: identity, scale 2, offset 3) is exact.
Words carry random M1, 9-bit offsets (0..511) and sign flags per column; bits 32-36 are set in some words and
must be ignored."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded
from test_oracle import fp8_bytes

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def words_for(rng, n, lo=2.0 ** -8, hi=2.0 ** -2, extra_bits=True):
    m1 = rng.uniform(lo, hi, n).astype(np.float32)
    off = rng.integers(0, 512, n)
    off[: n // 2] = rng.integers(0, 8, n // 2)  # half the columns with small offsets (no blanket saturation)
    sign = rng.integers(0, 2, n)
    w = np.array([O.lib().oq_pack_quant_pre(float(a), int(o), int(s)) for a, o, s in zip(m1, off, sign)], np.uint64)
    if extra_bits:
        w |= (rng.integers(0, 32, n).astype(np.uint64) << np.uint64(32))
    return w


def run(ascq, a_t, b_t, c_t, A, B, M, N, K, trans_b=False, bias=None, qvec=None, qscalar=None, bias_t=0):
    mm = ascq.Matmul(a_t, b_t, c_t, bias_t if bias is not None else 0)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B), trans_b)
    if bias is not None:
        mm.SetBias(_dev(bias))
    if qvec is not None:
        mm.SetQuantVector(_dev(qvec.view(np.int64)))
    else:
        mm.SetQuantScalar(int(qscalar))
    c = torch.full((M, N), 0x5A, dtype=torch.uint8, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    return c.cpu().numpy()


# --------------------------------------------------------------------------- REQ8 (int8 operands)
@pytest.mark.parametrize("c_type", ["INT8", "UINT8"])
def test_req8_golden_seed9(ascq_gpu, c_type):
    f = np.load(GOLD / "req8_seed9.npz")
    M, K = f["x1"].shape
    N = f["x2"].shape[1]
    w = int(f["quant_word"][0])
    got = run(ascq_gpu, ascq_gpu.INT8, ascq_gpu.INT8, getattr(ascq_gpu, c_type), f["x1"], f["x2"], M, N, K, qscalar=w)
    assert np.array_equal(got.view(np.int8), f["golden"])
    qv = np.full(N, w, np.uint64)
    got = run(ascq_gpu, ascq_gpu.INT8, ascq_gpu.INT8, getattr(ascq_gpu, c_type), f["x1"], f["x2"], M, N, K, qvec=qv)
    assert np.array_equal(got.view(np.int8), f["golden"])


@pytest.mark.parametrize("M,N,K", [(200, 136, 208), (64, 64, 64), (1100, 1040, 1040), (1024, 2048, 512), (37, 19, 53)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_req8_vs_oracle(ascq_gpu, M, N, K, trans_b):
    rng = seeded(M * 7 + N * 3 + K + trans_b)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (N, K) if trans_b else (K, N)).astype(np.int8)
    bias = rng.integers(-(1 << 16), 1 << 16, N).astype(np.int32)
    acc = O.matmul_i8(A, B, bias=bias, trans_b=trans_b)
    qv = words_for(rng, N, 2.0 ** -14, 2.0 ** -9)  # |acc| up to ~K * 2^14: map into the int8 range
    got = run(ascq_gpu, ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.INT8, A, B, M, N, K, trans_b, bias, qvec=qv,
              bias_t=ascq_gpu.INT32)
    exp = O.mm_requant(acc, qvec=qv)
    assert np.array_equal(got, exp), f"{(got != exp).sum()} mismatches"
    ws = int(qv[3])
    got = run(ascq_gpu, ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.UINT8, A, B, M, N, K, trans_b, bias, qscalar=ws,
              bias_t=ascq_gpu.INT32)
    assert np.array_equal(got, O.mm_requant(acc, qscalar=ws))


# --------------------------------------------------------------------------- QF322B8 / QF322FP8 (fp8 operands)
def fp8_inputs(rng, M, N, K, fa, fb, trans_b):
    A = fp8_bytes(rng, (M, K), fa, 0, 0x40) | (rng.integers(0, 2, (M, K)) * 128).astype(np.uint8)
    B = fp8_bytes(rng, (N, K) if trans_b else (K, N), fb, 0, 0x40)
    B = B | (rng.integers(0, 2, B.shape) * 128).astype(np.uint8)
    return A.astype(np.uint8), B.astype(np.uint8)


def requant_np(v, words):
    off = ((words >> np.uint64(37)) & np.uint64(0x1FF)).astype(np.float64)
    sign = ((words >> np.uint64(46)) & np.uint64(1)).astype(bool)
    t = np.round(np.clip(np.nan_to_num(v, nan=0.0), -256, 255)) + off[None, :]
    return np.where(sign[None, :], np.clip(t, -128, 127), np.clip(t, 0, 255))


def as_value(bytes_, words):
    """output bytes (uint8 storage) as numbers: int8 in columns whose word has the sign flag, else uint8"""
    sign = ((words >> np.uint64(46)) & np.uint64(1)).astype(bool)
    return np.where(sign[None, :], bytes_.view(np.int8).astype(np.float64), bytes_.astype(np.float64))


def fp8_encode_np(v, fmt):
    """torch's rne cast with the fixpipe's e4m3 saturation (+-448, NaN -> 0); e5m2 overflows to inf"""
    t = torch.from_numpy(np.ascontiguousarray(v, np.float32))
    if fmt == O.FP8_E4M3:
        t = torch.nan_to_num(t, nan=0.0).clamp(-448.0, 448.0)
        return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return t.to(torch.float8_e5m2).view(torch.uint8).numpy()


def fp8_value(codes, fmt):
    dt = torch.float8_e4m3fn if fmt == O.FP8_E4M3 else torch.float8_e5m2
    return torch.from_numpy(np.ascontiguousarray(codes)).view(dt).to(torch.float64).numpy()


@pytest.mark.parametrize("M,N,K", [(16, 16, 16), (200, 136, 208), (1100, 1040, 1040)])
@pytest.mark.parametrize("out", ["INT8", "FP8_E4M3", "FP8_E5M2"])
def test_fp8_requant_vs_oracle(ascq_gpu, M, N, K, out):
    fa, fb = O.FP8_E4M3, O.FP8_E5M2
    rng = seeded(M + N + K + len(out))
    trans_b = M > 512
    A, B = fp8_inputs(rng, M, N, K, fa, fb, trans_b)
    bias = rng.standard_normal(N).astype(np.float32)
    lo_m1, hi_m1 = (2.0 ** -2, 2.0 ** 2) if out == "INT8" else (2.0 ** -4, 2.0 ** 6)
    qv = words_for(rng, N, lo_m1, hi_m1)
    o_t = getattr(O, out)
    exp, exact, absd, bmax = O.matmul_fp8(A, B, fa, fb, bias=bias, out_type=o_t, trans_b=trans_b, use_q=True, qvec=qv)
    got = run(ascq_gpu, ascq_gpu.FP8_E4M3, ascq_gpu.FP8_E5M2, getattr(ascq_gpu, out), A, B, M, N, K, trans_b, bias,
              qvec=qv, bias_t=ascq_gpu.F32)
    m1 = (qv & np.uint64(0xFFFFE000)).astype(np.uint32).view(np.float32).astype(np.float64)
    d = 2.0 ** -8 * bmax + K * 2.0 ** -24 * (absd + np.abs(bias)[None, :].astype(np.float64))
    v_lo, v_hi = (exact - d) * m1[None, :], (exact + d) * m1[None, :]
    if out == "INT8":
        g = as_value(got, qv)
        lo, hi = requant_np(v_lo, qv), requant_np(v_hi, qv)
        e = as_value(exp.view(np.uint8), qv)  # the oracle returns int8 storage; the words pick the sign
    else:
        g = fp8_value(got, o_t)
        lo, hi = fp8_value(fp8_encode_np(v_lo, o_t), o_t), fp8_value(fp8_encode_np(v_hi, o_t), o_t)
        e = fp8_value(exp, o_t)
    assert ((g >= lo) & (g <= hi)).all(), f"{(~((g >= lo) & (g <= hi))).sum()} outputs outside the interval"
    settled = lo == hi
    assert np.array_equal(g[settled], e[settled])
    # the measured fp8 error is ~20x below d: almost every output equals the oracle's
    assert (g == e).mean() > 0.97, f"only {(g == e).mean():.4f} equal to the oracle"


def test_prequant_doc_example_fp8(ascq_gpu):
    """asc_set_l0c_copy_prequant.md: identity x identity, scale 2, offset 3, signed int8 -> 5 / 3"""
    A = np.zeros((16, 16), np.uint8)
    np.fill_diagonal(A, 0x38)  # e4m3 1.0
    w = int(O.lib().oq_pack_quant_pre(2.0, 3, 1))
    got = run(ascq_gpu, ascq_gpu.FP8_E4M3, ascq_gpu.FP8_E4M3, ascq_gpu.INT8, A, A, 16, 16, 16, qscalar=w)
    exp = np.full((16, 16), 3, np.int8)
    np.fill_diagonal(exp, 5)
    assert np.array_equal(got.view(np.int8), exp)


def test_requant_needs_quant_word(ascq_gpu):
    """int8 / fp8 C without SetQuantScalar / SetQuantVector is a state error, as for f16 C"""
    mm = ascq_gpu.Matmul(ascq_gpu.FP8_E4M3, ascq_gpu.FP8_E4M3, ascq_gpu.INT8)
    mm.SetOrgShape(16, 16, 16)
    a = torch.zeros((16, 16), dtype=torch.uint8, device="cuda")
    mm.SetTensorA(a)
    mm.SetTensorB(a)
    with pytest.raises(ascq_gpu.AscqError):
        mm.IterateAll(torch.empty((16, 16), dtype=torch.uint8, device="cuda"))


# --------------------------------------------------------------------------- REQ4 / QF322S4 (int4 C)
def words4(rng, n, lo, hi):
    """QUANT_PRE words for int4 output: M1 log-uniform in [lo, hi], offsets 0..3 (a larger offset saturates every
    output at 7), random sign flags (ignored by the int4 modes), bits 32-36 set at random"""
    m1 = np.exp(rng.uniform(np.log(lo), np.log(hi), n)).astype(np.float32)
    off = rng.integers(0, 4, n)
    sign = rng.integers(0, 2, n)
    w = np.array([O.lib().oq_pack_quant_pre(float(a), int(o), int(s)) for a, o, s in zip(m1, off, sign)], np.uint64)
    return w | (rng.integers(0, 32, n).astype(np.uint64) << np.uint64(32))


def run4(ascq, a_t, b_t, A, B, M, N, K, trans_b=False, bias=None, qvec=None, qscalar=None, bias_t=0):
    mm = ascq.Matmul(a_t, b_t, ascq.INT4, bias_t if bias is not None else 0)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B), trans_b)
    if bias is not None:
        mm.SetBias(_dev(bias))
    if qvec is not None:
        mm.SetQuantVector(_dev(qvec.view(np.int64)))
    else:
        mm.SetQuantScalar(int(qscalar))
    c = torch.full((M, N // 2), 0x5A, dtype=torch.uint8, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    return c.cpu().numpy()


@pytest.mark.parametrize("M,N,K", [(200, 136, 208), (64, 64, 64), (1100, 1040, 1040), (37, 18, 53)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_req4_vs_oracle(ascq_gpu, M, N, K, trans_b):
    """(V)REQ4 bit-exact: int32 sums are exact on both sides; (37, 18, 53) takes the untiled kernel"""
    rng = seeded(M * 5 + N * 11 + K + trans_b)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (N, K) if trans_b else (K, N)).astype(np.int8)
    bias = rng.integers(-(1 << 14), 1 << 14, N).astype(np.int32)
    acc = O.matmul_i8(A, B, bias=bias, trans_b=trans_b)
    qv = words4(rng, N, 2.0 ** -15, 2.0 ** -10)  # |acc| up to ~K * 2^14: spreads over the int4 range
    got = run4(ascq_gpu, ascq_gpu.INT8, ascq_gpu.INT8, A, B, M, N, K, trans_b, bias, qvec=qv, bias_t=ascq_gpu.INT32)
    exp = O.mm_requant4(acc, qvec=qv)
    assert np.array_equal(got, exp), f"{(got != exp).sum()} mismatching bytes"
    vals = O.unpack_int4(exp, N)
    assert (vals == 7).mean() < 0.5 and (vals == -8).mean() < 0.5  # not a blanket saturation
    ws = int(qv[1])
    got = run4(ascq_gpu, ascq_gpu.INT8, ascq_gpu.INT8, A, B, M, N, K, trans_b, bias, qscalar=ws, bias_t=ascq_gpu.INT32)
    assert np.array_equal(got, O.mm_requant4(acc, qscalar=ws))


@pytest.mark.parametrize("M,N,K", [(16, 16, 16), (200, 136, 208), (1100, 1040, 1040)])
def test_fp8_qf322s4_vs_oracle(ascq_gpu, M, N, K):
    """(V)QF322S4_PRE: each output lies between the mode applied to the low and the high end of the oracle's
    interval [s - d, s + d] (the fp8 MFMA's group-alignment error, test_gpu_fp8.py), equals the oracle where
    those agree, and overall at least 97 % equal it"""
    fa, fb = O.FP8_E4M3, O.FP8_E5M2
    rng = seeded(M + 3 * N + K)
    trans_b = M > 512
    A, B = fp8_inputs(rng, M, N, K, fa, fb, trans_b)
    bias = rng.standard_normal(N).astype(np.float32)
    qv = words4(rng, N, 2.0 ** -1, 2.0 ** 2)
    _, exact, absd, bmax = O.matmul_fp8(A, B, fa, fb, bias=bias, out_type=O.F32, trans_b=trans_b)
    got = O.unpack_int4(run4(ascq_gpu, ascq_gpu.FP8_E4M3, ascq_gpu.FP8_E5M2, A, B, M, N, K, trans_b, bias, qvec=qv,
                             bias_t=ascq_gpu.F32), N)
    d = 2.0 ** -8 * bmax + K * 2.0 ** -24 * (absd + np.abs(bias)[None, :].astype(np.float64))
    lo = O.unpack_int4(O.requant4_f32((exact - d).astype(np.float32), qvec=qv), N)
    hi = O.unpack_int4(O.requant4_f32((exact + d).astype(np.float32), qvec=qv), N)
    e = O.unpack_int4(O.requant4_f32(exact.astype(np.float32), qvec=qv), N)
    assert ((got >= lo) & (got <= hi)).all(), f"{(~((got >= lo) & (got <= hi))).sum()} outputs outside the interval"
    settled = lo == hi
    assert np.array_equal(got[settled], e[settled])
    assert (got == e).mean() > 0.97


def test_int4_output_needs_even_n(ascq_gpu):
    """int4 C packs two codes per byte: an odd N is an argument error, not a half-written byte"""
    mm = ascq_gpu.Matmul(ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.INT4)
    mm.SetOrgShape(16, 15, 32)
    a = torch.zeros((16, 32), dtype=torch.int8, device="cuda")
    b = torch.zeros((32, 15), dtype=torch.int8, device="cuda")
    mm.SetTensorA(a)
    mm.SetTensorB(b)
    mm.SetQuantScalar(int(O.lib().oq_pack_quant_pre(1.0, 0, 1)))
    with pytest.raises(ascq_gpu.AscqError):
        mm.IterateAll(torch.empty((16, 8), dtype=torch.uint8, device="cuda"))
