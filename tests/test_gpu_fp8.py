"""GPU parity: fp8 operand Matmul (e4m3fn / e5m2, QF322{F16,BF16,F32}_PRE epilogue, f32 bias) and MX-FP8
(fp8 elements, E8M0 per 32 K) through the C ABI, vs the oracle's fp64 sums.

Tolerance.  v_mfma_f32_32x32x64_f8f6f4 sums the fp8 products of each group of 16 consecutive K (one register
quad of one lane) aligned to the group's largest product and truncated toward zero at 2^(e_max - 13)
(measured with two-term probes: a second product below that step is dropped within a group and kept exactly
across groups and k-steps; every fp8 code decodes exactly).  So per element, with v = (s + bias) * M1 from the
oracle's fp64 sum,
    |out - v| <= 0.5 ulp_out(|v| + d) + d,
    d = (2^-8 * sum_groups max_group |a b| + K * 2^-24 * (sum |a b| + |bias|)) * |M1|
(16 products lose less than one 2^(e_max - 13) step each, 2^-9 of the group maximum, doubled to cover a
32-product group; groups and the bias are combined in fp32), and normwise ||out - v|| / ||v|| <= eps_out +
2^-12 (measured ~5e-5; one misplaced element costs ~max |a b|, 256x the per-group term, a dropped k-step tens
of percent).  The reference's own check of the fp8 sample is np.isclose(rtol = atol = 1e-3)
against a fp32 TensorFlow golden with error ratio <= 1e-3 (matmul_fp8/scripts/verify_result.py:20-40); that
check is applied too on the sample's shape."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded
from test_oracle import fp8_bytes, torch_decode

pytestmark = pytest.mark.gpu

_TORCH_OUT = {O.F16: torch.float16, O.BF16: torch.bfloat16, O.F32: torch.float32}
_EPS = {O.F16: 2.0 ** -11, O.BF16: 2.0 ** -8, O.F32: 0.0}
_ULP_BITS = {O.F16: 10, O.BF16: 7, O.F32: 23}
_MIN_EXP = {O.F16: -14, O.BF16: -126, O.F32: -126}


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _ulp(v, out_type):
    a = np.maximum(np.abs(v), 2.0 ** _MIN_EXP[out_type])
    return 2.0 ** (np.floor(np.log2(a)) - _ULP_BITS[out_type])


def check_out(got, v, d, out_type, what=""):
    tol = 0.5 * _ulp(np.abs(v) + d, out_type) + d
    err = np.abs(got - v)
    bad = err > tol
    assert not bad.any(), f"{what}: {bad.sum()} elements outside the bound; first {np.argwhere(bad)[:3].tolist()}"
    nv = np.linalg.norm(v)
    if nv > 0:
        r = np.linalg.norm(got - v) / nv
        assert r <= _EPS[out_type] + 2.0 ** -12, f"{what}: normwise error {r}"


def run_fp8(ascq, A, B, fa, fb, M, N, K, out_type, trans_a=False, trans_b=False, bias=None, qscalar=None,
            qvec=None, single=None):
    mm = ascq.Matmul(fa, fb, out_type, ascq.F32 if bias is not None else 0)
    mm.SetOrgShape(M, N, K)
    if single is not None:
        mm.SetSingleShape(*single)
    mm.SetTensorA(_dev(A), trans_a)
    mm.SetTensorB(_dev(B), trans_b)
    if bias is not None:
        mm.SetBias(_dev(bias))
    if qvec is not None:
        mm.SetQuantVector(_dev(qvec.view(np.int64)))
    elif qscalar is not None:
        mm.SetQuantScalar(int(qscalar))
    c = torch.full((M, N), float("nan"), dtype=_TORCH_OUT[out_type], device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    return c.cpu().to(torch.float64).numpy()


def signed_codes(rng, shape, fmt, hi):
    """fp8 codes with magnitude code < hi and a random sign"""
    c = fp8_bytes(rng, shape, fmt, 0, hi)
    return (c | (rng.integers(0, 2, shape) * 128).astype(np.uint8)).astype(np.uint8)


def fp8_case(seed, M, N, K, fa, fb, out_type, trans_a=False, trans_b=False, bias=True, quant="none", hi=128):
    """hi bounds the magnitude codes: 0x40 keeps both formats below 2 (f16 outputs stay in range); 128 is the
    full range"""
    rng = seeded(seed)
    A = signed_codes(rng, (K, M) if trans_a else (M, K), fa, hi)
    B = signed_codes(rng, (N, K) if trans_b else (K, N), fb, hi)
    b = rng.standard_normal(N).astype(np.float32) * 4 if bias else None
    words = np.array([O.lib().oq_pack_quant_pre(float(x), 0, 0) for x in rng.uniform(2.0 ** -6, 2.0 ** -2, N)],
                     np.uint64)
    qs = qv = None
    if quant == "scalar":
        qs = int(words[0])
    elif quant == "vector":
        qv = words
    return A, B, b, qs, qv


def expected(A, B, fa, fb, b, qs, qv, trans_a, trans_b, K):
    _, exact, absd, bmax = O.matmul_fp8(A, B, fa, fb, bias=b, trans_a=trans_a, trans_b=trans_b)
    m1 = np.ones(exact.shape[1])
    if qv is not None:
        m1 = (qv & np.uint64(0xFFFFE000)).astype(np.uint32).view(np.float32).astype(np.float64)
    elif qs is not None:
        m1 = np.full(exact.shape[1], float(np.array([qs & 0xFFFFE000], np.uint32).view(np.float32)[0]))
    babs = np.zeros(exact.shape[1]) if b is None else np.abs(b.astype(np.float64))
    v = exact * m1[None, :]
    d = (2.0 ** -8 * bmax + K * 2.0 ** -24 * (absd + babs[None, :])) * np.abs(m1)[None, :]
    return v, d


FORMATS = [(O.FP8_E4M3, O.FP8_E4M3), (O.FP8_E5M2, O.FP8_E5M2), (O.FP8_E4M3, O.FP8_E5M2), (O.FP8_E5M2, O.FP8_E4M3)]


@pytest.mark.parametrize("fa,fb", FORMATS)
@pytest.mark.parametrize("M,N,K", [(428, 479, 158), (428, 480, 160)])
def test_fp8_sample_shape(ascq_gpu, fa, fb, M, N, K):
    """the reference sample (matmul_fp8.asc, gen_data.py): M=428, N=479, K=158, uniform(-1, 1) cast to fp8,
    f32 bias, f32 C, the four fp8 scenarios.  K % 16 != 0 takes the element-wise kernel; the same data at
    N = 480, K = 160 takes the MFMA kernel"""
    rng = seeded(100 + fa * 16 + fb)
    T = {O.FP8_E4M3: torch.float8_e4m3fn, O.FP8_E5M2: torch.float8_e5m2}
    A = torch.from_numpy(rng.uniform(-1, 1, (M, K)).astype(np.float32)).to(T[fa]).view(torch.uint8).numpy()
    B = torch.from_numpy(rng.uniform(-1, 1, (K, N)).astype(np.float32)).to(T[fb]).view(torch.uint8).numpy()
    b = rng.uniform(-1, 1, N).astype(np.float32)
    got = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, O.F32, bias=b)
    v, d = expected(A, B, fa, fb, b, None, None, False, False, K)
    check_out(got, v, d, O.F32, "sample")
    # verify_result.py: isclose(rtol=1e-3, atol=1e-3) against the fp32 golden, error ratio <= 1e-3
    golden = (torch_decode(A, fa).astype(np.float32) @ torch_decode(B, fb).astype(np.float32) + b).astype(np.float32)
    bad = ~np.isclose(got, golden, rtol=1e-3, atol=1e-3)
    assert bad.mean() <= 1e-3


@pytest.mark.parametrize("fa,fb", FORMATS)
@pytest.mark.parametrize("out_type", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("quant", ["none", "scalar", "vector"])
def test_fp8_tiled_small(ascq_gpu, fa, fb, out_type, quant):
    """64 x 64 / 64 x 128 tiles, ragged M / N, both B layouts, K not a multiple of 64"""
    M, N, K = 200, 136, 208
    for trans_b in (True, False):
        # f16 C: magnitudes below 2 keep the sums inside the f16 range; otherwise every code
        hi = 0x40 if out_type == O.F16 else 128
        A, B, b, qs, qv = fp8_case(7, M, N, K, fa, fb, out_type, trans_b=trans_b, quant=quant, hi=hi)
        got = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, out_type, trans_b=trans_b, bias=b, qscalar=qs, qvec=qv)
        v, d = expected(A, B, fa, fb, b, qs, qv, False, trans_b, K)
        check_out(got, v, d, out_type, f"trans_b={trans_b}")


@pytest.mark.parametrize("out_type", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("M,N,K", [(1, 200, 512), (1, 208, 512), (16, 136, 1024), (29, 96, 256), (40, 304, 768),
                                   (64, 1100, 2048), (64, 1104, 2048), (1, 4096, 8192), (16, 12400, 768)])
def test_fp8_decode_ksplit(ascq_gpu, out_type, trans_b, M, N, K):
    """decode-sized batches with K % 256 == 0: 32 x 32 tiles whose K is split over four waves (fp32 partials added
    in one fixed order), B given [N, K], or [K, N] with N % 16 == 0 (its K rows staged like A's and read by LDS
    transpose reads; other N take the general tiles); with B given [K, N] and long K or wide N (the last two shapes)
    32 x 128 tiles whose K is split across workgroups too, the fp32 partials added in split order by a second
    launch.  Ragged N, bias and per-channel scales; a second call returns the same bits"""
    fa, fb = O.FP8_E4M3, O.FP8_E5M2
    hi = 0x40 if out_type == O.F16 else 128
    A, B, b, qs, qv = fp8_case(31 + M, M, N, K, fa, fb, out_type, trans_b=trans_b, quant="vector", hi=hi)
    got = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, out_type, trans_b=trans_b, bias=b, qvec=qv)
    v, d = expected(A, B, fa, fb, b, qs, qv, False, trans_b, K)
    check_out(got, v, d, out_type, f"M={M}")
    again = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, out_type, trans_b=trans_b, bias=b, qvec=qv)
    assert np.array_equal(np.nan_to_num(got, nan=7.0), np.nan_to_num(again, nan=7.0))


@pytest.mark.parametrize("M,N,K", [(100, 1104, 512), (300, 272, 1040), (64, 11008, 4096), (65, 160, 208)])
def test_fp8_kn_b_transposed_reads(ascq_gpu, M, N, K):
    """B given [K, N] with 16-byte K rows below the sizes where the host transposes it: the 64 x 128 tiles stage B's
    K rows like A's and read them with LDS transpose reads (an fp8 k-step = two int8-sized transposed reads); K not
    a multiple of 64 among them (the last stage's rows past K read zeros)"""
    fa, fb = O.FP8_E5M2, O.FP8_E4M3
    A, B, b, qs, qv = fp8_case(41 + M, M, N, K, fa, fb, O.BF16, trans_b=False, quant="vector")
    got = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, O.BF16, trans_b=False, bias=b, qvec=qv)
    v, d = expected(A, B, fa, fb, b, qs, qv, False, False, K)
    check_out(got, v, d, O.BF16, f"M={M}")


@pytest.mark.parametrize("fa,fb", [(O.FP8_E4M3, O.FP8_E4M3), (O.FP8_E5M2, O.FP8_E4M3)])
@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (1100, 1040, 1040), (2048, 1280, 512)])
def test_fp8_tiled_big(ascq_gpu, fa, fb, M, N, K):
    """256 x 256 tiles: 128-byte stages (K % 128 == 0) and 64-byte stages; [K, N] B is transposed first"""
    for trans_b in (True, False):
        A, B, b, qs, qv = fp8_case(11, M, N, K, fa, fb, O.BF16, trans_b=trans_b, quant="vector")
        got = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, O.BF16, trans_b=trans_b, bias=b, qvec=qv)
        v, d = expected(A, B, fa, fb, b, qs, qv, False, trans_b, K)
        check_out(got, v, d, O.BF16, f"{M}x{N}x{K} trans_b={trans_b}")


@pytest.mark.parametrize("M,N,K", [(96, 80, 64), (600, 1100, 256)])
def test_fp8_trans_a(ascq_gpu, M, N, K):
    """isTransA: A given [K, M] is transposed into the workspace, then the tiled kernel runs"""
    fa, fb = O.FP8_E4M3, O.FP8_E5M2
    A, B, b, qs, qv = fp8_case(13, M, N, K, fa, fb, O.F32, trans_a=True, trans_b=True, quant="scalar")
    got = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, O.F32, trans_a=True, trans_b=True, bias=b, qscalar=qs)
    v, d = expected(A, B, fa, fb, b, qs, qv, True, True, K)
    check_out(got, v, d, O.F32, "trans_a")


def test_fp8_single_shape_block(ascq_gpu):
    """SetSingleShape: a sub-block of the org shape (leading dimensions from the org shape)"""
    M, N, K = 300, 260, 192
    fa = fb = O.FP8_E4M3
    A, B, b, qs, qv = fp8_case(17, M, N, K, fa, fb, O.F32, quant="none", bias=False)
    sm, sn, sk = 130, 100, 128
    got = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, O.F32, single=(sm, sn, sk))
    v, d = expected(np.ascontiguousarray(A[:sm, :sk]), np.ascontiguousarray(B[:sk, :sn]), fa, fb, None, None, None,
                    False, False, sk)
    check_out(got[:sm, :sn], v, d, O.F32, "single shape")
    assert np.isnan(got[sm:, :]).all() and np.isnan(got[:, sn:]).all()


# --------------------------------------------------------------------------- MX-FP8
def mx_fp8_inputs(rng, M, N, K, fa, fb, trans_b):
    sK = (K + 63) // 64 * 2
    A = fp8_bytes(rng, (M, K), fa)
    B = fp8_bytes(rng, (N, K) if trans_b else (K, N), fb)
    sA = rng.integers(118, 136, (M, sK), dtype=np.uint8)
    sB = rng.integers(118, 136, (N, sK), dtype=np.uint8)  # [N, sK]
    return A, B, sA, sB


def mx_bound(absd, bmax, K):
    """the fp8 block alignment term plus fp32 accumulation (the block scales multiply whole blocks)"""
    return 2.0 ** -8 * bmax + K * 2.0 ** -24 * absd


def pairs(s_rows):
    """[R, sK] -> [sK/2, R, 2] (the sample's pair layout)"""
    R, sK = s_rows.shape
    return np.ascontiguousarray(s_rows.T.reshape(sK // 2, 2, R).transpose(0, 2, 1))


def run_mx_fp8(ascq, A, B, sA, sB, fa, fb, M, N, K, trans_b, sa_t, sb_t, c_type):
    mm = ascq.Matmul(fa, fb, c_type, 0, ascq.E8M0)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B), trans_b)
    mm.SetTensorScaleA(_dev(sA), sa_t)
    mm.SetTensorScaleB(_dev(sB), sb_t)
    c = torch.empty((M, N), dtype=_TORCH_OUT[c_type], device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    return c.cpu().to(torch.float64).numpy()


def test_mx_fp8_sample_shape(ascq_gpu):
    """matmul_mx.asc:90-244: M=32, N=128, K=128, e5m2 elements, E8M0 scales, fp32 C"""
    M, N, K = 32, 128, 128
    fa = fb = O.FP8_E5M2
    A, B, sA, sB = mx_fp8_inputs(seeded(21), M, N, K, fa, fb, False)
    got = run_mx_fp8(ascq_gpu, A, B, sA, pairs(sB), fa, fb, M, N, K, False, 0, 0, O.F32)
    _, Ce, Ca, Cb = O.mx_matmul(A, B, sA, pairs(sB), M, N, K, trans_b=False, sa_layout=0, sb_layout=0, elem_fmt=fa,
                                fmt_b=fb, blockmax=True)
    check_out(got, Ce, mx_bound(Ca, Cb, K), O.F32, "mx sample")


@pytest.mark.parametrize("fa,fb", FORMATS)
@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("sa_t,sb_t", [(0, 0), (1, 1)])
def test_mx_fp8_small(ascq_gpu, fa, fb, trans_b, sa_t, sb_t):
    M, N, K = 96, 200, 320
    A, B, sA, sB = mx_fp8_inputs(seeded(23), M, N, K, fa, fb, trans_b)
    sA_in = pairs(sA) if sa_t else sA       # isTransposeScaleA: [sK/2, M, 2]
    sB_in = sB if sb_t else pairs(sB)       # isTransposeScaleB: [N, sK]; default pairs [sK/2, N, 2]
    got = run_mx_fp8(ascq_gpu, A, B, sA_in, sB_in, fa, fb, M, N, K, trans_b, sa_t, sb_t, O.BF16)
    _, Ce, Ca, Cb = O.mx_matmul(A, B, sA, sB, M, N, K, trans_b=trans_b, sa_layout=0, sb_layout=1, elem_fmt=fa,
                                fmt_b=fb, blockmax=True)
    check_out(got, Ce, mx_bound(Ca, Cb, K), O.BF16, "mx small")


@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("M,N,K", [(1, 200, 512), (40, 136, 384), (64, 96, 1024)])
def test_mx_fp8_decode(ascq_gpu, trans_b, M, N, K):
    """decode-sized batches (M <= 64, a single row among them), both B layouts"""
    fa, fb = O.FP8_E4M3, O.FP8_E5M2
    A, B, sA, sB = mx_fp8_inputs(seeded(29 + M), M, N, K, fa, fb, trans_b)
    got = run_mx_fp8(ascq_gpu, A, B, sA, pairs(sB), fa, fb, M, N, K, trans_b, 0, 0, O.BF16)
    _, Ce, Ca, Cb = O.mx_matmul(A, B, sA, pairs(sB), M, N, K, trans_b=trans_b, sa_layout=0, sb_layout=0, elem_fmt=fa,
                                fmt_b=fb, blockmax=True)
    check_out(got, Ce, mx_bound(Ca, Cb, K), O.BF16, "mx decode")


@pytest.mark.parametrize("fa,fb", [(O.FP8_E4M3, O.FP8_E4M3), (O.FP8_E4M3, O.FP8_E5M2)])
@pytest.mark.parametrize("M,N,K", [(1024, 1024, 512), (1100, 1300, 448)])
def test_mx_fp8_big(ascq_gpu, fa, fb, M, N, K):
    """256 x 256 tiles with 64-byte stages; ragged M / N, K % 128 == 64"""
    rng = seeded(29)
    A, B, sA, sB = mx_fp8_inputs(rng, M, N, K, fa, fb, True)
    rows = np.sort(rng.choice(M, 48, replace=False)).astype(np.int64)
    got = run_mx_fp8(ascq_gpu, A, B, sA, pairs(sB), fa, fb, M, N, K, True, 0, 0, O.F32)
    _, Ce, Ca, Cb = O.mx_matmul(A, B, sA, sB, M, N, K, trans_b=True, sa_layout=0, sb_layout=1, elem_fmt=fa, fmt_b=fb,
                                rows=rows, blockmax=True)
    check_out(got[rows], Ce[rows], mx_bound(Ca[rows], Cb[rows], K), O.F32, "mx big")
