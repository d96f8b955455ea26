"""GPU parity: the hifloat8 Matmul (A and B hifloat8, the default scenario of the reference's fp8 sample,
matmul_fp8.asc:229, MatmulFp8Kernel<hifloat8_t, hifloat8_t, float, float>) and hifloat8 C ((V)QF322HIF8_PRE) through
the C ABI, against the oracle.

Both operands are decoded exactly to bf16 and multiplied on the bf16 MFMA with fp32 accumulation.  Integer-valued
data (the sample's own class: integers 0 .. 4, and -4 .. 4) gives exact sums, so every output type is compared bit
for bit.  Random codes over the whole finite range (2^-22 .. 2^15) are compared per element within
|out - v| <= 0.5 ulp_out(|v| + d) + d, d = (2^-8 * sum_groups max |a b| + K * 2^-24 * (sum |a b| + |bias|)) * |M1|,
the bound the fp8 Matmul tests use (fp32 accumulation plus an alignment term per 16-product group)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded
from test_gpu_fp8 import check_out
from test_oracle import hif8_codes, ref_verify

pytestmark = pytest.mark.gpu

_TORCH_OUT = {O.F16: torch.float16, O.BF16: torch.bfloat16, O.F32: torch.float32}


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_hif8(ascq, A, B, M, N, K, c_type, trans_a=False, trans_b=False, bias=None, qvec=None, qscalar=None,
             single=None, fa=None, fb=None):
    fa = ascq.HIF8 if fa is None else fa
    fb = ascq.HIF8 if fb is None else fb
    mm = ascq.Matmul(fa, fb, c_type, ascq.F32 if bias is not None else 0)
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
    if c_type in _TORCH_OUT:
        c = torch.full((M, N), float("nan"), dtype=_TORCH_OUT[c_type], device="cuda")
    else:
        c = torch.full((M, N), 0x5A, dtype=torch.uint8, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    return c.cpu()


def _bits(t):
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("trans_a,trans_b", [(False, False), (True, False), (False, True), (True, True)])
def test_hif8_sample_shape(ascq_gpu, oracle, trans_a, trans_b):
    """M = 428, N = 479, K = 158 (K not a multiple of 8: the decoded rows are zero-padded), integers 0 .. 4 encoded to
    hifloat8, f32 bias uniform(-1, 1), f32 C: bit-exact against the oracle and within the sample's own check
    (verify_result.py: rtol = atol = 1e-3, error ratio <= 1e-3) of the fp32 golden"""
    rng = seeded(229)
    M, N, K = 428, 479, 158
    a_int = rng.uniform(0, 5, (M, K)).astype(np.uint8)
    b_int = rng.uniform(0, 5, (K, N)).astype(np.uint8)
    bias = rng.uniform(-1, 1, N).astype(np.float32)
    A = O.hif8_encode(a_int.astype(np.float32).reshape(-1)).reshape(M, K)
    B = O.hif8_encode(b_int.astype(np.float32).reshape(-1)).reshape(K, N)
    got = run_hif8(ascq_gpu, np.ascontiguousarray(A.T) if trans_a else A, np.ascontiguousarray(B.T) if trans_b else B,
                   M, N, K, O.F32, trans_a, trans_b, bias=bias).numpy()
    ref, _, _, _ = O.matmul_fp8(A, B, O.HIF8, O.HIF8, bias=bias, out_type=O.F32)
    np.testing.assert_array_equal(got, ref)
    golden = ((a_int.astype(np.float32) @ b_int.astype(np.float32)) + bias[None, :]).astype(np.float32)
    assert ref_verify(got, golden)


@pytest.mark.parametrize("c_type", [O.HIF8, O.F16, O.BF16, O.INT8, O.FP8_E4M3])
@pytest.mark.parametrize("shape", [(64, 96, 160), (1030, 1100, 256)])
def test_hif8_integer_data_exact(ascq_gpu, oracle, c_type, shape):
    """integer-valued codes (-4 .. 4): the sums are exact, so (sum + bias) * M1 and its cast are bit-exact for every
    C type (hifloat8 C: ties away, saturating at +-32768); the 1030 x 1100 shape runs the 256 x 256 tiles"""
    M, N, K = shape
    rng = seeded(M + N + K + c_type)
    A = hif8_codes(rng, (M, K), -4, 4)
    B = hif8_codes(rng, (N, K), -4, 4)
    bias = rng.integers(-64, 65, N).astype(np.float32) * np.float32(0.25)
    m1 = (np.exp2(rng.integers(-6, 3, N)) * rng.choice([1.0, 1.375, 1.8125], N)).astype(np.float32)
    sign = 1 if c_type == O.INT8 else 0
    words = np.array([O.lib().oq_pack_quant_pre(float(v), int(o), sign) for v, o in
                      zip(m1, rng.integers(0, 8, N) if c_type == O.INT8 else np.zeros(N, np.int64))], np.uint64)
    got = _bits(run_hif8(ascq_gpu, A, B, M, N, K, c_type, trans_b=True, bias=bias, qvec=words))
    ref, _, _, _ = O.matmul_fp8(A, B, O.HIF8, O.HIF8, bias=bias, out_type=c_type, trans_b=True, use_q=True,
                                qvec=words)
    np.testing.assert_array_equal(got.reshape(ref.shape).view(ref.dtype), ref)


@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("c_type", [O.F32, O.BF16])
@pytest.mark.parametrize("shape", [(1024, 1024, 512), (300, 520, 200)])
def test_hif8_random_codes(ascq_gpu, oracle, trans_b, c_type, shape):
    """every finite hifloat8 code (2^-22 .. 2^15, subnormal class included) in A and B, f32 bias, per-channel QUANT_PRE
    words: per element within the fp32-accumulation bound of the oracle's fp64 sums"""
    M, N, K = shape
    rng = seeded(7 + M + trans_b)
    A = hif8_codes(rng, (M, K))
    Bt = hif8_codes(rng, (N, K))
    bias = rng.standard_normal(N).astype(np.float32) * 16
    m1 = np.exp(rng.uniform(np.log(2.0 ** -30), np.log(2.0 ** -20), N)).astype(np.float32)
    words = (m1.view(np.uint32) & np.uint32(0xFFFFE000)).astype(np.uint64)
    got = run_hif8(ascq_gpu, A, Bt if trans_b else np.ascontiguousarray(Bt.T), M, N, K, c_type, trans_b=trans_b,
                   bias=bias, qvec=words).to(torch.float64).numpy()
    _, exact, absd, bmax = O.matmul_fp8(A, Bt, O.HIF8, O.HIF8, bias=bias, trans_b=True)
    mw = words.astype(np.uint32).view(np.float32).astype(np.float64)
    v = exact * mw[None, :]
    d = (2.0 ** -8 * bmax + K * 2.0 ** -24 * (absd + np.abs(bias.astype(np.float64))[None, :])) * mw[None, :]
    check_out(got, v, d, c_type, f"hif8 {shape} trans_b={trans_b}")


def test_hif8_single_shape_unaligned_k(ascq_gpu, oracle):
    """SetSingleShape with k = 150 < K = 158 (k not a multiple of 8: the element-wise kernel on the decoded rows)
    and a tiled sub-block with k = 152"""
    rng = seeded(31)
    M, N, K = 200, 180, 158
    A = hif8_codes(rng, (M, K), -4, 4)
    B = hif8_codes(rng, (K, N), -4, 4)
    for sm, sn, sk in [(130, 100, 150), (200, 180, 152)]:
        got = run_hif8(ascq_gpu, A, B, M, N, K, O.F32, single=(sm, sn, sk)).numpy()
        ref, _, _, _ = O.matmul_fp8(np.ascontiguousarray(A[:sm, :sk]), np.ascontiguousarray(B[:sk, :sn]), O.HIF8,
                                    O.HIF8, out_type=O.F32)
        np.testing.assert_array_equal(got[:sm, :sn], ref)
        assert np.isnan(got[sm:, :]).all() and np.isnan(got[:, sn:]).all()


def test_hif8_special_codes(ascq_gpu, oracle):
    """NaN (0x80) and +-inf (0x6F / 0xEF) operands propagate as in IEEE fp32 sums; f32 C"""
    M, N, K = 32, 32, 64
    A = np.full((M, K), 0x08, np.uint8)  # 1.0
    B = np.full((K, N), 0x08, np.uint8)
    A[1, 5] = 0x80
    A[2, 7] = 0x6F
    A[3, 9] = 0xEF
    B[9, 4] = 0xEF  # -inf * -inf = +inf in row 3, column 4
    got = run_hif8(ascq_gpu, A, B, M, N, K, O.F32).numpy()
    ref, _, _, _ = O.matmul_fp8(A, B, O.HIF8, O.HIF8, out_type=O.F32)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    np.testing.assert_array_equal(got[fin], ref[fin])
    assert np.isnan(got[1]).all() and got[2, 0] == np.inf and got[3, 4] == np.inf


@pytest.mark.parametrize("fa", [O.FP8_E4M3, O.FP8_E5M2])
def test_fp8_operands_hif8_output(ascq_gpu, oracle, fa):
    """(V)QF322HIF8_PRE on fp8 operands (quant_processor_utils.h:36-41 takes hifloat8 C for fp8 A): integer-valued
    fp8 codes, exact sums, bit-exact hifloat8 C"""
    rng = seeded(41 + fa)
    M, N, K = 96, 160, 128
    a_int = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b_int = rng.integers(-4, 5, (N, K)).astype(np.float32)
    t8 = torch.float8_e4m3fn if fa == O.FP8_E4M3 else torch.float8_e5m2
    A = torch.from_numpy(a_int).to(t8).view(torch.uint8).numpy()
    Bt = torch.from_numpy(b_int).to(t8).view(torch.uint8).numpy()
    m1 = np.exp2(rng.integers(-2, 10, N)).astype(np.float32) * np.float32(1.25)
    words = m1.view(np.uint32).astype(np.uint64)
    got = run_hif8(ascq_gpu, A, Bt, M, N, K, O.HIF8, trans_b=True, qvec=words, fa=fa, fb=fa).numpy()
    ref, _, _, _ = O.matmul_fp8(A, Bt, fa, fa, out_type=O.HIF8, trans_b=True, use_q=True, qvec=words)
    np.testing.assert_array_equal(got, ref)
