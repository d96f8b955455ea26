"""GPU parity sweep over the decode-batch forms of the quantized Matmuls (M <= 64, B streamed once): shapes chosen on
both sides of each dispatch rule -- K split over the waves of a workgroup, K split across workgroups as well (B [N, K]
with few 32 x 32 tiles and long K; B [K, N] on 32 x 128 tiles with long K or wide N; MX-FP4 with few 64 x 64 tiles),
B [K, N] on 32 x 64 tiles from N = 10240 on, 64 x 32 tiles for 33-64 rows at N = 7169-8192,
B [K, N] rows that are not 16-byte multiples, row-major and block-pair MX scales -- against the oracle: int8 bit-exact
(int32 and DEQF16 C), fp8 and MX-FP4 within the bounds their own test files state (fp32 accumulation, the fp8 MFMA's
16-element group alignment)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded
from test_gpu_fp8 import check_out, expected, fp8_case, run_fp8
from test_gpu_matmul import _bits, _quant_words, _run
from test_gpu_mx import bf16_to_f64, check, mx_inputs, run_mx, scale_pairs

pytestmark = pytest.mark.gpu

# (M, N, K, B given [N, K])
_I8 = [(1, 4096, 8192, False), (7, 4104, 8448, False), (16, 12416, 512, False), (32, 4000, 8192, True),
       (3, 5120, 9216, True), (20, 4096, 10240, True), (12, 8192, 8192, True), (1, 2048, 8192, False),
       (29, 4608, 11264, False), (64, 4096, 8192, True), (33, 4096, 8192, False), (1, 11008, 4096, False),
       (16, 10256, 2048, False), (40, 10240, 1024, False), (50, 4096, 11008, True), (64, 12416, 768, False),
       (40, 8008, 1024, True), (64, 8192, 2048, True), (48, 8000, 1024, False), (64, 9216, 2048, False)]


@pytest.mark.parametrize("M,N,K,trans_b", _I8)
def test_int8_decode_forms(ascq_gpu, oracle, M, N, K, trans_b):
    rng = seeded(M * 7 + N + K + trans_b)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (N, K) if trans_b else (K, N), dtype=np.int8)
    bias = rng.integers(-(1 << 20), 1 << 20, N, dtype=np.int32)
    acc = O.matmul_i8(A, B, bias, trans_b=trans_b)
    np.testing.assert_array_equal(_run(ascq_gpu, A, B, bias, ascq_gpu.INT32, trans_b=trans_b).numpy(), acc)
    words = _quant_words(rng, N, 2.0 ** -20, 2.0 ** -4)
    c = _run(ascq_gpu, A, B, bias, ascq_gpu.F16, words=words, trans_b=trans_b)
    np.testing.assert_array_equal(_bits(c), O.mm_dequant(acc, O.F16, qvec=words))


@pytest.mark.parametrize("M,N,K,trans_b", [(1, 4096, 8192, False), (16, 12416, 512, False), (32, 4000, 8192, True),
                                           (5, 5120, 9216, True), (9, 4104, 8192, False), (8, 11008, 4096, False),
                                           (48, 4096, 8192, True), (64, 4096, 8192, False), (40, 8008, 1024, True),
                                           (48, 8000, 1024, False)])
def test_fp8_decode_forms(ascq_gpu, M, N, K, trans_b):
    fa, fb = O.FP8_E4M3, O.FP8_E4M3
    A, B, b, qs, qv = fp8_case(5 * M + N + K, M, N, K, fa, fb, O.BF16, trans_b=trans_b, quant="vector")
    got = run_fp8(ascq_gpu, A, B, fa, fb, M, N, K, O.BF16, trans_b=trans_b, bias=b, qvec=qv)
    v, d = expected(A, B, fa, fb, b, qs, qv, False, trans_b, K)
    check_out(got, v, d, O.BF16, f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K", [(1, 2048, 4096), (16, 4096, 2048), (64, 1024, 8192), (5, 8192, 1024)])
@pytest.mark.parametrize("pairs", [False, True])
def test_mx_decode_forms(ascq_gpu, oracle, M, N, K, pairs):
    rng = seeded(M + N + K + pairs)
    A, sA, Bt, sBt = mx_inputs(rng, M, N, K)
    sB_dev = scale_pairs(sBt) if pairs else sBt
    c = run_mx(ascq_gpu, A, sA, Bt, sB_dev, M, N, K, True, 0, 0 if pairs else 1, ascq_gpu.BF16)
    C, Ce, Ca = O.mx_matmul(A, Bt, sA, sBt, M, N, K, trans_b=True, sa_layout=0, sb_layout=1)
    check(bf16_to_f64(c.view(torch.int16).numpy().view(np.uint16)), Ce, Ca, K, C)
