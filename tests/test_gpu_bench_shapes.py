"""GPU parity at the dense GEMM shapes the benchmark times (M = N = K = 8192): int8 with the DEQF16 epilogue (B given
[K, N] and [N, K]), fp8 e4m3 with QF322BF16_PRE (B given [N, K] and [K, N]) and MX-FP8 (e4m3 elements, E8M0 block
scales).  These run 1024 output tiles of 256 x 256 through the XCD-grouped tile order, so every test compares two
rows of each 256-row tile (the first and last rows of the matrix among them) -- all 8192 columns of each -- against
the oracle: a mistake in the tile order or in any tile's addressing changes at least one compared row.

int8: bit-exact (int32 accumulators, then the oracle's DEQF16).  fp8 / MX-FP8: the per-element bound of the fp8 MFMA
(16-product groups aligned to the group maximum, fp32 across groups; test_gpu_fp8.py states it) against the
oracle's fp64 sums."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded
from test_gpu_fp8 import check_out, mx_bound
from test_gpu_mx import tile_rows
from test_oracle import fp8_bytes

pytestmark = pytest.mark.gpu

S = 8192


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("trans_b", [False, True])
def test_int8_deqf16_8192_sampled(ascq_gpu, oracle, trans_b):
    """A int8 [8192, 8192], B int8 [K, N] (the benchmark's layout, transposed into the workspace first) or [N, K],
    int32 bias, per-channel QUANT_PRE words -> f16; sampled rows bit-exact against the oracle."""
    rng = seeded(81 + trans_b)
    A = rng.integers(-127, 128, (S, S), dtype=np.int8)
    Bkn = rng.integers(-127, 128, (S, S), dtype=np.int8)  # logical B [K, N]
    bias = rng.integers(-(1 << 15), (1 << 15) + 1, S, dtype=np.int32)
    sc = np.exp(rng.uniform(np.log(2.0 ** -20), np.log(2.0 ** -10), S)).astype(np.float32)
    words = sc.view(np.uint32).astype(np.uint64)
    mm = ascq_gpu.Matmul(ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.F16, ascq_gpu.INT32)
    mm.SetOrgShape(S, S, S)
    mm.SetQuantVector(_dev(words.view(np.int64)))
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(np.ascontiguousarray(Bkn.T)) if trans_b else _dev(Bkn), trans_b)
    mm.SetBias(_dev(bias))
    c = torch.empty((S, S), dtype=torch.float16, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    rows = tile_rows(rng, S)
    got = _bits(c.cpu())[rows]
    acc = O.matmul_i8(np.ascontiguousarray(A[rows]), Bkn, bias)
    np.testing.assert_array_equal(got, O.mm_dequant(acc, O.F16, qvec=words))


@pytest.mark.parametrize("trans_b", [True, False])
def test_fp8_qf322bf16_8192_sampled(ascq_gpu, oracle, trans_b):
    """fp8 e4m3 A, B [8192, 8192] (every finite code), per-channel QF322BF16_PRE -> bf16, B given [N, K] (the
    benchmark's layout) or [K, N]; sampled rows within the fp8-MFMA bound of the oracle's fp64 sums."""
    rng = seeded(83 + trans_b)
    f = O.FP8_E4M3
    A = fp8_bytes(rng, (S, S), f)
    Bt = fp8_bytes(rng, (S, S), f)  # logical B^T [N, K]
    m1 = np.exp(rng.uniform(np.log(2.0 ** -12), np.log(2.0 ** -6), S)).astype(np.float32)
    words = (m1.view(np.uint32) & np.uint32(0xFFFFE000)).astype(np.uint64)
    mm = ascq_gpu.Matmul(f, f, ascq_gpu.BF16)
    mm.SetOrgShape(S, S, S)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(Bt) if trans_b else _dev(np.ascontiguousarray(Bt.T)), trans_b)
    mm.SetQuantVector(_dev(words.view(np.int64)))
    c = torch.empty((S, S), dtype=torch.bfloat16, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    rows = tile_rows(rng, S)
    got = c.cpu()[torch.from_numpy(rows)].to(torch.float64).numpy()
    _, exact, absd, bmax = O.matmul_fp8(np.ascontiguousarray(A[rows]), Bt, f, f, trans_b=True)
    mw = words.astype(np.uint32).view(np.float32).astype(np.float64)
    v = exact * mw[None, :]
    d = (2.0 ** -8 * bmax + S * 2.0 ** -24 * absd) * mw[None, :]
    check_out(got, v, d, O.BF16, f"fp8 8192^3 trans_b={trans_b}")


def test_mx_fp8_8192_sampled(ascq_gpu, oracle):
    """MX-FP8: e4m3 A, B [8192, 8192], E8M0 scales per 32 K (A [M, sK], B [N, sK] as the benchmark passes them),
    bf16 out; sampled rows within the fp8-MFMA bound of the oracle's fp64 sums."""
    rng = seeded(85)
    f = O.FP8_E4M3
    sK = S // 32
    A = fp8_bytes(rng, (S, S), f)
    Bt = fp8_bytes(rng, (S, S), f)
    sA = rng.integers(118, 136, (S, sK), dtype=np.uint8)
    sB = rng.integers(118, 136, (S, sK), dtype=np.uint8)
    mm = ascq_gpu.Matmul(f, f, ascq_gpu.BF16, 0, ascq_gpu.E8M0)
    mm.SetOrgShape(S, S, S)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(Bt), True)
    mm.SetTensorScaleA(_dev(sA), False)
    mm.SetTensorScaleB(_dev(sB), True)
    c = torch.empty((S, S), dtype=torch.bfloat16, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    rows = tile_rows(rng, S)
    got = c.cpu()[torch.from_numpy(rows)].to(torch.float64).numpy()
    _, Ce, Ca, Cb = O.mx_matmul(A, Bt, sA, sB, S, S, S, trans_b=True, sa_layout=0, sb_layout=1, elem_fmt=f, fmt_b=f,
                                rows=rows, blockmax=True)
    check_out(got, Ce[rows], mx_bound(Ca[rows], Cb[rows], S), O.BF16, "mx-fp8 8192^3")
