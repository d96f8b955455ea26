"""GPU parity: the any-alignment MFMA tiles (K not a multiple of 16, operands at any byte offset) of the quantized
group matmul, the int8 Matmul and the fp8 Matmul, against the oracle; and ASCQ_LOG=1 naming the generic kernel a
launch falls back to.

Each operand is placed at a byte offset inside a larger device buffer whose other bytes hold 0x5A, so bytes read past
K, past a row or past the operand would enter the sums unless the kernel zeroes them.  int8: int32 accumulators,
bit-exact outputs.  fp8: integer-valued codes (-4 .. 4) give exact sums, so f32 C is bit-exact as well."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
FILL = 0x5A


def _dev_at(a, off):
    """a (int8 / uint8) on the device at byte offset `off` of a buffer filled with FILL"""
    a = np.ascontiguousarray(a)
    buf = torch.full((a.nbytes + off + 64,), FILL, dtype=torch.uint8, device="cuda")
    buf[off:off + a.nbytes] = torch.from_numpy(a.view(np.uint8).reshape(-1)).cuda()
    t = buf[off:off + a.nbytes]
    return (t.view(torch.int8) if a.dtype == np.int8 else t).view(a.shape)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("w_trans", [False, True])
@pytest.mark.parametrize("K,N,x_off,w_off", [(100, 160, 0, 0), (333, 150, 3, 5), (17, 162, 1, 0), (1, 64, 0, 7),
                                             (256, 160, 4, 2), (1000, 704, 1, 1)])
def test_group_matmul_any_alignment(ascq_gpu, oracle, w_trans, K, N, x_off, w_off):
    """K % 16 != 0 and / or X, W at odd byte offsets: the any-alignment tiles, bit-exact, rows outside the groups
    untouched"""
    rng = seeded(900 + K + N + x_off + 2 * w_off + w_trans)
    counts = np.array([97, 0, 140, 33], np.int64) if K < 1000 else np.array([400, 1, 333, 290], np.int64)
    G = len(counts)
    M = int(counts.sum()) + 5
    x = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (G, N, K) if w_trans else (G, K, N), dtype=np.int8)
    pts = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), M)).astype(np.float32)
    scale = np.exp(rng.uniform(np.log(1e-4), np.log(1e-2), (G, N))).astype(np.float32)
    gl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    y = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    ascq_gpu.quant_group_matmul(_dev_at(x, x_off), _dev(pts), _dev_at(w, w_off), _dev(scale), _dev(gl), 0, w_trans,
                                torch.bfloat16, out=y)
    y0 = torch.full((M, N), 3.0, dtype=torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()
    ref = O.group_matmul(x, pts, w, scale, gl, 0, G, M, K, N, O.BF16, w_trans, y=y0)
    np.testing.assert_array_equal(_bits(y.cpu()), ref)


def _int8_mm(ascq, A, B, bias, words, trans_a, trans_b, a_off, b_off, M, N, K, single=None):
    mm = ascq.Matmul(ascq.INT8, ascq.INT8, ascq.F16, ascq.INT32)
    mm.SetOrgShape(M, N, K)
    if single is not None:
        mm.SetSingleShape(*single)
    mm.SetQuantVector(_dev(words.view(np.int64)))
    mm.SetTensorA(_dev_at(A, a_off), trans_a)
    mm.SetTensorB(_dev_at(B, b_off), trans_b)
    mm.SetBias(_dev(bias))
    c = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    return _bits(c.cpu())


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("shape,a_off,b_off", [((77, 200, 99), 0, 0), ((300, 132, 1037), 3, 1), ((5, 7, 3), 1, 2),
                                               ((1030, 1100, 333), 2, 0), ((2100, 2080, 77), 0, 3)])
def test_int8_matmul_any_alignment(ascq_gpu, oracle, trans_b, shape, a_off, b_off):
    """int8 Matmul, DEQF16 C with int32 bias and per-channel words, K % 16 != 0 and / or A, B at odd byte offsets
    (64 x 64 and, for 2100 x 2080, 128 x 128 any-alignment tiles): bit-exact"""
    M, N, K = shape
    rng = seeded(M + N + K + a_off + trans_b)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    Bkn = rng.integers(-128, 128, (K, N), dtype=np.int8)
    bias = rng.integers(-(1 << 20), 1 << 20, N, dtype=np.int32)
    sc = np.exp(rng.uniform(np.log(2.0 ** -20), np.log(2.0 ** -8), N)).astype(np.float32)
    words = sc.view(np.uint32).astype(np.uint64)
    got = _int8_mm(ascq_gpu, A, np.ascontiguousarray(Bkn.T) if trans_b else Bkn, bias, words, False, trans_b, a_off,
                   b_off, M, N, K)
    ref = O.mm_dequant(O.matmul_i8(A, Bkn, bias), O.F16, qvec=words)
    np.testing.assert_array_equal(got, ref)


def test_int8_matmul_any_alignment_trans_a_single_shape(ascq_gpu, oracle):
    """A given [K, M] (transposed into the workspace, rows of K = 150 bytes) and a SetSingleShape block with k = 131"""
    rng = seeded(77)
    M, N, K = 200, 180, 150
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    Bkn = rng.integers(-128, 128, (K, N), dtype=np.int8)
    bias = rng.integers(-(1 << 20), 1 << 20, N, dtype=np.int32)
    words = np.full(N, np.float32(2.0 ** -12).view(np.uint32), np.uint64)
    got = _int8_mm(ascq_gpu, np.ascontiguousarray(A.T), Bkn, bias, words, True, False, 1, 0, M, N, K)
    np.testing.assert_array_equal(got, O.mm_dequant(O.matmul_i8(A, Bkn, bias), O.F16, qvec=words))
    sm, sn, sk = 130, 100, 131
    got = _int8_mm(ascq_gpu, A, Bkn, bias, words, False, False, 3, 1, M, N, K, single=(sm, sn, sk))
    ref = O.mm_dequant(O.matmul_i8(np.ascontiguousarray(A[:sm, :sk]), np.ascontiguousarray(Bkn[:sk, :sn]), bias[:sn]),
                       O.F16, qvec=words[:sn])
    np.testing.assert_array_equal(got[:sm, :sn], ref)
    assert np.isnan(got[sm:].view(np.float16)).all() and np.isnan(got[:, sn:].view(np.float16)).all()


def _fp8_codes(rng, shape, t8):
    v = rng.integers(-4, 5, shape).astype(np.float32)
    return torch.from_numpy(v).to(t8).view(torch.uint8).numpy()


@pytest.mark.parametrize("fa,fb", [(O.FP8_E4M3, O.FP8_E4M3), (O.FP8_E5M2, O.FP8_E4M3)])
@pytest.mark.parametrize("shape,a_off,b_off", [((96, 160, 150), 0, 0), ((300, 200, 77), 5, 3),
                                               ((2100, 2080, 40), 1, 0)])
def test_fp8_matmul_any_alignment(ascq_gpu, oracle, fa, fb, shape, a_off, b_off):
    """fp8 A [M, K], B [N, K] with K % 16 != 0 and / or at odd byte offsets, f32 bias, f32 C: integer-valued codes,
    exact sums, bit-exact"""
    M, N, K = shape
    rng = seeded(M + K + fa + 3 * fb + a_off)
    tt = {O.FP8_E4M3: torch.float8_e4m3fn, O.FP8_E5M2: torch.float8_e5m2}
    A = _fp8_codes(rng, (M, K), tt[fa])
    Bt = _fp8_codes(rng, (N, K), tt[fb])
    bias = rng.integers(-64, 65, N).astype(np.float32)
    mm = ascq_gpu.Matmul(fa, fb, ascq_gpu.F32, ascq_gpu.F32)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev_at(A, a_off))
    mm.SetTensorB(_dev_at(Bt, b_off), True)
    mm.SetBias(_dev(bias))
    c = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    ref, _, _, _ = O.matmul_fp8(A, Bt, fa, fb, bias=bias, out_type=O.F32, trans_b=True)
    np.testing.assert_array_equal(c.cpu().numpy(), ref)


_LOG_SCRIPT = r"""
import sys
sys.path.insert(0, {pkg!r})
import numpy as np, torch, ascq
dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
rng = np.random.default_rng(5)
# group matmul, K = 100: the any-alignment tiles (no fallback)
x = rng.integers(-8, 8, (64, 100), dtype=np.int8)
w = rng.integers(-8, 8, (2, 100, 96), dtype=np.int8)
ascq.quant_group_matmul(dev(x), dev(np.ones(64, np.float32)), dev(w), dev(np.ones((2, 96), np.float32)),
                        dev(np.array([0, 30, 64], np.int64)), 0, False, torch.bfloat16)
torch.cuda.synchronize()
print("step group done", file=sys.stderr, flush=True)
# fp8 Matmul with B given [K, N] and K = 40: the generic kernel
mm = ascq.Matmul(ascq.FP8_E4M3, ascq.FP8_E4M3, ascq.F32)
mm.SetOrgShape(32, 32, 40)
mm.SetTensorA(dev(np.full((32, 40), 0x38, np.uint8)))
mm.SetTensorB(dev(np.full((40, 32), 0x38, np.uint8)), False)
c = torch.empty((32, 32), dtype=torch.float32, device="cuda")
mm.IterateAll(c)
mm.End()
torch.cuda.synchronize()
assert (c == 40.0).all(), c
print("step fp8 done", file=sys.stderr, flush=True)
"""


def test_fallback_logged_under_ascq_log():
    """ASCQ_LOG=1: a launch that takes a generic kernel prints 'ascq: fallback: <kernel> (<reason>)' on stderr;
    the any-alignment tiles print nothing.  One child process (the level is read once per process)."""
    code = _LOG_SCRIPT.format(pkg=str(ROOT / "asc-devkit_clone_amd"))
    env = dict(os.environ, ASCQ_LOG="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stderr.splitlines() if ln.startswith("ascq:")]
    assert lines == ["ascq: fallback: gemm_f8_generic_kernel (B given [K, N] with K not a multiple of 16 or operands "
                     "not aligned)"], r.stderr[-2000:]
