"""GPU parity: IterateAll(C, enAtomic) -- ATOMIC_ADD / MAX / MIN combine the result into C in C's type
(include/adv_api/matmul/matmul.h:255-265; impl/adv_api/detail/matmul/scheduler/base/scheduler_base.h:484-494).

Each case runs the handle once with en_atomic = 0 into R (that path's parity is tested elsewhere), then twice
with en_atomic = op into a C that starts from random values C0, and requires C to equal, bit for bit, the
oracle's op(op(C0, R), R).  The tiled kernels (256-row tiles, whose int32 / f32 accumulators go through LDS in
two chunks, and 64-row tiles), the element-wise kernels and the weight-only kernels are all reached."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded
from test_gpu_mx import mx_inputs

pytestmark = pytest.mark.gpu

_TORCH = {O.INT32: torch.int32, O.F32: torch.float32, O.F16: torch.float16, O.BF16: torch.bfloat16}


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host_bits(t):
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


def _random_c(rng, c_type, shape, scale):
    if c_type == O.INT32:
        return rng.integers(-(1 << 30), 1 << 30, shape).astype(np.int32)
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    if c_type == O.F32:
        return x
    if c_type == O.F16:
        return np.clip(x, -60000, 60000).astype(np.float16).view(np.uint16)
    return (x.view(np.uint32) >> 16).astype(np.uint16)  # bf16 by truncation: any bf16 values will do


def _check(ascq, mm, c_type, M, N, seed, ops=(1, 2, 3)):
    rng = seeded(seed)
    r = torch.empty((M, N), dtype=_TORCH[c_type], device="cuda")
    mm.IterateAll(r)
    torch.cuda.synchronize()
    R = _host_bits(r)
    scale = float(np.abs(R.astype(np.float64)).mean()) if c_type != O.INT32 else 1.0
    if c_type in (O.F16, O.BF16):
        dt = torch.float16 if c_type == O.F16 else torch.bfloat16
        scale = float(torch.from_numpy(R.view(np.int16)).view(dt).float().abs().mean())
    for op in ops:
        C0 = _random_c(rng, c_type, (M, N), scale or 1.0)
        c = _dev(C0.view(np.int16) if C0.dtype == np.uint16 else C0)
        if C0.dtype == np.uint16:
            c = c.view(_TORCH[c_type])
        mm.IterateAll(c, op)
        mm.IterateAll(c, op)
        torch.cuda.synchronize()
        want = O.c_combine(O.c_combine(C0, R, c_type, op), R, c_type, op)
        got = _host_bits(c)
        bad = got != want
        assert not bad.any(), f"op {op}: {bad.sum()} of {bad.size} elements differ"


def _quant_words(rng, n):
    s = np.exp(rng.uniform(np.log(2.0 ** -12), np.log(2.0 ** -6), n)).astype(np.float32)
    return s.view(np.uint32).astype(np.uint64)


@pytest.mark.parametrize("c_type", [O.INT32, O.F16, O.BF16])
@pytest.mark.parametrize("shape", [(1024, 1024, 256), (200, 136, 96), (77, 50, 40)])
def test_atomic_int8(ascq_gpu, oracle, c_type, shape):
    """int8 x int8 (+ int32 bias): int32 accumulators, DEQF16 / QS322BF16 per-channel outputs"""
    M, N, K = shape
    rng = seeded(M + N + K + c_type)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    bias = rng.integers(-(1 << 20), 1 << 20, N, dtype=np.int32)
    mm = ascq_gpu.Matmul(ascq_gpu.INT8, ascq_gpu.INT8, c_type, ascq_gpu.INT32)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B))
    mm.SetBias(_dev(bias))
    if c_type != O.INT32:
        mm.SetQuantVector(_dev(_quant_words(rng, N).view(np.int64)))
    _check(ascq_gpu, mm, c_type, M, N, seed=M + c_type)
    mm.End()


def test_atomic_int4_operands(ascq_gpu, oracle):
    M, N, K = 300, 256, 512
    rng = seeded(41)
    A = rng.integers(0, 256, (M, K // 2), dtype=np.uint8)
    B = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    mm = ascq_gpu.Matmul(ascq_gpu.INT4, ascq_gpu.INT4, ascq_gpu.INT32)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B), True)
    _check(ascq_gpu, mm, O.INT32, M, N, seed=42)
    mm.End()


@pytest.mark.parametrize("c_type", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("shape", [(1024, 1024, 256), (130, 70, 128), (50, 33, 40)])
def test_atomic_fp8(ascq_gpu, oracle, c_type, shape):
    """fp8 e4m3 x e5m2 with an f32 bias and a per-channel QF322*_PRE word"""
    M, N, K = shape
    rng = seeded(M + 7 * N + K + c_type)
    A = rng.integers(0, 256, (M, K), dtype=np.uint8)
    B = rng.integers(0, 256, (N, K), dtype=np.uint8)
    A[(A & 0x7F) == 0x7F] = 0  # e4m3: no NaN codes
    B[(B & 0x7C) == 0x7C] = 0  # e5m2: no inf / NaN codes
    bias = rng.standard_normal(N).astype(np.float32)
    mm = ascq_gpu.Matmul(ascq_gpu.FP8_E4M3, ascq_gpu.FP8_E5M2, c_type, ascq_gpu.F32)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B), True)
    mm.SetBias(_dev(bias))
    mm.SetQuantVector(_dev(_quant_words(rng, N).view(np.int64)))
    _check(ascq_gpu, mm, c_type, M, N, seed=N + c_type)
    mm.End()


@pytest.mark.parametrize("c_type", [O.F32, O.BF16])
@pytest.mark.parametrize("fmts", [("e2m1", "e2m1"), ("e1m2", "e2m1")])
@pytest.mark.parametrize("shape", [(1024, 1024, 256), (130, 70, 128)])
def test_atomic_mx(ascq_gpu, oracle, c_type, fmts, shape):
    """MX-FP4 (E2M1 kernel) and the fp6 kernel of an E1M2 operand, with an f32 bias"""
    M, N, K = shape
    rng = seeded(M + N + K + c_type + len(fmts[0]))
    A, sA, Bt, sBt = mx_inputs(rng, M, N, K)
    code = {"e2m1": ascq_gpu.FP4_E2M1, "e1m2": ascq_gpu.FP4_E1M2}
    bias = rng.standard_normal(N).astype(np.float32)
    mm = ascq_gpu.Matmul(code[fmts[0]], code[fmts[1]], c_type, ascq_gpu.F32, ascq_gpu.E8M0)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(Bt), True)
    mm.SetTensorScaleA(_dev(sA), False)
    mm.SetTensorScaleB(_dev(sBt), True)
    mm.SetBias(_dev(bias))
    _check(ascq_gpu, mm, c_type, M, N, seed=K + c_type)
    mm.End()


@pytest.mark.parametrize("M", [1, 16, 64, 70, 300])
def test_atomic_weight_only(ascq_gpu, oracle, M):
    """W4A16 through the Matmul handle: decode (M <= 4), the LDS-ring batch forms and the prefill GEMM (M > 64)"""
    from test_gpu_gemv import make_weights

    rng = seeded(500 + M)
    K, N, g = 1024, 512, 128
    w, scale, offset = make_weights(rng, K, N, O.INT4, g)
    x = rng.standard_normal((M, K)).astype(np.float16)
    mm = ascq_gpu.Matmul(ascq_gpu.F16, ascq_gpu.INT4, ascq_gpu.F16)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(x))
    mm.SetTensorB(_dev(w))
    mm.SetAntiQuantVector(_dev(offset), _dev(scale), g)
    _check(ascq_gpu, mm, O.F16, M, N, seed=M)
    mm.End()


def test_atomic_ignored_for_uint8_and_refused_for_int8(ascq_gpu, oracle):
    """SetAtomic covers float / half / int16 / int32 / int8 / bf16 C only (scheduler_base.h:484-494): a uint8 C is
    stored as without enAtomic; int8 C with enAtomic is refused here (its saturation is not published)"""
    M, N, K = 64, 64, 64
    rng = seeded(9)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    word = int(np.float32(2.0 ** -10).view(np.uint32)) | (1 << 46)  # sign flag: uint8 saturation
    mm = ascq_gpu.Matmul(ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.UINT8)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B))
    mm.SetQuantScalar(word)
    r = torch.empty((M, N), dtype=torch.uint8, device="cuda")
    c = torch.full((M, N), 7, dtype=torch.uint8, device="cuda")
    mm.IterateAll(r)
    mm.IterateAll(c, ascq_gpu.ATOMIC_ADD)
    torch.cuda.synchronize()
    assert torch.equal(r.cpu(), c.cpu())
    mm.End()
    mm8 = ascq_gpu.Matmul(ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.INT8)
    mm8.SetOrgShape(M, N, K)
    mm8.SetTensorA(_dev(A))
    mm8.SetTensorB(_dev(B))
    mm8.SetQuantScalar(int(np.float32(2.0 ** -10).view(np.uint32)))
    c8 = torch.zeros((M, N), dtype=torch.int8, device="cuda")
    with pytest.raises(ascq_gpu.AscqError, match="enAtomic"):
        mm8.IterateAll(c8, ascq_gpu.ATOMIC_ADD)
    with pytest.raises(ascq_gpu.AscqError, match="enAtomic"):
        mm8.IterateAll(c8, 4)
