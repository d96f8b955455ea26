"""GPU parity: NZ fractal <-> ND converters through the C ABI, bit-exact against the oracle (a byte
permutation), and the reference's NZ expert weights fed to the group matmul after ascq_nz_to_nd."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu

_ESIZE = {"INT8": 1, "F16": 2, "F32": 4}


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("dt", ["INT8", "F16", "F32"])
@pytest.mark.parametrize("B,R,C", [(1, 16, 64), (3, 37, 45), (2, 128, 96), (1, 1, 1), (4, 255, 130)])
def test_nz_round_trip_vs_oracle(ascq_gpu, dt, B, R, C):
    es = _ESIZE[dt]
    rng = seeded(B * 1000 + R * 10 + C + es)
    nd = rng.integers(0, 256, (B, R, C * es)).astype(np.uint8)
    code = getattr(ascq_gpu, dt)
    nz = ascq_gpu.nd_to_nz(_dev(nd), code, B, R, C).cpu().numpy()
    assert np.array_equal(nz, O.nd_to_nz(nd, es, B, R, C))
    back = ascq_gpu.nz_to_nd(_dev(nz), code, B, R, C).cpu().numpy()
    assert np.array_equal(back, nd)
    assert np.array_equal(back, O.nz_to_nd(nz, es, B, R, C))


@pytest.mark.parametrize("B,R,C", [(2, 64, 96), (1, 40, 70), (16, 4096, 1408)])
def test_nz_to_nd_transposed(ascq_gpu, B, R, C):
    """1-byte NZ -> [batch, cols, rows] (K-contiguous weights), aligned (16-byte stores) and ragged rows"""
    rng = seeded(R + C)
    nz = rng.integers(0, 256, O.nz_size(1, B, R, C)).astype(np.uint8)
    got = ascq_gpu.nz_to_nd(_dev(nz), ascq_gpu.INT8, B, R, C, transpose_out=True).cpu().numpy()
    if B * R * C <= 1 << 20:
        assert np.array_equal(got, O.nz_to_nd(nz, 1, B, R, C, transpose_out=True))
    else:  # full MoE weight size: check against numpy's reshape of the same fractal order
        w = nz.reshape(B, C // 32, R // 16, 16, 32).transpose(0, 2, 3, 1, 4).reshape(B, R, C)
        assert np.array_equal(got, np.ascontiguousarray(w.transpose(0, 2, 1)))


def test_group_matmul_from_nz_weights(ascq_gpu, oracle):
    """the reference feeds the group matmul NZ weights (gen_data.py:62); ascq_nz_to_nd(transpose_out) turns them
    into [G, N, K] once, and the group matmul on them equals the oracle on the ND weights bit for bit"""
    rng = seeded(99)
    G, K, N = 4, 256, 160
    counts = np.array([40, 7, 0, 81], np.int64)
    M = int(counts.sum())
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (G, K, N), dtype=np.int8)
    nz = np.ascontiguousarray(w.reshape(G, K // 16, 16, N // 32, 32).transpose(0, 3, 1, 2, 4))
    pts = rng.normal(0, 0.01, M).astype(np.float32)
    scale = rng.normal(0, 0.01, (G, N)).astype(np.float32)
    wt = ascq_gpu.nz_to_nd(_dev(nz.view(np.uint8)), ascq_gpu.INT8, G, K, N, transpose_out=True)
    y = ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), wt.view(torch.int8), _dev(scale), _dev(counts), 1, True,
                                    torch.float16, activation=ascq_gpu.ACT_FASTER_GELU)
    ref = O.group_matmul(x, pts, w, scale, counts, 1, G, M, K, N, O.F16, act=1)
    got = y.cpu().view(torch.int16).numpy().view(np.uint16)
    assert (got == ref).mean() >= 0.99  # FasterGelu's expf: within one ulp elsewhere
    y0 = ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), wt.view(torch.int8), _dev(scale), _dev(counts), 1, True,
                                     torch.bfloat16)
    ref0 = O.group_matmul(x, pts, w, scale, counts, 1, G, M, K, N, O.BF16)
    assert np.array_equal(y0.cpu().view(torch.int16).numpy().view(np.uint16), ref0)


def _nz_of(b):
    """the NZ form of one [rows, cols] 1-byte matrix (the oracle's restatement of the fractal layout)"""
    rows, cols = b.shape
    return O.nd_to_nz(b.view(np.uint8)[None], 1, 1, rows, cols)


@pytest.mark.parametrize("M,N,K", [(64, 96, 128), (100, 72, 96), (1024, 1280, 512)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_matmul_nz_b_int8(ascq_gpu, oracle, M, N, K, trans_b):
    """an int8 Matmul whose B is declared NZ (MatmulType<GM, NZ, int8_t>, the group-matmul sample's B,
    quant_group_matmul_custom.asc:110): IterateAll on the NZ bytes equals the oracle on the ND B bit for bit, int32 C
    and DEQF16 f16 C with bias, B given [K, N] or (isTransposeB) [N, K], shapes padded inside the fractals and one
    on the 256 x 256 tiles"""
    rng = seeded(M + 3 * N + 7 * K + int(trans_b))
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-127, 128, (K, N), dtype=np.int8)
    nz = _nz_of(np.ascontiguousarray(B.T) if trans_b else B)
    mm = ascq_gpu.Matmul(ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.INT32, 0, 0, ascq_gpu.FORMAT_NZ)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(nz), trans_b)
    c = torch.full((M, N), 7, dtype=torch.int32, device="cuda")
    mm.IterateAll(c)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(c.cpu().numpy(), O.matmul_i8(A, B))
    mm.End()
    bias = rng.integers(-(1 << 15), 1 << 15, N, dtype=np.int32)
    sc = np.exp(rng.uniform(np.log(2.0 ** -12), np.log(2.0 ** -6), N)).astype(np.float32)
    words = sc.view(np.uint32).astype(np.uint64)
    mq = ascq_gpu.Matmul(ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.F16, ascq_gpu.INT32, 0, ascq_gpu.FORMAT_NZ)
    mq.SetOrgShape(M, N, K)
    mq.SetQuantVector(_dev(words.view(np.int64)))
    mq.SetTensorA(_dev(A))
    mq.SetTensorB(_dev(nz), trans_b)
    mq.SetBias(_dev(bias))
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    mq.IterateAll(y)
    torch.cuda.synchronize()
    ref = O.mm_dequant(O.matmul_i8(A, B, bias), O.F16, qvec=words)
    np.testing.assert_array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), ref)
    mq.End()


@pytest.mark.parametrize("M,N,K", [(96, 160, 192), (1024, 1024, 256)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_matmul_nz_b_fp8(ascq_gpu, M, N, K, trans_b):
    """an fp8 Matmul with B declared NZ equals the same Matmul with the ND B, bit for bit (f32 C: the same kernel
    on the same K-contiguous B)"""
    rng = seeded(5 * M + N + K + int(trans_b))
    A = torch.randn((M, K), generator=torch.Generator().manual_seed(M + K)).to(torch.float8_e4m3fn).view(torch.uint8)
    B = torch.randn((K, N), generator=torch.Generator().manual_seed(N + K)).to(torch.float8_e4m3fn).view(torch.uint8)
    Bn = np.ascontiguousarray(B.numpy().T) if trans_b else B.numpy()
    outs = []
    for fmt, b in ((ascq_gpu.FORMAT_ND, Bn), (ascq_gpu.FORMAT_NZ, _nz_of(Bn))):
        mm = ascq_gpu.Matmul(ascq_gpu.FP8_E4M3, ascq_gpu.FP8_E4M3, ascq_gpu.F32, 0, 0, fmt)
        mm.SetOrgShape(M, N, K)
        mm.SetTensorA(A.cuda())
        mm.SetTensorB(_dev(b), trans_b)
        c = torch.full((M, N), float(rng.integers(1, 9)), dtype=torch.float32, device="cuda")
        mm.IterateAll(c)
        torch.cuda.synchronize()
        outs.append(c.cpu().view(torch.int32).numpy())
        mm.End()
    np.testing.assert_array_equal(outs[1], outs[0])
