"""GPU parity: int8 Matmul with fused dequant (DEQF16 / QS322BF16 / raw int32) through the Matmul handle.

int32 accumulators and the dequantised outputs are bit-exact vs the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _quant_words(rng, n, lo=2.0 ** -12, hi=2.0 ** -6):
    s = np.exp(rng.uniform(np.log(lo), np.log(hi), n)).astype(np.float32)
    return s.view(np.uint32).astype(np.uint64)  # (uint64)(*(uint32*)&f): matmul_quant.asc:111-113


def _run(ascq, A, B, bias, c_type, words=None, scalar=None, trans_b=False, M=None, N=None, K=None):
    M = M or A.shape[0]
    K = K or A.shape[1]
    N = N or (B.shape[0] if trans_b else B.shape[1])
    torch_c = {ascq.F16: torch.float16, ascq.BF16: torch.bfloat16, ascq.INT32: torch.int32}[c_type]
    mm = ascq.Matmul(ascq.INT8, ascq.INT8, c_type, ascq.INT32 if bias is not None else 0)
    mm.SetOrgShape(M, N, K)
    if words is not None:
        mm.SetQuantVector(_dev(words.view(np.int64)))
    elif scalar is not None:
        mm.SetQuantScalar(scalar)
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B), trans_b)
    if bias is not None:
        mm.SetBias(_dev(bias))
    c = torch.empty((M, N), dtype=torch_c, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    return c.cpu()


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype in (torch.float16, torch.bfloat16) else t.numpy()


def test_config1_w8a8_per_channel_deqf16(ascq_gpu, oracle):
    """W8A8: A [128,512], B [512,256] uniform [-127,127], int32 bias [-2^15,2^15], per-channel scale
    log-uniform [2^-12, 2^-6] -> fp16 [128,256].  int32 bit-exact, fp16 bit-exact vs the oracle."""
    rng = seeded(1)
    M, K, N = 128, 512, 256
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-127, 128, (K, N), dtype=np.int8)
    bias = rng.integers(-(1 << 15), (1 << 15) + 1, N, dtype=np.int32)
    words = _quant_words(rng, N)
    acc_ref = O.matmul_i8(A, B, bias)
    c32 = _run(ascq_gpu, A, B, bias, ascq_gpu.INT32)
    np.testing.assert_array_equal(c32.numpy(), acc_ref)
    c16 = _run(ascq_gpu, A, B, bias, ascq_gpu.F16, words=words)
    np.testing.assert_array_equal(_bits(c16), O.mm_dequant(acc_ref, O.F16, qvec=words))


@pytest.mark.parametrize("c_type", ["f16", "bf16"])
@pytest.mark.parametrize("vector", [False, True])
@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("shape", [(128, 256, 512), (77, 200, 96), (300, 132, 1040), (1, 16, 16), (1024, 1024, 1024),
                                   (600, 272, 1040), (520, 200, 96)])
def test_int8_matmul_variants(ascq_gpu, oracle, c_type, vector, trans_b, shape):
    rng = seeded(sum(shape) + 3 * vector + trans_b)
    M, N, K = shape
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (N, K) if trans_b else (K, N), dtype=np.int8)
    bias = rng.integers(-(1 << 20), 1 << 20, N, dtype=np.int32)
    acc_ref = O.matmul_i8(A, B, bias, trans_b=trans_b)
    code = ascq_gpu.F16 if c_type == "f16" else ascq_gpu.BF16
    ocode = O.F16 if c_type == "f16" else O.BF16
    if vector:
        words = _quant_words(rng, N, 2.0 ** -20, 2.0 ** -4)
        c = _run(ascq_gpu, A, B, bias, code, words=words, trans_b=trans_b)
        ref = O.mm_dequant(acc_ref, ocode, qvec=words)
    else:
        word = int(np.float32(0.00123).view(np.uint32))
        c = _run(ascq_gpu, A, B, bias, code, scalar=word, trans_b=trans_b)
        ref = O.mm_dequant(acc_ref, ocode, qscalar=word)
    np.testing.assert_array_equal(_bits(c), ref)


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("shape", [(1, 4096, 8192), (16, 12400, 768), (32, 4096, 11008), (29, 4000, 9216), (5, 12300, 512),
                                   (16, 5000, 768)])
def test_int8_decode_split(ascq_gpu, oracle, trans_b, shape):
    """decode-sized batches (M <= 32, K % 256 == 0).  B given [K, N] with long K or wide N: 32 x 128 tiles whose K is
    split over several workgroups of four waves, the int32 partials meeting in the workspace and added (exactly) by a
    second launch before the epilogue -- K split as evenly as its 256-byte units allow (K = 11008: 43 units; K = 512:
    two splits); the other shapes and B given [N, K] take the 32 x 32 K-split tiles.  Ragged N; every epilogue: int32,
    DEQF16 with per-channel words, bf16 with a scalar word, bit-exact vs the oracle"""
    rng = seeded(sum(shape) + trans_b)
    M, N, K = shape
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (N, K) if trans_b else (K, N), dtype=np.int8)
    bias = rng.integers(-(1 << 20), 1 << 20, N, dtype=np.int32)
    acc_ref = O.matmul_i8(A, B, bias, trans_b=trans_b)
    np.testing.assert_array_equal(_run(ascq_gpu, A, B, bias, ascq_gpu.INT32, trans_b=trans_b).numpy(), acc_ref)
    words = _quant_words(rng, N, 2.0 ** -20, 2.0 ** -4)
    c = _run(ascq_gpu, A, B, bias, ascq_gpu.F16, words=words, trans_b=trans_b)
    np.testing.assert_array_equal(_bits(c), O.mm_dequant(acc_ref, O.F16, qvec=words))
    word = int(np.float32(0.00123).view(np.uint32))
    c = _run(ascq_gpu, A, B, bias, ascq_gpu.BF16, scalar=word, trans_b=trans_b)
    np.testing.assert_array_equal(_bits(c), O.mm_dequant(acc_ref, O.BF16, qscalar=word))


def test_int8_matmul_int32_big(ascq_gpu, oracle):
    rng = seeded(9)
    M, N, K = 2048, 1536, 2048
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    c = _run(ascq_gpu, A, B, None, ascq_gpu.INT32)
    # exact in float64 BLAS: |sum| < 2^53
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64).astype(np.int32)
    np.testing.assert_array_equal(c.numpy(), ref)


def test_deqf16_saturation_and_sign(ascq_gpu, oracle):
    """DEQF16 saturates to +-65504; negative and power-of-two scales; acc = 0."""
    M, K, N = 32, 64, 64
    A = np.full((M, K), 127, np.int8)
    A[1] = -127
    A[2] = 0
    B = np.full((K, N), 127, np.int8)
    s = np.full(N, 1.0, np.float32)
    s[1::4] = -0.5
    s[2::4] = 2.0 ** -10
    s[3::4] = 123.456  # acc*s far beyond 65504 -> saturates
    words = s.view(np.uint32).astype(np.uint64)
    c = _run(ascq_gpu, A, B, None, ascq_gpu.F16, words=words)
    ref = O.mm_dequant(O.matmul_i8(A, B), O.F16, qvec=words)
    got = _bits(c)
    np.testing.assert_array_equal(got, ref)
    # saturation to +-65504; acc = 0 gives +-0 (IEEE: 0 * negative scale = -0)
    assert (got[0, 3::4] == 0x7BFF).all() and (got[1, 3::4] == 0xFBFF).all() and ((got[2] & 0x7FFF) == 0).all()


def test_single_shape_block(ascq_gpu, oracle):
    """SetSingleShape / SetTail: compute one block of a larger matrix with org-shape leading dimensions,
    the way the reference kernel offsets its GlobalTensors per core (matmul_quant.asc:135-154)."""
    rng = seeded(5)
    M, N, K = 256, 512, 256
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    ref = O.matmul_i8(A, B)
    a_d, b_d = _dev(A), _dev(B)
    c = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    m0, n0, bm, bn = 64, 128, 100, 200
    mm = ascq_gpu.Matmul(ascq_gpu.INT8, ascq_gpu.INT8, ascq_gpu.INT32)
    mm.SetOrgShape(M, N, K)
    mm.SetSingleShape(128, 256, K)
    mm.SetTail(bm, bn)
    mm.SetTensorA(a_d.data_ptr() + m0 * K)
    mm.SetTensorB(b_d.data_ptr() + n0)
    mm.IterateAll(c.data_ptr() + (m0 * N + n0) * 4)
    mm.End()
    got = c.cpu().numpy()
    np.testing.assert_array_equal(got[m0:m0 + bm, n0:n0 + bn], ref[m0:m0 + bm, n0:n0 + bn])
    mask = np.ones_like(got, bool)
    mask[m0:m0 + bm, n0:n0 + bn] = False
    assert (got[mask] == 0).all()


# --------------------------------------------------------------------------- int4b_t A / B (W4A4)
def pack_int4_rows(x):
    """int values in [-8, 7], [R, C] (C even) -> [R, C/2] bytes, the packing of matmul_int4/scripts/gen_data.py:
    byte = (x[j + 1] << 4) + (x[j] & 0xF) in int8 arithmetic"""
    x = np.asarray(x, np.int8)
    return ((x[:, 1::2].astype(np.int32) << 4) + (x[:, 0::2].astype(np.int32) & 0xF)).astype(np.int8)


def _run4(ascq, A4, B4, M, N, K, c_type, bias=None, words=None, trans_b=False, trans_a=False):
    torch_c = {ascq.F16: torch.float16, ascq.INT32: torch.int32}[c_type]
    mm = ascq.Matmul(ascq.INT4, ascq.INT4, c_type, ascq.INT32 if bias is not None else 0)
    mm.SetOrgShape(M, N, K)
    if words is not None:
        mm.SetQuantVector(_dev(words.view(np.int64)))
    mm.SetTensorA(_dev(A4), trans_a)
    mm.SetTensorB(_dev(B4), trans_b)
    if bias is not None:
        mm.SetBias(_dev(bias))
    c = torch.empty((M, N), dtype=torch_c, device="cuda")
    mm.IterateAll(c)
    mm.End()
    torch.cuda.synchronize()
    return c.cpu().numpy()


def test_int4_matmul_sample_shape(ascq_gpu, oracle):
    """the matmul_int4 sample: M = 256, N = 7680, K = 128, values from uniform(-5, 5) cast to int8 (so -4..4),
    int32 bias, int32 C; golden = int32 A @ B + bias (gen_data.py)"""
    rng = seeded(404)
    M, N, K = 256, 7680, 128
    x1 = rng.uniform(-5, 5, (M, K)).astype(np.int8)
    x2 = rng.uniform(-5, 5, (K, N)).astype(np.int8)
    bias = rng.uniform(-5, 5, N).astype(np.int32)
    golden = x1.astype(np.int64) @ x2.astype(np.int64) + bias
    got = _run4(ascq_gpu, pack_int4_rows(x1), pack_int4_rows(x2), M, N, K, ascq_gpu.INT32, bias=bias)
    assert np.array_equal(got, golden.astype(np.int32))


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("shape", [(200, 136, 208), (1024, 1024, 1024), (6, 18, 34)])
def test_int4_matmul_deqf16(ascq_gpu, oracle, trans_b, shape):
    """full int4 range, per-channel DEQF16: bit-exact vs the oracle's int32 sums and epilogue; B given [K, N]
    (packed along N) or [N, K] (isTransposeB, packed along K)"""
    M, N, K = shape
    rng = seeded(M + N + K + 7 * trans_b)
    a = rng.integers(-8, 8, (M, K)).astype(np.int8)
    b = rng.integers(-8, 8, (K, N)).astype(np.int8)
    bias = rng.integers(-(1 << 10), 1 << 10, N).astype(np.int32)
    words = _quant_words(rng, N, 2.0 ** -6, 2.0 ** -1)
    B4 = pack_int4_rows(np.ascontiguousarray(b.T)) if trans_b else pack_int4_rows(b)
    got = _run4(ascq_gpu, pack_int4_rows(a), B4, M, N, K, ascq_gpu.F16, bias=bias, words=words, trans_b=trans_b)
    acc = O.matmul_i8(a, b, bias=bias)
    exp = O.mm_dequant(acc, O.F16, qvec=words)
    assert np.array_equal(got.view(np.uint16), exp)


def test_int4_a_transposed_rejected(ascq_gpu, oracle):
    """matmul_int4 README: an int4 A cannot be transposed"""
    a = np.zeros((16, 8), np.int8)
    with pytest.raises(ascq_gpu.AscqError):
        _run4(ascq_gpu, a, a, 16, 16, 16, ascq_gpu.INT32, trans_a=True)
