"""GPU parity: weight-only antiquant matmul (W4A16 / W8A16) vs the oracle.

The dequantised weights follow AscendAntiQuant bit-exactly; the dot products accumulate in fp32, whose
order differs from any reference, so the output is checked against the exact (fp64) sum with the rigorous
bound  |y - s| <= ulp16(|s| + d)/2 + d,  d = K * 2^-24 * sum|x*w|  (fp32 summation error bound), and most
outputs must equal the correctly rounded exact sum."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _ulp16(v):
    a = np.maximum(np.abs(v), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(a)) - 10)


def make_weights(rng, K, N, w_type, group, with_offset=True):
    G = K // group if group else 1
    if w_type == O.INT8:
        w = rng.integers(-128, 128, (K, N), dtype=np.int8)
    else:
        nib = rng.integers(0, 16, K * N, dtype=np.uint8)
        w = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8).reshape(K, N // 2)
    scale = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), (G, N))).astype(np.float16)
    offset = rng.uniform(-8, 8, (G, N)).astype(np.float16) if with_offset else None
    return w, scale, offset


def check_close(y_gpu, y_exact, y_abs, K, frac_exact=0.98):
    y = y_gpu.astype(np.float64)
    d = K * 2.0 ** -24 * y_abs
    tol = 0.5 * _ulp16(np.abs(y_exact) + d) + d
    err = np.abs(y - y_exact)
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} outputs outside the fp32-accumulation bound; max err {err.max()}"
    exact = (y_gpu == np.float16(y_exact)).mean()
    assert exact >= frac_exact, f"only {exact:.4f} of outputs equal the correctly rounded sum"


@pytest.mark.parametrize("w_type", ["int4", "int8"])
@pytest.mark.parametrize("M", [1, 16, 64, 3, 29, 40, 100])
def test_config3_decode_shape(ascq_gpu, oracle, w_type, M):
    """x f16 [M, 4096] ~ N(0,1); W [4096, 11008]; g=128 f16 scale log-uniform [1e-3,1e-1], offset U[-8,8]."""
    rng = seeded(300 + M)
    K, N, g = 4096, 11008, 128
    code = O.INT8 if w_type == "int8" else O.INT4
    w, scale, offset = make_weights(rng, K, N, code, g)
    x = rng.standard_normal((M, K)).astype(np.float16)
    wp = ascq_gpu.weight_pack(_dev(w), ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4, K, N)
    y = ascq_gpu.antiquant_matmul(_dev(x), wp, ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4, _dev(scale),
                                  _dev(offset), g, N)
    y_ref, y_exact, y_abs = O.antiquant_matmul(x.view(np.uint16), w, code, scale.view(np.uint16),
                                               offset.view(np.uint16), g, M, N, K)
    check_close(y.cpu().numpy(), y_exact, y_abs, K)


@pytest.mark.parametrize("w_type", ["int4", "int8"])
@pytest.mark.parametrize("group", [0, 32, 64, 256])
@pytest.mark.parametrize("with_offset", [True, False])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("M", [5, 1])
def test_groups_and_layouts(ascq_gpu, oracle, w_type, group, with_offset, transpose, M):
    rng = seeded(17 + group)
    K, N = 512, 96
    code = O.INT8 if w_type == "int8" else O.INT4
    w, scale, offset = make_weights(rng, K, N, code, group, with_offset)
    if transpose:  # weight given [N, K]
        if code == O.INT8:
            w = np.ascontiguousarray(w.T)
        else:
            nib = np.stack([w & 0xF, w >> 4], -1).reshape(K, N)
            t = np.ascontiguousarray(nib.T).reshape(-1)
            w = (t[0::2] | (t[1::2] << 4)).astype(np.uint8)
    x = (rng.standard_normal((M, K)) * 2).astype(np.float16)
    at = ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4
    wp = ascq_gpu.weight_pack(_dev(w), at, K, N, is_transpose=transpose)
    y = ascq_gpu.antiquant_matmul(_dev(x), wp, at, _dev(scale), None if offset is None else _dev(offset), group, N)
    # oracle scale layout is [K/g, N] for the [K, N] weight; for the transposed weight it is [N, K/g]
    sc = scale if not transpose else np.ascontiguousarray(scale.T)
    of = None if offset is None else (offset if not transpose else np.ascontiguousarray(offset.T))
    _, y_exact, y_abs = O.antiquant_matmul(x.view(np.uint16), w, code, sc.view(np.uint16),
                                           None if of is None else of.view(np.uint16), group, M, N, K,
                                           w_transpose=transpose)
    check_close(y.cpu().numpy(), y_exact, y_abs, K)


@pytest.mark.parametrize("w_type", ["int4", "int8"])
@pytest.mark.parametrize("M", [6, 16, 24, 48, 64])
@pytest.mark.parametrize("K", [640, 384])
def test_batch_ring_partial_rounds(ascq_gpu, oracle, w_type, M, K):
    """K = 640 / 384 (5 / 3 k tiles): the waves of a K-split block (M <= 32) get uneven tile counts, one of them none
    at K = 384; batches above 32 rows end their LDS ring in a partial round.  N = 48: three one-strip blocks."""
    rng = seeded(900 + M + K)
    N, g = 48, 128
    code = O.INT8 if w_type == "int8" else O.INT4
    at = ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4
    w, scale, offset = make_weights(rng, K, N, code, g)
    x = rng.standard_normal((M, K)).astype(np.float16)
    wp = ascq_gpu.weight_pack(_dev(w), at, K, N)
    y = ascq_gpu.antiquant_matmul(_dev(x), wp, at, _dev(scale), _dev(offset), g, N)
    _, y_exact, y_abs = O.antiquant_matmul(x.view(np.uint16), w, code, scale.view(np.uint16), offset.view(np.uint16),
                                           g, M, N, K)
    check_close(y.cpu().numpy(), y_exact, y_abs, K)


@pytest.mark.parametrize("w_type", ["int4", "int8"])
@pytest.mark.parametrize("with_offset", [True, False])
@pytest.mark.parametrize("M,K,N,group", [
    (1, 512, 112, 128),      # one k tile per wave: ring slots past the end
    (7, 1536, 1008, 256),    # 3 tiles per wave, group of two tiles
    (16, 4096, 4112, 128),   # 257 strips over 256 blocks: one block of two strips
    (12, 2048, 272, 2048),   # one group over all of K
    (9, 8192, 112, 128),     # x too large for LDS residency: earlier ring form
    (17, 1024, 4112, 128),   # 32-row ring, a single round
    (32, 3072, 1008, 512),
    (33, 512, 112, 128),     # 64-row ring, a single round
    (64, 2048, 4112, 256),
    (50, 4096, 1008, 128),
    (3, 1024, 16384, 128),   # 1024 strips: four per block
    (20, 768, 13072, 256),   # 817 strips: three or four per block, 32 rows
    (5, 512, 16400, 128),    # 1025 strips: 257 K-split blocks of up to four strips (more than one block per CU)
    (20, 512, 16400, 128),   # 1025 strips, 32 rows
    (1, 4096, 32000, 128),   # a vocabulary-sized N, one row: x resident in LDS
    (16, 1024, 32000, 256),  # a vocabulary-sized N: 500 K-split blocks of four strips
    (1, 4096, 1008, 32),     # groups of 32: four scale / offset rows per k tile
    (16, 2048, 4112, 64),    # groups of 64: two per k tile
    (29, 1536, 2000, 32),
    (2, 512, 16400, 64),     # groups of 64 past 1024 strips, one row
    (40, 2048, 1008, 32),    # groups of 32 / 64 above 32 rows: the K-split blocks with four row tiles
    (64, 1024, 4112, 64),
])
def test_column_block_kernels(ascq_gpu, oracle, w_type, with_offset, M, K, N, group):
    """Column blocks of 1 - 4 strips (sizes within one strip of each other): K-split waves with x read into registers
    (M <= 32; about 256 blocks, more above 1024 strips but for a single row), x resident in LDS (one row above 1024
    strips) or x streamed through an LDS ring (M > 32); group sizes 128 << s, and 32 / 64 (the K-split blocks up to
    64 rows), with and without offset."""
    rng = seeded(M * 7 + K + N + group)
    code = O.INT8 if w_type == "int8" else O.INT4
    at = ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4
    w, scale, offset = make_weights(rng, K, N, code, group, with_offset)
    x = rng.standard_normal((M, K)).astype(np.float16)
    wp = ascq_gpu.weight_pack(_dev(w), at, K, N)
    y = ascq_gpu.antiquant_matmul(_dev(x), wp, at, _dev(scale), None if offset is None else _dev(offset), group, N)
    _, y_exact, y_abs = O.antiquant_matmul(x.view(np.uint16), w, code, scale.view(np.uint16),
                                           None if offset is None else offset.view(np.uint16), group, M, N, K)
    check_close(y.cpu().numpy(), y_exact, y_abs, K)


@pytest.mark.parametrize("w_type", ["int4", "int8"])
@pytest.mark.parametrize("M,K,N,group", [
    (1, 1408, 272, 0),       # per channel (one group over K), 11 k tiles: K-split waves with uneven tile counts
    (16, 1408, 272, 0),
    (40, 1408, 272, 0),      # LDS ring of four k-split waves: a partial last round (11 = 2 x 4 + 3)
    (100, 1408, 272, 0),     # row blocks of the ring, partial last round
    (40, 11008, 4096, 128),  # a down projection: 86 k tiles (4 does not divide them), 256 strips
    (200, 11008, 4096, 0),
    (256, 11008, 4096, 128), # 86 scale rows: 64-row blocks of two k-split waves (the wider forms lack LDS for them)
    (48, 28672, 1024, 128),  # 224 scale rows at 48 rows: no LDS for the ring, the K-split blocks with four row tiles
])
def test_partial_rounds_and_per_channel(ascq_gpu, oracle, w_type, M, K, N, group):
    """per-channel scales (group 0: one group over all of K) on the column-block kernels, and k-tile counts that the
    ring's k-split waves do not divide (its last round partial: the tiles past K read zeros)"""
    rng = seeded(M + K + N + group)
    code = O.INT8 if w_type == "int8" else O.INT4
    at = ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4
    w, scale, offset = make_weights(rng, K, N, code, group)
    x = rng.standard_normal((M, K)).astype(np.float16)
    wp = ascq_gpu.weight_pack(_dev(w), at, K, N)
    y = ascq_gpu.antiquant_matmul(_dev(x), wp, at, _dev(scale), _dev(offset), group, N)
    _, y_exact, y_abs = O.antiquant_matmul(x.view(np.uint16), w, code, scale.view(np.uint16), offset.view(np.uint16),
                                           group, M, N, K)
    check_close(y.cpu().numpy(), y_exact, y_abs, K)


@pytest.mark.parametrize("w_type", ["int4", "int8"])
@pytest.mark.parametrize("with_offset", [True, False])
@pytest.mark.parametrize("M,K,N,group", [
    (65, 512, 112, 128),      # one row past the decode kernels; a single column block narrower than the tile
    (200, 1024, 4112, 256),   # partial row block; 257 strips: the last column block holds one strip
    (128, 2048, 272, 2048),   # one group over all of K
    (1000, 768, 1008, 128),   # eight row blocks, the last one partial
    (300, 640, 272, 128),     # K = 5 tiles of 128: the LDS-staged MFMA GEMM (the ring kernels split K in 2 or 4)
])
def test_prefill_gemm(ascq_gpu, oracle, w_type, with_offset, M, K, N, group):
    """M > 64: the ring kernel over row blocks (64-row blocks while they make about one block per CU, else 128-row
    blocks) or, for K not a multiple of 256, the LDS-staged MFMA GEMM of aq_gemm.hip; the weights bit-exact as
    AscendAntiQuant, fp32 accumulation within the bound of check_close"""
    rng = seeded(M + K + N + group + with_offset)
    code = O.INT8 if w_type == "int8" else O.INT4
    at = ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4
    w, scale, offset = make_weights(rng, K, N, code, group, with_offset)
    x = rng.standard_normal((M, K)).astype(np.float16)
    wp = ascq_gpu.weight_pack(_dev(w), at, K, N)
    y = ascq_gpu.antiquant_matmul(_dev(x), wp, at, _dev(scale), None if offset is None else _dev(offset), group, N)
    _, y_exact, y_abs = O.antiquant_matmul(x.view(np.uint16), w, code, scale.view(np.uint16),
                                           None if offset is None else offset.view(np.uint16), group, M, N, K)
    check_close(y.cpu().numpy(), y_exact, y_abs, K)


@pytest.mark.parametrize("w_type", ["int4", "int8"])
def test_prefill_gemm_config3_weight(ascq_gpu, oracle, w_type):
    """M = 512 prefill rows against the config-3 weight (K = 4096, N = 11008, g = 128, f16 scale and offset): every
    output of 64 sampled rows (16 in each 128 rows, the first and last rows among them)"""
    rng = seeded(512)
    M, K, N, g = 512, 4096, 11008, 128
    code = O.INT8 if w_type == "int8" else O.INT4
    at = ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4
    w, scale, offset = make_weights(rng, K, N, code, g)
    x = rng.standard_normal((M, K)).astype(np.float16)
    wp = ascq_gpu.weight_pack(_dev(w), at, K, N)
    y = ascq_gpu.antiquant_matmul(_dev(x), wp, at, _dev(scale), _dev(offset), g, N).cpu().numpy()
    rows = np.unique(np.concatenate([[0, M - 1]] + [b + rng.choice(128, 16, replace=False) for b in range(0, M, 128)]))
    _, y_exact, y_abs = O.antiquant_matmul(np.ascontiguousarray(x[rows]).view(np.uint16), w, code,
                                           scale.view(np.uint16), offset.view(np.uint16), g, len(rows), N, K)
    check_close(y[rows], y_exact, y_abs, K)


@pytest.mark.parametrize("w_type", ["int4", "int8"])
@pytest.mark.parametrize("b_format", ["nd", "packed"])
def test_matmul_handle_antiquant(ascq_gpu, oracle, w_type, b_format):
    """Matmul<half, int8|int4, half> with SetAntiQuantVector (per group) and SetAntiQuantScalar."""
    rng = seeded(23)
    K, N, M, g = 256, 64, 7, 128
    code = O.INT8 if w_type == "int8" else O.INT4
    at = ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4
    w, scale, offset = make_weights(rng, K, N, code, g)
    x = rng.standard_normal((M, K)).astype(np.float16)
    fmt = ascq_gpu.FORMAT_ND if b_format == "nd" else ascq_gpu.FORMAT_PACKED
    wd = _dev(w) if b_format == "nd" else ascq_gpu.weight_pack(_dev(w), at, K, N)
    for mode in ("vector", "scalar"):
        mm = ascq_gpu.Matmul(ascq_gpu.F16, at, ascq_gpu.F16, b_format=fmt)
        mm.SetOrgShape(M, N, K)
        mm.SetTensorA(_dev(x))
        mm.SetTensorB(wd)
        if mode == "vector":
            mm.SetAntiQuantVector(_dev(offset), _dev(scale), g)
            sc, of, gg = scale, offset, g
        else:
            mm.SetAntiQuantScalar(1.5, 0.0123)
            sc = np.full((1, N), 0.0123, np.float16)
            of = np.full((1, N), 1.5, np.float16)
            gg = 0
        y = torch.empty((M, N), dtype=torch.float16, device="cuda")
        mm.IterateAll(y)
        mm.End()
        _, y_exact, y_abs = O.antiquant_matmul(x.view(np.uint16), w, code, sc.view(np.uint16), of.view(np.uint16),
                                               gg, M, N, K)
        check_close(y.cpu().numpy(), y_exact, y_abs, K)
