"""GPU parity: quantized group matmul (MoE) vs the oracle, bit-exact (int32 accumulate + fp32 epilogue)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import group_cases as GC
import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def zipf_counts(rng, tokens, experts, s=1.1):
    p = 1.0 / (np.arange(1, experts + 1) ** s)
    p /= p.sum()
    return rng.multinomial(tokens, p).astype(np.int64)


def bf16_bits_of_f32(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("list_type", [0, 1])
@pytest.mark.parametrize("w_trans", [False, True])
@pytest.mark.parametrize("out", ["bf16", "f16"])
@pytest.mark.parametrize("K", [320, 384])
def test_group_matmul_small(ascq_gpu, oracle, list_type, w_trans, out, K):
    rng = seeded(40 + list_type + 2 * w_trans)
    G, N = 5, 160
    counts = np.array([70, 0, 133, 1, 96], np.int64)  # includes an empty and a single-row group
    M = int(counts.sum()) + 9  # trailing rows belong to no group and must stay untouched
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (G, N, K) if w_trans else (G, K, N), dtype=np.int8)
    pts = rng.normal(0, 0.01, M).astype(np.float32)
    scale = rng.normal(0, 0.01, (G, N)).astype(np.float32)
    gl = np.concatenate([[0], np.cumsum(counts)]) if list_type == 0 else counts
    ycode, tdt = (O.BF16, torch.bfloat16) if out == "bf16" else (O.F16, torch.float16)
    y = torch.full((M, N), 3.0, dtype=tdt, device="cuda")
    ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), _dev(w), _dev(scale), _dev(gl), list_type, w_trans, tdt, out=y)
    y0 = torch.full((M, N), 3.0, dtype=tdt).view(torch.int16).numpy().view(np.uint16).copy()
    ref = O.group_matmul(x, pts, w, scale, gl, list_type, G, M, K, N, ycode, w_trans, y=y0)
    np.testing.assert_array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), ref)


@pytest.mark.parametrize("w_trans", [False, True])
def test_config4_moe_full_size(ascq_gpu, oracle, w_trans):
    """16 experts, 4096 tokens routed by a seeded multinomial (Zipf s=1.1), K=4096, N=1408, int64 prefix-sum
    offsets, bf16 out; the expert weights given [G, K, N] or K-contiguous [G, N, K].  Reference: exact int
    accumulators from fp64 BLAS (|acc| < 2^53), then the epilogue f32(f32(acc)*scale[g,n])*pts[m] in numpy float32
    (f32(acc) ties away from zero) and torch's rne bfloat16 cast."""
    rng = seeded(4)
    G, T, K, N = 16, 4096, 4096, 1408
    counts = zipf_counts(rng, T, G)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    x = rng.integers(-127, 128, (T, K), dtype=np.int8)
    pts = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), T)).astype(np.float32)
    w = rng.integers(-127, 128, (G, K, N), dtype=np.int8)
    scale = np.exp(rng.uniform(np.log(1e-4), np.log(1e-2), (G, N))).astype(np.float32)
    w_dev = _dev(np.ascontiguousarray(w.transpose(0, 2, 1))) if w_trans else _dev(w)
    y = ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), w_dev, _dev(scale), _dev(offsets), 0, w_trans)
    got = y.cpu().view(torch.int16).numpy().view(np.uint16)
    xf = x.astype(np.float64)
    for g in range(G):
        s, e = offsets[g], offsets[g + 1]
        if e == s:
            continue
        acc = GC.i32_to_f32_rna((xf[s:e] @ w[g].astype(np.float64)).astype(np.int64))  # ties away above 2^24
        v = (acc * scale[g][None, :]).astype(np.float32) * pts[s:e, None]
        np.testing.assert_array_equal(got[s:e], bf16_bits_of_f32(v.astype(np.float32)), err_msg=f"group {g}")


@pytest.mark.parametrize("w_trans", [False, True])
@pytest.mark.parametrize("list_type", [0, 1])
def test_group_ties_above_2_24(ascq_gpu, oracle, w_trans, list_type):
    """Accumulators on fp32 ties in [2^24, 2^26) with scales chosen so that the int32 -> fp32 rounding rule shows in
    the bf16 output: the group epilogue rounds ties away from zero, as AscendDequant does
    (ascend_dequant_3510_impl.h:61); bit-exact against the oracle and the numpy restatement, and more than 50 outputs
    differ from what a nearest-even conversion gives."""
    x, w, pts, sc, counts = GC.tie_case(11)
    M, K = x.shape
    G, _, N = w.shape
    gl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64) if list_type == 0 else counts
    w_dev = _dev(np.ascontiguousarray(w.transpose(0, 2, 1))) if w_trans else _dev(w)
    y = ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), w_dev, _dev(sc), _dev(gl), list_type, w_trans)
    got = y.cpu().view(torch.int16).numpy().view(np.uint16)
    ref = O.group_matmul(x, pts, w, sc, gl, list_type, G, M, K, N, O.BF16)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, GC.group_reference(x, w, pts, sc, counts))
    assert GC.rne_differs(x, w, pts, sc, counts) > 50


@pytest.mark.parametrize("T,K,N", [(1, 512, 160), (16, 1024, 256), (64, 768, 96), (200, 4096, 1408), (150, 1024, 208)])
@pytest.mark.parametrize("w_trans", [False, True])
@pytest.mark.parametrize("list_type", [0, 1])
def test_group_decode_ksplit(ascq_gpu, oracle, T, K, N, w_trans, list_type):
    """decode-sized MoE batches (at most 16 rows per expert on average, K % 256 == 0): 32 x 32 tiles with each
    tile's K split over four waves (int32 partials, exact); 16 Zipf-ragged experts, a leading offset and trailing
    rows outside every group, bit-exact vs the oracle"""
    G = 16
    rng = seeded(T + K + N + 2 * w_trans + list_type)
    counts = zipf_counts(rng, T, G)
    lead = 3
    M = lead + T + 5
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    pts = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), M)).astype(np.float32)
    w = rng.integers(-127, 128, (G, N, K) if w_trans else (G, K, N), dtype=np.int8)
    scale = np.exp(rng.uniform(np.log(1e-4), np.log(1e-2), (G, N))).astype(np.float32)
    # offsets start at row `lead`; counts start at row 0 (the rows past the last group stay untouched either way)
    gl = (np.concatenate([[lead], lead + np.cumsum(counts)]) if list_type == 0 else counts).astype(np.int64)
    y = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), _dev(w), _dev(scale), _dev(gl), list_type, w_trans, out=y)
    y0 = torch.full((M, N), 3.0, dtype=torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()
    ref = O.group_matmul(x, pts, w, scale, gl, list_type, G, M, K, N, O.BF16, w_trans, y=y0)
    np.testing.assert_array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), ref)


@pytest.mark.parametrize("w_trans", [False, True])
def test_group_decode_ties_above_2_24(ascq_gpu, oracle, w_trans):
    """the fp32-tie accumulators of test_group_ties_above_2_24 over eight 8-row experts (the K-split 32 x 32 tiles):
    the four waves' int32 partials add exactly, and the group epilogue rounds ties away from zero"""
    x, w, pts, sc, counts = GC.tie_case(13, M=64, N=64, K=4096, groups=(8,) * 8)
    M, K = x.shape
    G, _, N = w.shape
    gl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    w_dev = _dev(np.ascontiguousarray(w.transpose(0, 2, 1))) if w_trans else _dev(w)
    y = ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), w_dev, _dev(sc), _dev(gl), 0, w_trans)
    got = y.cpu().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, O.group_matmul(x, pts, w, sc, gl, 0, G, M, K, N, O.BF16))
    np.testing.assert_array_equal(got, GC.group_reference(x, w, pts, sc, counts))
    assert GC.rne_differs(x, w, pts, sc, counts) > 20


def _f16_ulp(v):
    a = np.maximum(np.abs(v), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(a)) - 10)


@pytest.mark.parametrize("w_trans", [False, True])
@pytest.mark.parametrize("out", ["f16", "bf16"])
def test_group_matmul_faster_gelu(ascq_gpu, oracle, w_trans, out):
    """the sample's epilogue with FasterGelu (quant_group_matmul_custom.asc:442-450): device and oracle both run
    the fp32 op sequence x / (1 + exp(-1.702 x)); the device's expf may differ from the correctly rounded exp by
    an fp32 ulp, so outputs agree within one output ulp, and bit-exactly on >= 99 %"""
    rng = seeded(77 + w_trans)
    G, K, N = 6, 512, 272
    counts = np.array([300, 0, 17, 1, 250, 90], np.int64)
    M = int(counts.sum())
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (G, N, K) if w_trans else (G, K, N), dtype=np.int8)
    pts = rng.normal(0, 0.01, M).astype(np.float32)
    scale = rng.normal(0, 0.01, (G, N)).astype(np.float32)  # |v| up to ~ a few: the curved part of the Gelu
    ycode, tdt = (O.BF16, torch.bfloat16) if out == "bf16" else (O.F16, torch.float16)
    y = ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), _dev(w), _dev(scale), _dev(counts), 1, w_trans, tdt,
                                    activation=ascq_gpu.ACT_FASTER_GELU)
    got = y.cpu().to(torch.float64).numpy()
    ref_bits = O.group_matmul(x, pts, w, scale, counts, 1, G, M, K, N, ycode, w_trans, act=1)
    ref = torch.from_numpy(ref_bits.view(np.int16)).view(tdt).to(torch.float64).numpy()
    ulp = _f16_ulp(ref) if out == "f16" else 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    assert (np.abs(got - ref) <= ulp).all()
    assert (got == ref).mean() >= 0.99


def test_group_matmul_gelu_sample_golden(ascq_gpu, oracle):
    """the restated sample golden with FastGelu (tests/golden/group_matmul_gelu_example.npz), judged by the
    sample's verify_result.py criterion (isclose rtol = atol = 1e-3, error ratio <= 1e-4)"""
    from pathlib import Path

    f = np.load(Path(__file__).resolve().parent / "golden" / "group_matmul_gelu_example.npz")
    y = ascq_gpu.quant_group_matmul(_dev(f["x"]), _dev(f["pts"]), _dev(f["weight"]), _dev(f["scale"]),
                                    _dev(f["group_list"]), 1, False, torch.float16,
                                    activation=ascq_gpu.ACT_FASTER_GELU)
    out = y.cpu().numpy().astype(np.float64)
    bad = ~np.isclose(out, f["golden"].astype(np.float64), rtol=1e-3, atol=1e-3)
    assert bad.mean() <= 1e-4


@pytest.mark.parametrize("G,list_type,w_trans,K", [(128, 0, True, 512), (128, 1, False, 512), (256, 1, True, 1024),
                                                   (1024, 0, True, 256)])
def test_many_experts_zipf(ascq_gpu, oracle, G, list_type, w_trans, K):
    """128 to 1024 experts with Zipf(1.1)-ragged groups (most of them empty or a handful of rows): the MFMA kernel
    takes up to 1024 groups (the table is a block-wide prefix sum, no per-group LDS), bit-exact vs the oracle.
    The sample's group list forms: prefix offsets (list_type 0) and counts (1); a leading offset > 0 and trailing
    rows outside every group stay untouched."""
    rng = seeded(G + K + list_type)
    T, N = 4096, 256
    counts = zipf_counts(rng, T, G)
    lead = 5
    M = lead + T + 7
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    pts = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), M)).astype(np.float32)
    w = rng.integers(-127, 128, (G, N, K) if w_trans else (G, K, N), dtype=np.int8)
    scale = np.exp(rng.uniform(np.log(1e-4), np.log(1e-2), (G, N))).astype(np.float32)
    if list_type == 0:
        gl = np.concatenate([[lead], lead + np.cumsum(counts)]).astype(np.int64)
    else:
        gl = counts.astype(np.int64)
    y = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), _dev(w), _dev(scale), _dev(gl), list_type, w_trans, out=y)
    y0 = torch.full((M, N), 3.0, dtype=torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()
    ref = O.group_matmul(x, pts, w, scale, gl, list_type, G, M, K, N, O.BF16, w_trans, y=y0)
    np.testing.assert_array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), ref)


@pytest.mark.parametrize("N,shift", [(150, 0), (162, 0), (160, 1)])
@pytest.mark.parametrize("w_trans", [False, True])
def test_group_matmul_store_fallback(ascq_gpu, oracle, N, shift, w_trans):
    """Output rows that are not whole 8-byte quads (N % 4 != 0) or a Y that is not 8-byte aligned (a view one
    element into its buffer) take the element-wise stores of the tiled kernel (w_trans) or the generic kernel; both
    bit-exact vs the oracle, and nothing outside Y is written."""
    rng = seeded(700 + N + shift + w_trans)
    G, K = 4, 256
    counts = np.array([97, 0, 140, 33], np.int64)
    M = int(counts.sum()) + 3
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (G, N, K) if w_trans else (G, K, N), dtype=np.int8)
    pts = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), M)).astype(np.float32)
    scale = np.exp(rng.uniform(np.log(1e-4), np.log(1e-2), (G, N))).astype(np.float32)
    gl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    buf = torch.full((M * N + 2 * shift,), 3.0, dtype=torch.float16, device="cuda")
    y = buf[shift:shift + M * N].view(M, N)
    ascq_gpu.quant_group_matmul(_dev(x), _dev(pts), _dev(w), _dev(scale), _dev(gl), 0, w_trans, torch.float16, out=y)
    y0 = torch.full((M, N), 3.0, dtype=torch.float16).view(torch.int16).numpy().view(np.uint16).copy()
    ref = O.group_matmul(x, pts, w, scale, gl, 0, G, M, K, N, O.F16, w_trans, y=y0)
    got = buf.cpu().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got[shift:shift + M * N].reshape(M, N), ref)
    three = np.float16(3.0).view(np.uint16)
    assert (got[:shift] == three).all() and (got[shift + M * N:] == three).all()
