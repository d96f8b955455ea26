"""GPU parity: AscendQuant policy form (arch 3510; PER_TOKEN / PER_GROUP to int8, fp8 e4m3 / e5m2 and E2M1) through
the C ABI, bit-exact against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu

_TD = {O.F16: torch.float16, O.BF16: torch.bfloat16, O.F32: torch.float32}
_MODES = [O.ROUND_RINT, O.ROUND_FLOOR, O.ROUND_CEIL, O.ROUND_ROUND, O.ROUND_TRUNC, O.ROUND_NONE]


def _bits(v, t):
    """float64 values -> the host array of type t (f16 / bf16 as uint16 bit patterns)"""
    if t == O.F16:
        return v.astype(np.float16).view(np.uint16)
    if t == O.BF16:
        return torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return v.astype(np.float32)


def _dev(a, t=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return x.view(_TD[t]) if t in (O.F16, O.BF16) else x


def _sshape(policy, m, n, g, k_dim):
    if policy == O.PER_TOKEN:
        return (m,)
    return (m, (n + g - 1) // g) if k_dim == 1 else ((m + g - 1) // g, n)


def _run(ascq, x, st, sc, sct, dst, policy, m, n, g=0, of=None, osc=None, k_dim=1, mode=O.ROUND_RINT):
    q = ascq.ascend_quant_policy(_dev(x, st), _dev(sc, sct), policy, dst, g, None if of is None else _dev(of, sct),
                                 osc, k_dim, mode, scale_type=sct)
    torch.cuda.synchronize()
    return q.cpu().numpy().view(np.uint8)


def _check(ascq, x, st, sc, sct, dst, policy, m, n, g=0, of=None, osc=None, k_dim=1, mode=O.ROUND_RINT):
    got = _run(ascq, x, st, sc, sct, dst, policy, m, n, g, of, osc, k_dim, mode)
    exp = O.quant_policy(x, st, sc, sct, dst, policy, m, n, g, of, osc, k_dim, mode).view(np.uint8)
    bad = int((got != exp).sum())
    assert bad == 0, (dst, policy, k_dim, mode, bad, np.argwhere(got != exp)[:4].tolist())


def _src(rng, m, n, t, lo, hi):
    v = rng.uniform(lo, hi, (m, n))
    v.flat[:6] = [np.nan, np.inf, -np.inf, 0.5, -2.5, 1e30]  # NaN, infinities, ties, overflow (f16: inf)
    return _bits(v, t)


_PAIRS = [(O.F16, O.F16), (O.BF16, O.BF16), (O.F32, O.F32), (O.F16, O.F32), (O.BF16, O.F32)]
_LAYOUTS = [(O.PER_TOKEN, 0, 1), (O.PER_GROUP, 32, 1), (O.PER_GROUP, 64, 0)]


@pytest.mark.parametrize("pair", _PAIRS)
@pytest.mark.parametrize("layout", _LAYOUTS)
@pytest.mark.parametrize("shape", [(75, 160), (37, 96), (37, 100)])  # vector path (m % 4 of 3 and 1), ragged rows
def test_int8(ascq_gpu, pair, layout, shape):
    st, sct = pair
    policy, g, k_dim = layout
    m, n = shape
    rng = seeded(1100 + 10 * st + sct + g + k_dim + n)
    x = _src(rng, m, n, st, -200.0, 200.0)
    ss = _sshape(policy, m, n, g, k_dim)
    sc = _bits(rng.uniform(0.05, 2.0, ss), sct)
    of = _bits(rng.uniform(-9.0, 9.0, ss), sct)
    for i, mode in enumerate(_MODES):
        offs = [(of, None), (None, 0.3), (None, None)][i % 3]
        _check(ascq_gpu, x, st, sc, sct, O.INT8, policy, m, n, g, offs[0], offs[1], k_dim, mode)


@pytest.mark.parametrize("fmt", [O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("pair", _PAIRS + [(O.F32, O.F16), (O.F16, O.BF16)])
def test_fp8(ascq_gpu, fmt, pair):
    st, sct = pair
    m, n = 64, 192
    rng = seeded(1200 + fmt + 10 * st + sct)
    v = rng.standard_normal((m, n)) * np.exp2(rng.integers(-14, 17, (m, n)))
    v.flat[:5] = [np.nan, np.inf, -np.inf, 7e4, -7e4]
    x = _bits(v, st)
    for policy, g, k_dim in _LAYOUTS:
        ss = _sshape(policy, m, n, g, k_dim)
        sc = _bits(rng.uniform(0.25, 4.0, ss), sct)
        of = _bits(rng.uniform(-2.0, 2.0, ss), sct)
        _check(ascq_gpu, x, st, sc, sct, fmt, policy, m, n, g, of, None, k_dim)
        _check(ascq_gpu, x, st, sc, sct, fmt, policy, m, n, g, None, -1.7, k_dim, O.ROUND_FLOOR)  # mode unused


@pytest.mark.parametrize("pair", _PAIRS)
@pytest.mark.parametrize("k_dim", [0, 1])
@pytest.mark.parametrize("fp4", [O.FP4_E2M1, O.FP4_E1M2])
def test_e2m1(ascq_gpu, pair, k_dim, fp4):
    """fp4 outputs (E2M1 and E1M2) in every round mode, with the tie points of both code tables"""
    st, sct = pair
    m, n, g = 96, 128, 32
    rng = seeded(1300 + 10 * st + sct + k_dim + 7 * fp4)
    v = rng.uniform(-8.0 if fp4 == O.FP4_E2M1 else -2.5, 8.0 if fp4 == O.FP4_E2M1 else 2.5, (m, n))
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 7.0, -0.25, -0.75, -2.5, -5.0, 0.3, -0.3, 1e9,
                     0.125, 0.375, 0.625, 0.875, 1.125, 1.375, 1.625, -0.125, -1.375, -1.625, 1.8, -1.9, 0.1, -0.1])
    v[0, :ties.size] = ties
    v[1, :3] = [np.nan, np.inf, -np.inf]
    x = _bits(v, st)
    ss = _sshape(O.PER_GROUP, m, n, g, k_dim)
    s = rng.uniform(0.5, 1.5, ss)
    s[0] = 1.0  # row 0 / row group 0: the ties reach the cast unchanged
    sc = _bits(s, sct)
    of = _bits(np.full(ss, 3.0), sct)  # ignored for fp4
    for mode in _MODES:
        _check(ascq_gpu, x, st, sc, sct, fp4, O.PER_GROUP, m, n, g, of, None, k_dim, mode)


def test_unaligned_pointers(ascq_gpu):
    """a source or scale one element off a 16-byte boundary takes the per-element path"""
    m, n, g = 40, 256, 64
    rng = seeded(1400)
    x = _bits(rng.uniform(-100.0, 100.0, (m, n)), O.F16)
    sc = _bits(rng.uniform(0.1, 2.0, ((m + g - 1) // g, n)), O.F16)
    xd = torch.empty(m * n + 1, dtype=torch.float16, device="cuda")
    xd[1:] = _dev(x.reshape(-1), O.F16)
    sd = torch.empty(sc.size + 1, dtype=torch.float16, device="cuda")
    sd[1:] = _dev(sc.reshape(-1), O.F16)
    for dst in (O.INT8, O.FP8_E4M3, O.FP4_E2M1, O.FP4_E1M2):
        q = ascq_gpu.ascend_quant_policy(xd[1:].view(m, n), sd[1:], O.PER_GROUP, dst, g, k_dim=0)
        torch.cuda.synchronize()
        exp = O.quant_policy(x, O.F16, sc, O.F16, dst, O.PER_GROUP, m, n, g, k_dim=0).view(np.uint8)
        assert np.array_equal(q.cpu().numpy().view(np.uint8), exp), dst


def test_per_token_matches_fp32_entry(ascq_gpu):
    """PER_TOKEN int8 with f32 scale / offset gives the same bytes as the f32 per-token entry point"""
    m, n = 128, 1024
    rng = seeded(1500)
    x = torch.from_numpy(rng.uniform(-300.0, 300.0, (m, n)).astype(np.float16)).cuda()
    s = torch.from_numpy(rng.uniform(0.01, 1.0, m).astype(np.float32)).cuda()
    o = torch.from_numpy(rng.uniform(-3.0, 3.0, m).astype(np.float32)).cuda()
    for mode in (O.ROUND_RINT, O.ROUND_CEIL):
        a = ascq_gpu.ascend_quant_policy(x, s, O.PER_TOKEN, O.INT8, offset=o, round_mode=mode)
        b = ascq_gpu.quant_per_token(x, s, o, round_mode=mode)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


def test_full_size_group_int8_and_e2m1(ascq_gpu):
    """[8192, 8192] f16 source, groups of 128 along the rows (kDim 1; int8 and E2M1) and down the columns (kDim 0;
    int8), against the oracle"""
    m, n, g = 8192, 8192, 128
    rng = seeded(1600)
    x = rng.standard_normal((m, n), dtype=np.float32).astype(np.float16).view(np.uint16)
    sc = _bits(rng.uniform(0.5, 40.0, (m, n // g)), O.F16)
    for dst in (O.INT8, O.FP4_E2M1):
        _check(ascq_gpu, x, O.F16, sc, O.F16, dst, O.PER_GROUP, m, n, g, None, None, 1)
    sc0 = _bits(rng.uniform(0.5, 40.0, (m // g, n)), O.F16)  # groups of 128 rows (kDim 0)
    _check(ascq_gpu, x, O.F16, sc0, O.F16, O.INT8, O.PER_GROUP, m, n, g, None, None, 0)


def test_argument_checks(ascq_gpu):
    x = torch.zeros((4, 64), dtype=torch.float16, device="cuda")
    s16 = torch.ones(4, dtype=torch.bfloat16, device="cuda")
    s = torch.ones((4, 2), dtype=torch.float16, device="cuda")
    with pytest.raises(ascq_gpu.AscqError):  # int8 with a bf16 scale needs a bf16 source
        ascq_gpu.ascend_quant_policy(x, s16, O.PER_TOKEN, O.INT8)
    with pytest.raises(ascq_gpu.AscqError):  # PER_TOKEN writes int8 or fp8
        ascq_gpu.ascend_quant_policy(x, s16.half(), O.PER_TOKEN, O.FP4_E2M1)
    with pytest.raises(ascq_gpu.AscqError):  # group size must be a multiple of 32
        ascq_gpu.ascend_quant_policy(x, s, O.PER_GROUP, O.INT8, 48)
    with pytest.raises(ascq_gpu.AscqError):  # no hifloat8 / int4 output
        ascq_gpu.ascend_quant_policy(x, s, O.PER_GROUP, O.INT4, 32)
    with pytest.raises(ascq_gpu.AscqError):  # E2M1 rows pack two a byte
        ascq_gpu.ascend_quant_policy(torch.zeros((4, 63), dtype=torch.float16, device="cuda"), s, O.PER_GROUP,
                                     O.FP4_E2M1, 32)


def test_conversion_sweeps(ascq_gpu):
    """the vector kernels convert with the gfx950 instructions (fp32 -> fp8 / bf16, bf16 / fp32 -> E2M1, E2M1 -> fp32):
    every bf16 pattern and every f16 pattern to E2M1 and E1M2 in all five modes, and 2^22 fp32 patterns spread over
    the whole range to fp8 e4m3 / e5m2 and, through bf16, to E2M1 / E1M2 in all five modes, each against the oracle"""
    bf = np.arange(0x10000, dtype=np.uint32).astype(np.uint16).reshape(256, 256)
    one_b = _bits(np.ones((256, 256 // 32)), O.BF16)
    one_h = _bits(np.ones((256, 256 // 32)), O.F16)
    for mode in _MODES:
        # E2M1: rint is the bf16 -> E2M1 instruction; the directed modes start from the fp32 -> E2M1 nearest-even
        # instruction and step one code where its value lies on the wrong side (round: a 2^-10 nudge).  E1M2 has no
        # conversion instruction: the software encoder.  Every bf16 pattern, and every f16 pattern through the f16
        # product and the bf16 step (scale 1, exact).
        for fp4 in (O.FP4_E2M1, O.FP4_E1M2):
            _check(ascq_gpu, bf, O.BF16, one_b, O.BF16, fp4, O.PER_GROUP, 256, 256, 32, None, None, 1, mode)
            _check(ascq_gpu, bf, O.F16, one_h, O.F16, fp4, O.PER_GROUP, 256, 256, 32, None, None, 1, mode)
    rng = seeded(1700)
    f = (np.arange(1 << 22, dtype=np.uint64) * 1021 + rng.integers(0, 1021, 1 << 22)).astype(np.uint32)
    f = f.view(np.float32).reshape(2048, 2048)
    one_f = np.ones(2048, np.float32)
    for fmt in (O.FP8_E4M3, O.FP8_E5M2):
        _check(ascq_gpu, f, O.F32, one_f, O.F32, fmt, O.PER_TOKEN, 2048, 2048)
    one_g = np.ones((2048, 2048 // 32), np.float32)
    for mode in _MODES:
        _check(ascq_gpu, f, O.F32, one_g, O.F32, O.FP4_E2M1, O.PER_GROUP, 2048, 2048, 32, None, None, 1, mode)
        _check(ascq_gpu, f, O.F32, one_g, O.F32, O.FP4_E1M2, O.PER_GROUP, 2048, 2048, 32, None, None, 1, mode)


def test_empty_inputs(ascq_gpu):
    """rows = 0 (cal_count 0) is a no-op for the quant and antiquant policy forms, as calCount = 0 is in the reference"""
    x = torch.zeros((0, 64), dtype=torch.float16, device="cuda")
    s = torch.ones((0, 2), dtype=torch.float16, device="cuda")
    q = ascq_gpu.ascend_quant_policy(x, s, O.PER_GROUP, O.INT8, 32)
    assert q.shape == (0, 64)
    y = ascq_gpu.ascend_antiquant_policy(torch.zeros((0, 64), dtype=torch.int8, device="cuda"), O.INT8, s, O.F16,
                                         O.PER_GROUP, 0, 64, 32, None, 1)
    torch.cuda.synchronize()
    assert y.shape == (0, 64)
