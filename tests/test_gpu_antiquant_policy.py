"""GPU parity: AscendAntiQuant policy form (arch 3510; PER_TOKEN / PER_GROUP, int8 / fp8 / fp4 sources) through
the C ABI, bit-exact against the oracle (NaN patterns compared as NaN)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu

_TD = {O.F16: torch.float16, O.BF16: torch.bfloat16, O.F32: torch.float32}


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _scale_bits(v, t):
    if t == O.F16:
        return v.astype(np.float16).view(np.uint16)
    if t == O.BF16:
        return torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return v.astype(np.float32)


def _run(ascq, src, src_type, scale, scale_type, dst_type, policy, m, n, g=0, offset=None, k_dim=0, tr=False):
    y = ascq.ascend_antiquant_policy(_dev(src), src_type, _dev(scale), scale_type, policy, m, n, g,
                                     None if offset is None else _dev(offset), k_dim, tr, _TD[dst_type])
    torch.cuda.synchronize()
    out = y.cpu()
    return out.numpy() if dst_type == O.F32 else out.view(torch.int16).numpy().view(np.uint16)


def _same(got, exp, dst_type):
    if dst_type == O.F32:
        return np.array_equal(got, exp, equal_nan=True)
    if dst_type == O.F16:
        g, e = got.view(np.float16), exp.view(np.float16)
    else:
        g = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float().numpy()
        e = torch.from_numpy(exp.view(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(g) & np.isnan(e)
    return bool(np.array_equal(got[~nan], exp[~nan]) and (np.isnan(g) == np.isnan(e)).all())


def _scales(rng, shape, t):
    return _scale_bits(rng.uniform(0.002, 4.0, shape), t), _scale_bits(rng.uniform(-30.0, 30.0, shape), t)


def _sshape(policy, m, n, g, k_dim, tr):
    if policy == O.PER_TOKEN:
        return (n,) if tr else (m,)
    col = (k_dim == 1 and not tr) or (k_dim == 0 and tr)
    return (m, (n + g - 1) // g) if col else ((m + g - 1) // g, n)


@pytest.mark.parametrize("scale_type", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("layout", [(O.PER_TOKEN, 0, 0, False), (O.PER_TOKEN, 0, 0, True), (O.PER_GROUP, 32, 0, False),
                                    (O.PER_GROUP, 64, 1, False), (O.PER_GROUP, 32, 1, True)])
@pytest.mark.parametrize("with_offset", [True, False])
def test_int8_source(ascq_gpu, scale_type, layout, with_offset):
    policy, g, k_dim, tr = layout
    m, n = 75, 160
    rng = seeded(31 + scale_type + 7 * g + k_dim + 3 * tr + with_offset)
    q = rng.integers(-128, 128, (m, n)).astype(np.int8)
    sc, of = _scales(rng, _sshape(policy, m, n, g, k_dim, tr), scale_type)
    of = of if with_offset else None
    dsts = [scale_type] if scale_type != O.F32 else [O.F32, O.F16, O.BF16]
    for dt in dsts:
        got = _run(ascq_gpu, q, O.INT8, sc, scale_type, dt, policy, m, n, g, of, k_dim, tr)
        exp = O.antiquant_policy(q, O.INT8, sc, scale_type, dt, policy, m, n, g, of, k_dim, tr)
        assert _same(got, exp, dt), (dt, int((got != exp).sum()))


@pytest.mark.parametrize("src_type", [O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("scale_type", [O.F16, O.F32])
@pytest.mark.parametrize("dst_type", [O.F16, O.BF16, O.F32])
def test_fp8_source(ascq_gpu, src_type, scale_type, dst_type):
    m, n, g = 64, 96, 32
    rng = seeded(51 + src_type + scale_type + dst_type)
    codes = rng.integers(0, 256, (m, n)).astype(np.uint8)  # NaN / inf codes included
    for policy, k_dim in ((O.PER_GROUP, 1), (O.PER_GROUP, 0), (O.PER_TOKEN, 0)):
        sc, of = _scales(rng, _sshape(policy, m, n, g, k_dim, False), scale_type)
        got = _run(ascq_gpu, codes, src_type, sc, scale_type, dst_type, policy, m, n, g, of, k_dim)
        exp = O.antiquant_policy(codes, src_type, sc, scale_type, dst_type, policy, m, n, g, of, k_dim)
        assert _same(got, exp, dst_type), (policy, k_dim)


@pytest.mark.parametrize("dst_type", [O.BF16, O.F16])
@pytest.mark.parametrize("k_dim", [0, 1])
@pytest.mark.parametrize("fp4", [O.FP4_E2M1, O.FP4_E1M2])
def test_fp4_source_e8m0(ascq_gpu, dst_type, k_dim, fp4):
    m, n, g = 96, 128, 32
    rng = seeded(71 + dst_type + k_dim + 3 * fp4)
    packed = rng.integers(0, 256, (m, n // 2)).astype(np.uint8)
    e = rng.integers(100, 155, _sshape(O.PER_GROUP, m, n, g, k_dim, False)).astype(np.uint8)
    e.flat[:4] = [0, 255, 254, 1]  # 2^-127, NaN, overflowing products, tiny products
    got = _run(ascq_gpu, packed, fp4, e, O.E8M0, dst_type, O.PER_GROUP, m, n, g, None, k_dim)
    exp = O.antiquant_policy(packed, fp4, e, O.E8M0, dst_type, O.PER_GROUP, m, n, g, None, k_dim)
    assert _same(got, exp, dst_type)


def test_argument_checks(ascq_gpu):
    q = torch.zeros((4, 64), dtype=torch.int8, device="cuda")
    s = torch.ones(4, dtype=torch.float16, device="cuda")
    with pytest.raises(ascq_gpu.AscqError):  # int8 with a half scale writes half, not bf16
        ascq_gpu.ascend_antiquant_policy(q, O.INT8, s, O.F16, O.PER_TOKEN, 4, 64, dst_dtype=torch.bfloat16)
    with pytest.raises(ascq_gpu.AscqError):  # group size must be a multiple of 32
        ascq_gpu.ascend_antiquant_policy(q, O.INT8, s, O.F16, O.PER_GROUP, 4, 64, 16)
    with pytest.raises(ascq_gpu.AscqError):  # fp4 takes no offset
        ascq_gpu.ascend_antiquant_policy(q, O.FP4_E2M1, q, O.E8M0, O.PER_GROUP, 4, 64, 32, offset=s,
                                         dst_dtype=torch.bfloat16)


@pytest.mark.parametrize("src_type", [O.INT8, O.FP8_E5M2, O.FP4_E2M1, O.FP4_E1M2])
def test_ragged_rows_and_unaligned(ascq_gpu, src_type):
    """n % 8 != 0, or a destination off a 16-byte boundary, takes the per-element kernel"""
    m, n, g = 21, 98, 32
    rng = seeded(91 + src_type)
    if src_type in (O.FP4_E2M1, O.FP4_E1M2):
        src = rng.integers(0, 256, (m, n // 2)).astype(np.uint8)
        sc, sct, of, dt, k_dim = rng.integers(110, 140, (m, (n + g - 1) // g)).astype(np.uint8), O.E8M0, None, O.BF16, 1
    else:
        src = rng.integers(-128 if src_type == O.INT8 else 0, 128 if src_type == O.INT8 else 256, (m, n))
        src = src.astype(np.int8 if src_type == O.INT8 else np.uint8)
        sct, dt, k_dim = O.F16, O.F16, 0
        sc, of = _scales(rng, ((m + g - 1) // g, n), sct)
    got = _run(ascq_gpu, src, src_type, sc, sct, dt, O.PER_GROUP, m, n, g, of, k_dim)
    exp = O.antiquant_policy(src, src_type, sc, sct, dt, O.PER_GROUP, m, n, g, of, k_dim)
    assert _same(got, exp, dt)
    if src_type == O.INT8:  # n % 8 == 0 but the output one element off alignment
        n2 = 96
        src2 = np.ascontiguousarray(src[:, :n2])
        sc2, of2 = _scales(rng, ((m + g - 1) // g, n2), sct)
        yd = torch.empty(m * n2 + 1, dtype=torch.float16, device="cuda")
        y = yd[1:].view(m, n2)
        ascq_gpu.ascend_antiquant_policy(_dev(src2), src_type, _dev(sc2), sct, O.PER_GROUP, m, n2, g, _dev(of2), k_dim,
                                         False, torch.float16, out=y)
        torch.cuda.synchronize()
        exp2 = O.antiquant_policy(src2, src_type, sc2, sct, dt, O.PER_GROUP, m, n2, g, of2, k_dim)
        assert _same(y.cpu().view(torch.int16).numpy().view(np.uint16), exp2, dt)


@pytest.mark.parametrize("dst_type", [O.BF16, O.F16])
@pytest.mark.parametrize("fp4", [O.FP4_E2M1, O.FP4_E1M2])
def test_fp4_every_byte_every_position(ascq_gpu, dst_type, fp4):
    """every byte value (two E2M1 or E1M2 codes) in each of the four byte positions of a 32-bit source word, under scales
    2^0, 2^-127 (e = 0), 2^127 and NaN (e = 255)"""
    m, n, g = 4, 2048, 32
    b = np.arange(256, dtype=np.uint8)
    packed = np.stack([np.roll(np.repeat(b, 4), p) for p in range(m)]).astype(np.uint8)  # [4, 1024] bytes
    e = np.tile(np.array([127, 0, 254, 255], np.uint8), (m, n // g // 4))
    got = _run(ascq_gpu, packed, fp4, e, O.E8M0, dst_type, O.PER_GROUP, m, n, g, None, 1)
    exp = O.antiquant_policy(packed, fp4, e, O.E8M0, dst_type, O.PER_GROUP, m, n, g, None, 1)
    assert _same(got, exp, dst_type)


@pytest.mark.parametrize("case", ["int8_g32_off", "int8_token_tr", "fp8_g64_f32", "fp4_g32", "int8_g96_f32"])
def test_large_row_blocks_with_tails(ascq_gpu, case):
    """Groups down the columns on [~2060, 16384] tensors (over 2^20 lanes of the row-blocked kernel): row counts
    that leave a partial last block of rows, a group size that is a multiple of the block, and PER_TOKEN by column
    as one group over every row."""
    n = 16384
    rng = seeded(131 + len(case))
    if case == "int8_g32_off":
        m, src_type, sct, dt, policy, g, tr = 2057, O.INT8, O.F16, O.F16, O.PER_GROUP, 32, False
    elif case == "int8_token_tr":
        m, src_type, sct, dt, policy, g, tr = 2050, O.INT8, O.BF16, O.BF16, O.PER_TOKEN, 0, True
    elif case == "fp8_g64_f32":
        m, src_type, sct, dt, policy, g, tr = 2113, O.FP8_E4M3, O.F32, O.F16, O.PER_GROUP, 64, False
    elif case == "fp4_g32":
        m, src_type, sct, dt, policy, g, tr = 2074, O.FP4_E2M1, O.E8M0, O.BF16, O.PER_GROUP, 32, False
    else:
        m, src_type, sct, dt, policy, g, tr = 2063, O.INT8, O.F32, O.BF16, O.PER_GROUP, 96, False
    shape = _sshape(policy, m, n, g, 0, tr)
    if src_type == O.FP4_E2M1:
        src = rng.integers(0, 256, (m, n // 2)).astype(np.uint8)
        sc, of = rng.integers(100, 155, shape).astype(np.uint8), None
    else:
        src = rng.integers(-128 if src_type == O.INT8 else 0, 128 if src_type == O.INT8 else 256, (m, n))
        src = src.astype(np.int8 if src_type == O.INT8 else np.uint8)
        sc, of = _scales(rng, shape, sct)
    got = _run(ascq_gpu, src, src_type, sc, sct, dt, policy, m, n, g, of, 0, tr)
    exp = O.antiquant_policy(src, src_type, sc, sct, dt, policy, m, n, g, of, 0, tr)
    assert _same(got, exp, dt), int((got != exp).sum())
