"""GPU parity, bit-exact against the oracle: hifloat8 across the path and the arch-3510 legacy forms.

- AscendQuant policy form to hifloat8 (PER_TOKEN / PER_GROUP, every scale-type pair), including every f16 pattern
  and 2^22 fp32 patterns through the device's hifloat8 coder;
- AscendAntiQuant policy form from hifloat8 (every code in every position);
- legacy AscendQuant, arch-3510 form: f16 / bf16 / f32 sources, int8 / hifloat8 / fp8 outputs, scale and offset
  tensors of the source type, a tensor scale with a scalar offset, or float scalars;
- legacy AscendAntiQuant from fp8 / hifloat8 (per channel, both layouts, rows narrower than 32 included) and the
  per-tensor scalar form from int8 / int4 / fp8 / hifloat8."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu

_TD = {O.F16: torch.float16, O.BF16: torch.bfloat16, O.F32: torch.float32}


def _raw(v, t):
    """float values -> host array of type t (f16 / bf16 as uint16 bits)"""
    v = np.asarray(v)
    if t == O.F16:
        return v.astype(np.float16).view(np.uint16)
    if t == O.BF16:
        return torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return v.astype(np.float32)


def _dev(a, t=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return x.view(_TD[t]) if t in (O.F16, O.BF16) else x


def _hif8_codes(rng, shape):
    c = rng.integers(0, 256, shape, dtype=np.uint8)
    c.reshape(-1)[:3] = [0x80, 0x6F, 0xEF]  # NaN, +-inf
    return c


def _bits_of(t):
    c = t.cpu()
    return c.view(torch.int16).numpy().view(np.uint16) if c.dtype != torch.float32 else c.numpy().view(np.uint32)


def _same(got, exp):
    """bit-exact, any NaN matching any NaN"""
    g, e = np.asarray(got), np.asarray(exp)
    if g.dtype == np.uint16:
        nan = lambda b: ((b & 0x7C00) == 0x7C00) & ((b & 0x3FF) != 0)
    else:
        nan = lambda b: ((b & 0x7F800000) == 0x7F800000) & ((b & 0x7FFFFF) != 0)
    return bool(((g == e) | (nan(g) & nan(e))).all())


# ------------------------------------------------------------------------------------------- policy form
_PAIRS = [(O.F16, O.F16), (O.BF16, O.BF16), (O.F32, O.F32), (O.F16, O.F32), (O.BF16, O.F32)]


@pytest.mark.parametrize("st,sct", _PAIRS)
@pytest.mark.parametrize("layout", [(O.PER_TOKEN, 0, 1), (O.PER_GROUP, 32, 1), (O.PER_GROUP, 64, 0)])
@pytest.mark.parametrize("off", ["tensor", "scalar", None])
def test_quant_policy_to_hif8(ascq_gpu, oracle, st, sct, layout, off):
    policy, g, k_dim = layout
    m, n = 70, 192
    rng = seeded(11 + st + 3 * sct + g + k_dim + (off == "tensor") + 2 * (off == "scalar"))
    x = rng.standard_normal((m, n)) * np.exp2(rng.uniform(-20, 14, (m, n)))
    x.flat[:5] = [np.nan, np.inf, -np.inf, 1e30, 2.0 ** -24]
    shape = (m,) if policy == O.PER_TOKEN else ((m, -(-n // g)) if k_dim == 1 else (-(-m // g), n))
    sc = np.exp2(rng.uniform(-6, 6, shape)) * np.where(rng.random(shape) < 0.5, -1, 1)
    of = rng.uniform(-8, 8, shape) if off == "tensor" else None
    xr, scr = _raw(x, st), _raw(sc, sct)
    ofr = None if of is None else _raw(of, sct)
    osc = 1.375 if off == "scalar" else None
    q = ascq_gpu.ascend_quant_policy(_dev(xr, st), _dev(scr, sct), policy, ascq_gpu.HIF8, g,
                                     None if ofr is None else _dev(ofr, sct), osc, k_dim, scale_type=sct)
    exp = O.quant_policy(xr, st, scr, sct, O.HIF8, policy, m, n, g, ofr, osc, k_dim).view(np.uint8)
    np.testing.assert_array_equal(q.cpu().numpy().view(np.uint8), exp)


def test_hif8_coder_every_f16_and_fp32_patterns(ascq_gpu, oracle):
    """PER_TOKEN with scale 1 passes each source value unchanged to the hifloat8 coder: all 65536 f16 patterns
    (half arithmetic) and 2^22 fp32 patterns (every 1024th, fp32 arithmetic), against the oracle's coder"""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(64, 1024)
    q = ascq_gpu.ascend_quant_policy(_dev(h, O.F16), _dev(_raw(np.ones(64), O.F16), O.F16), O.PER_TOKEN,
                                     ascq_gpu.HIF8, scale_type=O.F16)
    exp = O.quant_policy(h, O.F16, _raw(np.ones(64), O.F16), O.F16, O.HIF8, O.PER_TOKEN, 64, 1024).view(np.uint8)
    np.testing.assert_array_equal(q.cpu().numpy().view(np.uint8), exp)
    f = (np.arange(1 << 22, dtype=np.uint64) * 1024 + 517).astype(np.uint32).view(np.float32).reshape(4096, 1024)
    q = ascq_gpu.ascend_quant_policy(_dev(f), _dev(np.ones(4096, np.float32)), O.PER_TOKEN, ascq_gpu.HIF8)
    exp = O.quant_policy(f, O.F32, np.ones(4096, np.float32), O.F32, O.HIF8, O.PER_TOKEN, 4096, 1024).view(np.uint8)
    np.testing.assert_array_equal(q.cpu().numpy().view(np.uint8), exp)


@pytest.mark.parametrize("scale_type", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("layout", [(O.PER_TOKEN, 0, 0, False), (O.PER_TOKEN, 0, 0, True), (O.PER_GROUP, 32, 0, False),
                                    (O.PER_GROUP, 64, 1, False), (O.PER_GROUP, 32, 1, True)])
def test_antiquant_policy_from_hif8(ascq_gpu, oracle, scale_type, layout):
    policy, g, k_dim, tr = layout
    m, n = 75, 256
    rng = seeded(41 + scale_type + g + k_dim + 3 * tr)
    codes = np.tile(np.arange(256, dtype=np.uint8), m)[: m * n].reshape(m, n)  # every code, shifted per row
    codes = np.roll(codes, rng.integers(0, n), axis=1)
    if policy == O.PER_TOKEN:
        shape = (n,) if tr else (m,)
    else:
        cols = (k_dim == 1 and not tr) or (k_dim == 0 and tr)
        shape = (m, -(-n // g)) if cols else (-(-m // g), n)
    sc = _raw(rng.uniform(-2, 2, shape), scale_type)
    of = _raw(rng.uniform(-4, 4, shape), scale_type)
    for dt in ([scale_type] if scale_type != O.F32 else [O.F32, O.F16, O.BF16]):
        y = ascq_gpu.ascend_antiquant_policy(_dev(codes), ascq_gpu.HIF8, _dev(sc, scale_type), scale_type, policy,
                                             m, n, g, _dev(of, scale_type), k_dim, tr, _TD[dt])
        exp = O.antiquant_policy(codes, O.HIF8, sc, scale_type, dt, policy, m, n, g, of, k_dim, tr)
        assert _same(_bits_of(y), exp.view(np.uint32) if dt == O.F32 else exp), dt


# ------------------------------------------------------------------------------------------- legacy forms
@pytest.mark.parametrize("src", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("dst", [O.INT8, O.HIF8, O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("kind", ["tensor", "scalar_offset", "per_tensor"])
@pytest.mark.parametrize("shape", [(8192, 64), (4128, 12), (4093, 0)])
def test_legacy_quant_3510(ascq_gpu, oracle, src, dst, kind, shape):
    n, sc_n = shape
    if kind != "per_tensor" and sc_n == 0:
        sc_n = 32
    if kind == "per_tensor":
        sc_n = 0
    if sc_n and n % 32:
        n = n // 32 * 32
    rng = seeded(7 * src + dst + len(kind) + n % 13)
    x = rng.standard_normal(n) * np.exp2(rng.uniform(-8, 12, n))
    x[:6] = [1e6, -7e4, 70000.0, np.nan, 0.5, -2.5]
    s = rng.uniform(-2, 2, max(sc_n, 1)) * (0.01 if dst == O.INT8 else 1.0)
    o = rng.uniform(-30, 30, max(sc_n, 1))
    xr, sr, orr = _raw(x, src), _raw(s, src), _raw(o, src)
    ss, osc = 0.0137 if dst == O.INT8 else 1.7, 2.71875
    if kind == "tensor":
        a = dict(scale=_dev(sr, src), offset=_dev(orr, src), scale_count=sc_n)
        exp = O.quant_legacy(xr, src, dst, sr, orr, scale_count=sc_n)
    elif kind == "scalar_offset":
        a = dict(scale=_dev(sr, src), offset=None, offset_scalar=osc, scale_count=sc_n)
        exp = O.quant_legacy(xr, src, dst, sr, None, offset_scalar=osc, scale_count=sc_n)
    else:
        a = dict(scale_scalar=ss, offset_scalar=osc)
        exp = O.quant_legacy(xr, src, dst, scale_scalar=ss, offset_scalar=osc)
    q = ascq_gpu.ascend_quant(_dev(xr, src), dst, **a)
    np.testing.assert_array_equal(q.cpu().numpy().view(np.uint8), exp.view(np.uint8))


@pytest.mark.parametrize("src", [O.HIF8, O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("dst", [O.F16, O.BF16])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("kn", [(64, 96), (48, 16), (33, 40)])
@pytest.mark.parametrize("with_offset", [True, False])
def test_legacy_antiquant_fp8_hif8(ascq_gpu, oracle, src, dst, transpose, kn, with_offset):
    """per channel: [K, N] with [1, N] tables (bf16 from hifloat8: bf16 ops) or transposed [N, K] with [N, 1]
    (bf16 from hifloat8: fp32 ops); fp8 always fp32 ops; narrow and odd widths take the element kernel"""
    K, N = kn
    rng = seeded(src + 5 * dst + 3 * transpose + K + with_offset)
    codes = _hif8_codes(rng, (N, K) if transpose else (K, N))
    sc = _raw(rng.uniform(-1, 1, N), dst)
    of = _raw(rng.uniform(-4, 4, N), dst)
    y = ascq_gpu.ascend_antiquant(_dev(codes), src, _dev(sc, dst), _dev(of, dst) if with_offset else None, K, N, 0,
                                  transpose, _TD[dst], ascq_gpu.ARITH_F32)
    exp = O.antiquant(codes, src, sc, of if with_offset else None, K, N, 0, transpose, dst, O.ARITH_F32)
    assert _same(_bits_of(y), exp)


@pytest.mark.parametrize("src", [O.INT8, O.INT4, O.HIF8, O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("dst", [O.F16, O.BF16])
@pytest.mark.parametrize("count", [8192, 1000, 24])
@pytest.mark.parametrize("with_offset", [True, False])
def test_antiquant_scalar(ascq_gpu, oracle, src, dst, count, with_offset):
    rng = seeded(src + 7 * dst + count + with_offset)
    if src == O.INT4:
        codes = rng.integers(0, 256, count // 2, dtype=np.uint8)
    else:
        codes = _hif8_codes(rng, count)
    off, sc = -3.25, 0.1875
    y = ascq_gpu.ascend_antiquant_scalar(_dev(codes), src, off if with_offset else None, sc, count, _TD[dst])
    ob = int(_raw(np.array([off]), dst)[0])
    sb = int(_raw(np.array([sc]), dst)[0])
    exp = O.antiquant_scalar(codes, src, ob, sb, dst, with_offset)
    assert _same(_bits_of(y), exp)


@pytest.mark.parametrize("src", [O.INT8, O.HIF8])
@pytest.mark.parametrize("scale_type", [O.F16, O.BF16])
def test_antiquant_signed_zero(ascq_gpu, oracle, src, scale_type):
    """(q + offset) = +0 exactly, times a negative scale, is -0 in the reference's scale-type arithmetic"""
    m, n = 16, 64
    rng = seeded(99 + src + scale_type)
    if src == O.INT8:
        q = rng.integers(-8, 8, (m, n)).astype(np.int8)
        vals = q.astype(np.float64)
    else:
        q = np.full((m, n), 0x14, np.uint8)  # 3.0
        vals = np.full((m, n), 3.0)
    of = _raw(-vals[:, 0], scale_type)        # per-token offsets cancel column 0 exactly
    sc = _raw(-np.exp2(rng.uniform(-2, 2, m)), scale_type)
    y = ascq_gpu.ascend_antiquant_policy(_dev(q), src, _dev(sc, scale_type), scale_type, O.PER_TOKEN, m, n, 0,
                                         _dev(of, scale_type), 0, False, _TD[scale_type])
    exp = O.antiquant_policy(q, src, sc, scale_type, scale_type, O.PER_TOKEN, m, n, 0, of, 0, False)
    got = _bits_of(y)
    assert (exp[:, 0] == 0x8000).all()
    np.testing.assert_array_equal(got, exp)
