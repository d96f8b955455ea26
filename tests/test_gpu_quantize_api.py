"""GPU parity: the newer Quantize / Dequantize / AntiQuantize interface (quantize.h, dequantize.h, antiquantize.h:
every policy, fp32 arithmetic) through the C ABI, bit-exact against the oracle, on the vector paths (aligned rows of
a multiple of 8 elements) and the element-wise paths (pointers one element off)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded
from test_oracle import fp8_bytes, hif8_codes

pytestmark = pytest.mark.gpu

_TD = {O.F16: torch.float16, O.BF16: torch.bfloat16, O.F32: torch.float32}
_POLICIES = [O.PER_TENSOR, O.PER_CHANNEL, O.PER_TOKEN, O.PER_GROUP]
_MODES = [O.ROUND_RINT, O.ROUND_FLOOR, O.ROUND_CEIL, O.ROUND_ROUND, O.ROUND_TRUNC, O.ROUND_NONE]


def _bits(v, t):
    if t == O.F16:
        return v.astype(np.float16).view(np.uint16)
    if t == O.BF16:
        return torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return v.astype(np.float32)


def _dev(a, t=None, shift=0):
    """a on the device (f16 / bf16 bit patterns as that dtype); shift > 0: the view starts `shift` elements into a
    larger buffer, so its pointer is not 16-byte aligned"""
    a = np.ascontiguousarray(a)
    x = torch.from_numpy(a).cuda()
    if shift:
        buf = torch.zeros(a.size + shift, dtype=x.dtype, device="cuda")
        buf[shift:] = x.reshape(-1)
        x = buf[shift:].view(a.shape)
    return x.view(_TD[t]) if t in (O.F16, O.BF16) else x


def _scale_shape(policy, m, n, g, k_dim):
    if policy == O.PER_CHANNEL:
        return (n,)
    if policy == O.PER_TOKEN:
        return (m,)
    return (m, (n + g - 1) // g) if k_dim == 1 else ((m + g - 1) // g, n)


def _src(rng, m, n, t, lo, hi):
    v = rng.uniform(lo, hi, (m, n))
    v.flat[:6] = [np.nan, np.inf, -np.inf, 0.5, -2.5, 1e30]
    return _bits(v, t)


@pytest.mark.parametrize("policy", _POLICIES)
@pytest.mark.parametrize("dst", [O.INT8, O.HIF8, O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("st,sct", [(O.F16, O.F16), (O.BF16, O.BF16), (O.F32, O.F32), (O.F16, O.F32)])
@pytest.mark.parametrize("shift", [0, 1])
def test_quantize(ascq_gpu, oracle, policy, dst, st, sct, shift):
    rng = seeded(2000 + 97 * policy + 13 * dst + 5 * st + sct + shift)
    m, n, g, k_dim = 67, 160, 32, policy % 2  # PER_GROUP: kDim 1; PER_CHANNEL / TENSOR ignore it
    hi = 3000.0 if dst == O.HIF8 else (600.0 if dst != O.FP8_E5M2 else 60000.0)
    x = _src(rng, m, n, st, -hi, hi)
    tensor = policy != O.PER_TENSOR
    sc = _bits(rng.uniform(0.01, 1.5, _scale_shape(policy, m, n, g, k_dim)), sct) if tensor else None
    of = _bits(rng.uniform(-9.0, 9.0, _scale_shape(policy, m, n, g, k_dim)), sct) if tensor else None
    for mode in (_MODES if dst == O.INT8 else [O.ROUND_RINT]):
        q = ascq_gpu.quantize(_dev(x, st, shift), policy, dst, None if sc is None else _dev(sc, sct),
                              None if of is None else _dev(of, sct), scale_scalar=0.37, offset_scalar=-1.75,
                              scale_type=sct, group_size=g, kdim=k_dim, round_mode=mode)
        torch.cuda.synchronize()
        got = q.cpu().numpy().view(np.uint8)
        exp = O.quantize(x, st, dst, policy, m, n, scale=sc, scale_type=sct, offset=of, scale_scalar=0.37,
                         offset_scalar=-1.75, group=g, k_dim=k_dim, round_mode=mode).view(np.uint8)
        bad = np.argwhere(got != exp)
        assert bad.size == 0, (policy, dst, st, sct, shift, mode, bad[:4].tolist())


@pytest.mark.parametrize("fp4", [O.FP4_E2M1, O.FP4_E1M2])
@pytest.mark.parametrize("k_dim", [0, 1])
@pytest.mark.parametrize("st,sct", [(O.BF16, O.BF16), (O.F16, O.F16), (O.F32, O.F32)])
def test_quantize_fp4(ascq_gpu, oracle, fp4, k_dim, st, sct):
    """PER_GROUP fp4: fp32 product, bf16 step, the code in each round mode; the offset is not used"""
    rng = seeded(2100 + fp4 + 3 * k_dim + 7 * st + sct)
    m, n, g = 64, 128, 32
    x = _src(rng, m, n, st, -12.0, 12.0)
    sc = _bits(rng.uniform(0.05, 1.5, _scale_shape(O.PER_GROUP, m, n, g, k_dim)), sct)
    for mode in _MODES:
        q = ascq_gpu.quantize(_dev(x, st), O.PER_GROUP, fp4, _dev(sc, sct), scale_type=sct, group_size=g, kdim=k_dim,
                              round_mode=mode, offset_scalar=3.0)
        torch.cuda.synchronize()
        exp = O.quantize(x, st, fp4, O.PER_GROUP, m, n, scale=sc, scale_type=sct, group=g, k_dim=k_dim,
                         round_mode=mode, offset_scalar=3.0)
        assert np.array_equal(q.cpu().numpy(), exp), (fp4, k_dim, st, mode)


def test_quantize_full_size_per_channel_and_tensor(ascq_gpu, oracle):
    """[4096, 4096] f16 -> int8, PER_CHANNEL with an offset tensor and PER_TENSOR: every element against the oracle"""
    rng = seeded(2200)
    m = n = 4096
    x = rng.standard_normal((m, n)).astype(np.float16)
    sc = rng.uniform(10.0, 60.0, n).astype(np.float16)
    of = rng.uniform(-3.0, 3.0, n).astype(np.float16)
    xd = _dev(x.view(np.uint16), O.F16)
    q = ascq_gpu.quantize(xd, O.PER_CHANNEL, O.INT8, _dev(sc), _dev(of), scale_type=O.F16)
    exp = O.quantize(x.view(np.uint16), O.F16, O.INT8, O.PER_CHANNEL, m, n, scale=sc.view(np.uint16),
                     scale_type=O.F16, offset=of.view(np.uint16))
    assert np.array_equal(q.cpu().numpy(), exp)
    q = ascq_gpu.quantize(xd, O.PER_TENSOR, O.INT8, scale_scalar=42.7, offset_scalar=0.5, scale_type=O.F16)
    exp = O.quantize(x.view(np.uint16), O.F16, O.INT8, O.PER_TENSOR, m, n, scale_type=O.F16, scale_scalar=42.7,
                     offset_scalar=0.5)
    assert np.array_equal(q.cpu().numpy(), exp)


@pytest.mark.parametrize("policy,st,dt", [(O.PER_TENSOR, O.BF16, O.BF16), (O.PER_TENSOR, O.F32, O.F32),
                                          (O.PER_CHANNEL, O.U64, O.F16), (O.PER_CHANNEL, O.BF16, O.F32),
                                          (O.PER_CHANNEL, O.F32, O.BF16), (O.PER_TOKEN, O.F16, O.F16),
                                          (O.PER_TOKEN, O.F32, O.BF16), (O.PER_GROUP, O.BF16, O.BF16),
                                          (O.PER_GROUP, O.F32, O.F32)])
@pytest.mark.parametrize("src_type", [O.INT32, O.F32])
def test_dequantize(ascq_gpu, oracle, policy, st, dt, src_type):
    if src_type == O.F32 and policy in (O.PER_TENSOR, O.PER_CHANNEL):
        pytest.skip("PER_TENSOR / PER_CHANNEL take int32 sources only")
    rng = seeded(2300 + 11 * policy + st + 3 * dt + src_type)
    m, n, g = 72, 96, 32
    if src_type == O.INT32:
        src = rng.integers(-(1 << 28), 1 << 28, (m, n)).astype(np.int32)
        src.flat[:4] = [(1 << 24) + 1, -((1 << 24) + 3), 2 ** 31 - 1, -(2 ** 31)]  # ties above 2^24, the extremes
    else:
        src = rng.standard_normal((m, n)).astype(np.float32) * 1000
    sshape = _scale_shape(policy, m, n, g, 1)
    if st == O.U64:
        sc = rng.uniform(-1e-3, 1e-3, sshape).astype(np.float32).view(np.uint32).astype(np.uint64)
        sc |= np.uint64(0xABCD) << np.uint64(40)  # the high half is not used
        scd = torch.from_numpy(sc.view(np.int64)).cuda()
    else:
        sc = _bits(rng.uniform(-1e-3, 1e-3, sshape), st)
        scd = _dev(sc, st)
    tensor = policy != O.PER_TENSOR
    y = ascq_gpu.dequantize(torch.from_numpy(src).cuda(), policy, _TD[dt], scd if tensor else None,
                            scale_scalar=3.1e-4, scale_type=st, group_size=g, kdim=1)
    torch.cuda.synchronize()
    exp = O.dequantize(src, src_type, dt, policy, scale=sc if tensor else None, scale_type=st, scale_scalar=3.1e-4,
                       group=g, k_dim=1)
    got = y.cpu()
    got = got.numpy() if dt == O.F32 else got.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got.view(exp.dtype), exp)


@pytest.mark.parametrize("policy", _POLICIES)
@pytest.mark.parametrize("src_type", [O.INT8, O.HIF8, O.FP8_E4M3, O.FP8_E5M2])
@pytest.mark.parametrize("st,dt", [(O.F16, O.F16), (O.BF16, O.BF16), (O.F32, O.F32), (O.F32, O.F16)])
@pytest.mark.parametrize("shift", [0, 1])
def test_antiquantize(ascq_gpu, oracle, policy, src_type, st, dt, shift):
    if policy in (O.PER_TENSOR, O.PER_CHANNEL) and st == O.F32:
        pytest.skip("PER_TENSOR / PER_CHANNEL take f16 / bf16 scales of the dst type")
    rng = seeded(2400 + 31 * policy + 7 * src_type + 3 * st + dt + shift)
    m, n, g, k_dim = 70, 128, 32, policy % 2
    if src_type == O.INT8:
        q = rng.integers(-128, 128, (m, n)).astype(np.int8)
    elif src_type == O.HIF8:
        q = hif8_codes(rng, (m, n))
    else:
        q = fp8_bytes(rng, (m, n), src_type)
    tensor = policy != O.PER_TENSOR
    sshape = _scale_shape(policy, m, n, g, k_dim)
    sc = _bits(rng.uniform(-2.0, 2.0, sshape), st) if tensor else None
    of = _bits(rng.uniform(-40.0, 40.0, sshape), st) if tensor else None
    y = ascq_gpu.antiquantize(_dev(q, shift=shift), src_type, policy, m, n, _TD[dt],
                              None if sc is None else _dev(sc, st), None if of is None else _dev(of, st),
                              scale_scalar=0.8125, offset_scalar=-3.5, scale_type=st, group_size=g, kdim=k_dim)
    torch.cuda.synchronize()
    exp = O.antiquantize(q, src_type, dt, policy, m, n, scale=sc, scale_type=st, offset=of, scale_scalar=0.8125,
                         offset_scalar=-3.5, group=g, k_dim=k_dim)
    got = y.cpu()
    got = got.numpy() if dt == O.F32 else got.view(torch.int16).numpy().view(np.uint16)
    bad = np.argwhere(got.view(exp.dtype) != exp)
    nan = np.isnan(got.view(np.float32)) if dt == O.F32 else None
    if nan is not None:  # NaN payloads: compare NaN-ness there
        bad = np.argwhere((got.view(np.uint32) != exp.view(np.uint32)) & ~(nan & np.isnan(exp)))
    assert bad.size == 0, (policy, src_type, st, dt, shift, bad[:4].tolist())


@pytest.mark.parametrize("fp4", [O.FP4_E2M1, O.FP4_E1M2])
@pytest.mark.parametrize("k_dim", [0, 1])
@pytest.mark.parametrize("dt", [O.F16, O.BF16])
def test_antiquantize_fp4(ascq_gpu, oracle, fp4, k_dim, dt):
    rng = seeded(2500 + fp4 + 3 * k_dim + dt)
    m, n, g = 64, 128, 32
    packed = rng.integers(0, 256, (m, n // 2)).astype(np.uint8)
    e = rng.integers(100, 150, _scale_shape(O.PER_GROUP, m, n, g, k_dim)).astype(np.uint8)
    y = ascq_gpu.antiquantize(_dev(packed), fp4, O.PER_GROUP, m, n, _TD[dt], _dev(e), scale_type=O.E8M0,
                              group_size=g, kdim=k_dim)
    torch.cuda.synchronize()
    exp = O.antiquantize(packed, fp4, dt, O.PER_GROUP, m, n, scale=e, scale_type=O.E8M0, group=g, k_dim=k_dim)
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), exp)


def test_reference_examples_on_gpu(ascq_gpu, oracle):
    """the reference's three arch-3510 examples (quant.asc, dequant.asc, antiquant.asc) against their goldens"""
    from test_oracle import GOLD
    f = np.load(GOLD / "quant_example_3510.npz")
    q = ascq_gpu.quantize(torch.from_numpy(f["src"].reshape(1, -1)).cuda(), O.PER_TENSOR, O.INT8, scale_scalar=2.0,
                          offset_scalar=0.9)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy()[0], f["golden"])
    f = np.load(GOLD / "dequant_example.npz")
    y = ascq_gpu.dequantize(torch.from_numpy(f["inp"]).cuda(), O.PER_CHANNEL, torch.float32,
                            torch.from_numpy(f["scale"]).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), f["golden"].view(np.uint32))
    f = np.load(GOLD / "antiquant_seed10.npz")
    y = ascq_gpu.antiquantize(torch.from_numpy(f["src"]).cuda(), O.INT8, O.PER_CHANNEL, 8, 128, torch.float16,
                              torch.from_numpy(f["scale"].reshape(-1)).cuda(),
                              torch.from_numpy(f["offset"].reshape(-1)).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), f["golden_3510"].view(np.uint16))
