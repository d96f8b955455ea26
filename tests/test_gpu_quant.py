"""GPU parity: AscendQuant / AscendDequant / AscendAntiQuant through the C ABI vs the oracle (bit-exact)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu


def _f16_input(rng, m, n, outlier_frac=0.001, outlier_mult=50.0):
    x = rng.standard_normal((m, n)).astype(np.float32)
    k = max(1, int(m * n * outlier_frac))
    idx = rng.choice(m * n, size=k, replace=False)
    x.ravel()[idx] *= outlier_mult
    return x.astype(np.float16)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("m,n", [(64, 8192), (33, 4096), (7, 16384), (5, 1000), (3, 8), (2, 24), (1, 65536)])
def test_dynamic_per_token_f16(ascq_gpu, oracle, m, n):
    rng = seeded(100 + m + n)
    x = _f16_input(rng, m, n)
    q, s = ascq_gpu.quant_dynamic_per_token(_dev(x))
    torch.cuda.synchronize()
    q_ref, s_ref = O.quant_dynamic_per_token(x.view(np.uint16), O.F16)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("mode", [O.ROUND_RINT, O.ROUND_FLOOR, O.ROUND_CEIL, O.ROUND_ROUND, O.ROUND_TRUNC])
def test_dynamic_per_token_round_modes(ascq_gpu, oracle, mode):
    rng = seeded(7 + mode)
    x = _f16_input(rng, 16, 2048)
    # plant exact ties: values whose scaled magnitude lands on k + 0.5 (row absmax fixed at 127)
    x[:, 0] = np.float16(127.0)
    x[:, 1:9] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float16)
    q, s = ascq_gpu.quant_dynamic_per_token(_dev(x), round_mode=mode)
    q_ref, s_ref = O.quant_dynamic_per_token(x.view(np.uint16), O.F16, mode)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("dtype,code", [(torch.bfloat16, O.BF16), (torch.float32, O.F32)])
def test_dynamic_per_token_other_src(ascq_gpu, oracle, dtype, code):
    rng = seeded(11)
    x = torch.from_numpy(rng.standard_normal((9, 3000)).astype(np.float32)).to(dtype)
    q, s = ascq_gpu.quant_dynamic_per_token(x.cuda())
    xn = x.view(torch.int16).numpy().view(np.uint16) if dtype == torch.bfloat16 else x.numpy()
    q_ref, s_ref = O.quant_dynamic_per_token(xn, code)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


def test_dynamic_per_token_zero_rows(ascq_gpu, oracle):
    x = np.zeros((4, 512), np.float16)
    x[2, 5] = np.float16(-3.0)
    q, s = ascq_gpu.quant_dynamic_per_token(_dev(x))
    q_ref, s_ref = O.quant_dynamic_per_token(x.view(np.uint16), O.F16)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    assert s_ref[0] == 0 and q_ref[2, 5] == -127


@pytest.mark.parametrize("src", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("has_offset", [False, True])
def test_per_token_given_scale(ascq_gpu, oracle, src, has_offset):
    rng = seeded(21)
    m, n = 13, 777
    x32 = rng.standard_normal((m, n)).astype(np.float32) * 4
    scale = rng.uniform(0.5, 20.0, m).astype(np.float32)
    offset = rng.uniform(-5, 5, m).astype(np.float32) if has_offset else None
    if src == "f16":
        xt = torch.from_numpy(x32.astype(np.float16))
        xn, code = x32.astype(np.float16).view(np.uint16), O.F16
    elif src == "bf16":
        xt = torch.from_numpy(x32).to(torch.bfloat16)
        xn, code = xt.view(torch.int16).numpy().view(np.uint16), O.BF16
    else:
        xt = torch.from_numpy(x32)
        xn, code = x32, O.F32
    q = ascq_gpu.quant_per_token(xt.cuda(), _dev(scale), None if offset is None else _dev(offset))
    q_ref = O.quant_per_token(xn, code, scale, offset)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("case", [(4096, 64, True, True), (4096, 64, True, False), (4096, 0, False, False),
                                  (4128, 12, True, True), (4160, 20, True, False), (32, 8, True, True),
                                  (16392, 0, False, False), (4092, 0, False, False), (1 << 20, 4096, True, True)])
@pytest.mark.parametrize("src", ["f16", "f32"])
def test_legacy_quant_layouts(ascq_gpu, oracle, case, src):
    """legacy AscendQuant to int8: scale / offset tensors, a tensor scale with a scalar offset, or scalars; channel
    counts that are and are not multiples of 8 and ragged per-tensor totals (the vector and the element kernels);
    ties and saturation"""
    n_total, sc, sv, ov = case
    rng = seeded(37 + n_total % 97 + sc + 2 * sv + ov)
    x32 = rng.uniform(-300, 300, n_total).astype(np.float32)
    x32[:6] = [0.5, 1.5, 2.5, -0.5, 126.5, -127.5]
    scale = rng.uniform(0.25, 4, max(sc, 1)).astype(np.float32)
    offset = rng.uniform(-2, 2, max(sc, 1)).astype(np.float32)
    scale[0], offset[0] = 1.0, 0.0
    xs = x32.astype(np.float16) if src == "f16" else x32
    st = scale.astype(np.float16) if src == "f16" else scale
    ot = offset.astype(np.float16) if src == "f16" else offset
    q = ascq_gpu.ascend_quant(torch.from_numpy(xs).cuda(), ascq_gpu.INT8, scale=_dev(st) if sv else None,
                              offset=_dev(ot) if ov else None, scale_scalar=1.0 if sv else 0.75,
                              offset_scalar=0.25, scale_count=sc)
    code = O.F16 if src == "f16" else O.F32
    raw = lambda a: a.view(np.uint16) if src == "f16" else a
    q_ref = O.quant_legacy(raw(xs), code, O.INT8, raw(st) if sv else None, raw(ot) if ov else None,
                           scale_scalar=1.0 if sv else 0.75, offset_scalar=0.25, scale_count=sc)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("src_type", ["int8", "int4"])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("group", [0, 32, 128])
@pytest.mark.parametrize("dst,arith", [("f16", 0), ("f16", 1), ("bf16", 1)])
@pytest.mark.parametrize("with_offset", [True, False])
def test_antiquant(ascq_gpu, oracle, src_type, transpose, group, dst, arith, with_offset):
    rng = seeded(71)
    K, N = 256, 96
    G = K // group if group else 1
    if src_type == "int8":
        w = rng.integers(-128, 128, (N, K) if transpose else (K, N), dtype=np.int8)
        code = O.INT8
    else:
        nib = rng.integers(0, 16, K * N, dtype=np.uint8)
        w = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
        code = O.INT4
    sshape = (N, G) if transpose else (G, N)
    scale32 = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), sshape)).astype(np.float32)
    off32 = rng.uniform(-8, 8, sshape).astype(np.float32)
    if dst == "f16":
        scale_t, off_t = torch.from_numpy(scale32.astype(np.float16)), torch.from_numpy(off32.astype(np.float16))
        dtt, dcode = torch.float16, O.F16
    else:
        scale_t, off_t = torch.from_numpy(scale32).to(torch.bfloat16), torch.from_numpy(off32).to(torch.bfloat16)
        dtt, dcode = torch.bfloat16, O.BF16
    off_dev = off_t.cuda() if with_offset else None
    y = ascq_gpu.ascend_antiquant(_dev(w), ascq_gpu.INT8 if src_type == "int8" else ascq_gpu.INT4, scale_t.cuda(),
                                  off_dev, K, N, group, transpose, dtt, arith)
    y_ref = O.antiquant(w, code, scale_t.view(torch.int16).numpy().view(np.uint16),
                        off_t.view(torch.int16).numpy().view(np.uint16) if with_offset else None,
                        K, N, group, transpose, dcode, arith)
    np.testing.assert_array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), y_ref)


@pytest.mark.parametrize("src_type", ["int8", "int4"])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("group", [0, 20])
@pytest.mark.parametrize("dst,arith", [("f16", 0), ("bf16", 1)])
def test_antiquant_ragged(ascq_gpu, oracle, src_type, transpose, group, dst, arith):
    """K = 100, N = 90 and a group of 20: rows whose length is not a multiple of 8 or groups that split a unit take
    the per-element kernel, the others the vector kernels"""
    _antiquant_case(ascq_gpu, src_type, transpose, group, dst, arith, True, 100, 90, 73)


@pytest.mark.parametrize("src_type", ["int8", "int4"])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("with_offset", [True, False])
def test_antiquant_half_extremes(ascq_gpu, oracle, src_type, transpose, with_offset):
    """Half arithmetic to f16 with scales and offsets at the edges of binary16: +-inf, NaN, 65504, subnormals, and
    products that overflow; every non-NaN output equals the oracle bit for bit, NaN where the oracle has NaN."""
    rng = seeded(75)
    K, N, group = 256, 96, 32
    G = K // group
    if src_type == "int8":
        w = rng.integers(-128, 128, (N, K) if transpose else (K, N), dtype=np.int8)
        code = O.INT8
    else:
        nib = rng.integers(0, 16, K * N, dtype=np.uint8)
        w = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
        code = O.INT4
    sshape = (N, G) if transpose else (G, N)
    special = np.array([np.inf, -np.inf, np.nan, 65504.0, -65504.0, 6e-8, -6e-8, 1e-5, 0.0, -0.0, 300.0, 2.0],
                       np.float16)
    scale = rng.choice(special, sshape).astype(np.float16)
    off = rng.choice(np.concatenate([special, np.float16([-7.5, 0.125, 1000.0])]), sshape).astype(np.float16)
    off_dev = torch.from_numpy(off).cuda() if with_offset else None
    y = ascq_gpu.ascend_antiquant(_dev(w), ascq_gpu.INT8 if src_type == "int8" else ascq_gpu.INT4,
                                  torch.from_numpy(scale).cuda(), off_dev, K, N, group, transpose, torch.float16, 0)
    y_ref = O.antiquant(w, code, scale.view(np.uint16), off.view(np.uint16) if with_offset else None, K, N, group,
                        transpose, O.F16, 0)
    got = y.cpu().view(torch.int16).numpy().view(np.uint16)
    nan_g, nan_r = np.isnan(got.view(np.float16)), np.isnan(y_ref.view(np.float16))
    np.testing.assert_array_equal(nan_g, nan_r)
    np.testing.assert_array_equal(got[~nan_r], y_ref[~nan_r])


def test_antiquant_config3_full_size(ascq_gpu, oracle):
    """the weight of the antiquant matmul workload, int4 [4096, 11008] with f16 scale / offset per 128 rows, to f16
    (half arithmetic) and to bf16, against the oracle"""
    for dst, arith in (("f16", 0), ("bf16", 1)):
        _antiquant_case(ascq_gpu, "int4", False, 128, dst, arith, True, 4096, 11008, 74)


def _antiquant_case(ascq_gpu, src_type, transpose, group, dst, arith, with_offset, K, N, seed):
    rng = seeded(seed)
    G = K // group if group else 1
    if src_type == "int8":
        w = rng.integers(-128, 128, (N, K) if transpose else (K, N), dtype=np.int8)
        code = O.INT8
    else:
        nib = rng.integers(0, 16, K * N, dtype=np.uint8)
        w = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
        code = O.INT4
    sshape = (N, G) if transpose else (G, N)
    scale32 = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), sshape)).astype(np.float32)
    off32 = rng.uniform(-8, 8, sshape).astype(np.float32)
    if dst == "f16":
        scale_t, off_t = torch.from_numpy(scale32.astype(np.float16)), torch.from_numpy(off32.astype(np.float16))
        dtt, dcode = torch.float16, O.F16
    else:
        scale_t, off_t = torch.from_numpy(scale32).to(torch.bfloat16), torch.from_numpy(off32).to(torch.bfloat16)
        dtt, dcode = torch.bfloat16, O.BF16
    off_dev = off_t.cuda() if with_offset else None
    y = ascq_gpu.ascend_antiquant(_dev(w), ascq_gpu.INT8 if src_type == "int8" else ascq_gpu.INT4, scale_t.cuda(),
                                  off_dev, K, N, group, transpose, dtt, arith)
    y_ref = O.antiquant(w, code, scale_t.view(torch.int16).numpy().view(np.uint16),
                        off_t.view(torch.int16).numpy().view(np.uint16) if with_offset else None,
                        K, N, group, transpose, dcode, arith)
    np.testing.assert_array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), y_ref)


def test_config2_full_size_quant_dequant(ascq_gpu, oracle):
    """AscendQuant per-token dynamic quant f16 [8192, 8192] (0.1% outliers x50) -> int8 + fp32 scale, then
    AscendDequant back to f16: both outputs bit-exact vs the oracle at the full workload size."""
    rng = seeded(2)
    m = n = 8192
    x = _f16_input(rng, m, n)
    xd = _dev(x)
    q, s = ascq_gpu.quant_dynamic_per_token(xd)
    y = ascq_gpu.ascend_dequant_policy(q, s, ascq_gpu.PER_TOKEN, torch.float16)
    torch.cuda.synchronize()
    q_ref, s_ref = O.quant_dynamic_per_token(x.view(np.uint16), O.F16)
    qn = q.cpu().numpy()
    np.testing.assert_array_equal(qn, q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    assert np.abs(qn.astype(np.int32)).max() <= 127
    y_ref = O.dequant_policy(q_ref, O.INT8, s_ref, O.F32, O.PER_TOKEN, O.F16)
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint16), y_ref)


def test_launch_events_time_the_main_kernel(ascq_gpu):
    """ascq_set_launch_events: the next entry point's kernel is launched with the two events bound to its
    dispatch; they then hold a positive elapsed time, and the hook is one-shot (a second call leaves it clear)"""
    import ctypes
    from pathlib import Path

    p = Path(torch.__file__).resolve().parent / "lib" / "libamdhip64.so"
    hip = ctypes.CDLL(str(p) if p.exists() else "libamdhip64.so.7")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipEventCreate(ctypes.byref(a)) == 0 and hip.hipEventCreate(ctypes.byref(b)) == 0
    x = torch.randn((2048, 4096), device="cuda").half()
    L = ascq_gpu.lib()
    assert L.ascq_set_launch_events(a, None) == ascq_gpu.E_INVALID_ARG  # both or neither
    assert L.ascq_set_launch_events(a, b) == 0
    q, s = ascq_gpu.quant_dynamic_per_token(x)
    q2, s2 = ascq_gpu.quant_dynamic_per_token(x)  # not timed: the hook cleared itself
    torch.cuda.synchronize()
    ms = ctypes.c_float()
    assert hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
    assert 0.0 < ms.value < 50.0
    assert torch.equal(q, q2) and torch.equal(s, s2)
    hip.hipEventDestroy(a)
    hip.hipEventDestroy(b)
