"""GPU parity: AscendDequant, both forms, through the C ABI vs the oracle (bit-exact, whole dst buffers).

Legacy form (DequantParams{m, n, calCount}, DeQuantMode): the SINGLE_ROW reshape of {1, m*n, n}, dst rows padded
to 32 bytes, columns >= calCount and the padding left unwritten, int32 -> fp32 with ties away from zero, and the
reference's (deqScale, dst) type combinations.  Policy form: PER_TOKEN and PER_GROUP (kDim 0 / 1) on int32 / fp32
sources with f16 / bf16 / f32 scales, ragged row and column tails included."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu

_TORCH = {O.F16: torch.float16, O.BF16: torch.bfloat16, O.F32: torch.float32}
_NP = {O.F16: np.uint16, O.BF16: np.uint16, O.F32: np.float32}
# (deqScale type, dst type) pairs the legacy form accepts (IsTemplateValid)
TENSOR_COMBOS = [(O.U64, O.F16), (O.F32, O.F32), (O.BF16, O.F32), (O.BF16, O.BF16), (O.F32, O.BF16)]
SCALAR_COMBOS = [(O.BF16, O.BF16), (O.BF16, O.F32), (O.F32, O.F32), (O.F32, O.BF16)]


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(t):
    """device tensor -> numpy array of raw bits (uint16 for 16-bit types, uint32 for f32)"""
    c = t.cpu()
    if c.dtype == torch.float32:
        return c.numpy().view(np.uint32)
    return c.view(torch.int16).numpy().view(np.uint16)


def _scale_tensor(rng, n, st):
    """(device tensor, oracle array) of n per-channel scales of type st"""
    s32 = (rng.uniform(0.5, 2.0, n) * np.where(rng.random(n) < 0.5, -1, 1) * 2.0 ** rng.integers(-14, 2, n))
    s32 = s32.astype(np.float32)
    if st == O.F32:
        return _dev(s32), s32
    if st == O.F16:
        h = s32.astype(np.float16)
        return _dev(h), h
    if st == O.BF16:
        b = torch.from_numpy(s32).to(torch.bfloat16)
        return b.cuda(), b.view(torch.int16).numpy().view(np.uint16)
    words = s32.view(np.uint32).astype(np.uint64) | (np.uint64(0x5A5) << np.uint64(37))  # high word ignored
    return _dev(words.view(np.int64)), words


def _int32_src(rng, shape, big=False):
    lim = 2 ** 31 - 1 if big else 1 << 22
    v = rng.integers(-lim, lim, shape, dtype=np.int64).astype(np.int32)
    if big:  # exact ties of the int32 -> fp32 conversion
        flat = v.reshape(-1)
        k = flat.size // 8
        t = ((rng.integers(1 << 24, 2 ** 30, k, dtype=np.int64) >> 3) << 3) | 4
        flat[:k] = (t * np.where(rng.random(k) < 0.5, -1, 1)).astype(np.int32)
    return v


def _legacy_case(ascq_gpu, rng, m, n, cal, st, dt, per_tensor, mode, big=False):
    src = _int32_src(rng, (m * n,), big)
    rows, ldd = ascq_gpu.dequant_dst_shape(_TORCH[dt], m, n, cal, mode)
    assert (rows, ldd) == O.dequant_legacy_shape(dt, m, n, cal, mode)[::2]
    init = np.full((rows, ldd), 0x3C3C if dt != O.F32 else np.float32(-7.5), _NP[dt])
    out = _dev(init)
    if dt != O.F32:
        out = out.view(torch.int16).view(_TORCH[dt])
    ss = np.float32(0.0371)
    if per_tensor:
        ascq_gpu.ascend_dequant(_dev(src), None, _TORCH[dt], cal_count=cal, scale_scalar=float(ss), scale_type=st,
                                mode=mode, m=m, n=n, out=out)
        ssr = float(torch.tensor(float(ss)).to(torch.bfloat16).float()) if st == O.BF16 else ss
        ref = O.dequant_legacy(src, O.INT32, None, 0, per_tensor=True, dst_type=dt, cal_count=cal,
                               scale_scalar=ssr, mode=mode, m=m, n=n, dst=init.copy())
    else:
        sdev, sref = _scale_tensor(rng, n, st)
        ascq_gpu.ascend_dequant(_dev(src), sdev, _TORCH[dt], cal_count=cal, mode=mode, m=m, n=n, scale_type=st,
                                out=out)
        ref = O.dequant_legacy(src, O.INT32, sref, st, dst_type=dt, cal_count=cal, mode=mode, m=m, n=n,
                               dst=init.copy())
    got = _bits(out)
    exp = ref.view(np.uint32) if dt == O.F32 else ref
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("n", [8, 24, 40])
@pytest.mark.parametrize("st,dt", TENSOR_COMBOS)
@pytest.mark.parametrize("mode", [O.SINGLE_ROW, O.MULTI_ROW])
def test_legacy_single_row_and_padded_rows(ascq_gpu, oracle, n, st, dt, mode):
    """m = 1 (the SINGLE_ROW rule's domain) and m = 3, n in {8, 24, 40}, every calCount that is a multiple of 8
    (reshaped where calCount fills whole 32-byte dst blocks and divides n); the full padded dst compared"""
    for m in (1, 3):
        for cal in range(8, n + 1, 8):
            _legacy_case(ascq_gpu, seeded(n * 7 + cal + m), m, n, cal, st, dt, False, mode)


@pytest.mark.parametrize("st,dt", SCALAR_COMBOS)
@pytest.mark.parametrize("m,n,cal", [(1, 16, 8), (1, 48, 16), (3, 24, 24), (5, 40, 32), (37, 96, 88)])
def test_legacy_scalar(ascq_gpu, oracle, st, dt, m, n, cal):
    _legacy_case(ascq_gpu, seeded(m + n + cal), m, n, cal, st, dt, True, O.SINGLE_ROW)


@pytest.mark.parametrize("st,dt", TENSOR_COMBOS)
@pytest.mark.parametrize("m,n,cal", [(128, 32, 24), (37, 96, 90), (1000, 264, 256), (2048, 8192, 8192),
                                     (1, 4096, 1024)])
def test_legacy_tensor_shapes(ascq_gpu, oracle, st, dt, m, n, cal):
    """calCount < n (columns beyond it untouched), ragged calCount (element kernel), rows not a multiple of the
    vector kernel's row blocks, a large block, and a reshaped single row"""
    _legacy_case(ascq_gpu, seeded(m * 3 + cal), m, n, cal, st, dt, False, O.SINGLE_ROW)


@pytest.mark.parametrize("dt", [O.F16, O.BF16, O.F32])
def test_legacy_int32_ties_away(ascq_gpu, oracle, dt):
    """full-range int32 sources with exact conversion ties (|v| > 2^24): fp32 rounds them away from zero"""
    st = O.U64 if dt == O.F16 else O.F32
    _legacy_case(ascq_gpu, seeded(5), 64, 256, 256, st, dt, False, O.SINGLE_ROW, big=True)
    _legacy_case(ascq_gpu, seeded(6), 7, 40, 24, st, dt, False, O.SINGLE_ROW, big=True)


def _policy_case(ascq_gpu, rng, rows, n, src_kind, st, dt, policy, k_dim, g, big=False, cal=None):
    if src_kind == "int32":
        src, code = _int32_src(rng, (rows, n), big), O.INT32
    elif src_kind == "int8":
        src, code = rng.integers(-128, 128, (rows, n), dtype=np.int8), O.INT8
    else:
        src = (rng.standard_normal((rows, n)) * 300).astype(np.float32)
        src.reshape(-1)[:3] = [np.inf, -1e30, 65519.0]
        code = O.F32
    if policy == O.PER_TOKEN:
        cnt = rows
    elif k_dim == 1:
        cnt = rows * -(-n // g)
    else:
        cnt = -(-rows // g) * n
    sdev, sref = _scale_tensor(rng, cnt, st)
    init = np.full((rows, n), 0x1234 if dt != O.F32 else np.float32(9.0), _NP[dt])
    out = _dev(init)
    if dt != O.F32:
        out = out.view(torch.int16).view(_TORCH[dt])
    ascq_gpu.ascend_dequant_policy(_dev(src), sdev, policy, _TORCH[dt], group_size=g, kdim=k_dim, cal_count=cal,
                                   out=out)
    ref = O.dequant_policy(src, code, sref, st, policy, dt, k_dim=k_dim, group=g, cal_count=cal, dst=init.copy())
    np.testing.assert_array_equal(_bits(out), ref.view(np.uint32) if dt == O.F32 else ref)


@pytest.mark.parametrize("src_kind", ["int32", "f32"])
@pytest.mark.parametrize("st", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("dt", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("k_dim", [0, 1])
@pytest.mark.parametrize("rows,n,g", [(70, 200, 64), (256, 512, 128), (33, 96, 32)])
def test_policy_per_group(ascq_gpu, oracle, src_kind, st, dt, k_dim, rows, n, g):
    _policy_case(ascq_gpu, seeded(rows + n + g + k_dim), rows, n, src_kind, st, dt, O.PER_GROUP, k_dim, g)


@pytest.mark.parametrize("src_kind", ["int32", "f32", "int8"])
@pytest.mark.parametrize("st", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("dt", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("rows,n", [(64, 8192), (5, 48), (3, 20), (9, 1000), (1, 16392)])
def test_policy_per_token(ascq_gpu, oracle, src_kind, st, dt, rows, n):
    _policy_case(ascq_gpu, seeded(rows * 5 + n), rows, n, src_kind, st, dt, O.PER_TOKEN, 1, 0)


def test_policy_partial_last_row_and_ties(ascq_gpu, oracle):
    """rows = calCount / n: a partial last row is left unwritten; full-range int32 sources with conversion ties"""
    _policy_case(ascq_gpu, seeded(11), 9, 48, "int32", O.F32, O.F16, O.PER_TOKEN, 1, 0, big=True, cal=8 * 48 + 5)
    _policy_case(ascq_gpu, seeded(12), 64, 256, "int32", O.F32, O.F32, O.PER_GROUP, 1, 32, big=True)
    _policy_case(ascq_gpu, seeded(13), 64, 256, "int32", O.BF16, O.BF16, O.PER_GROUP, 0, 32, big=True)


@pytest.mark.parametrize("k_dim", [0, 1])
def test_policy_per_group_full_size(ascq_gpu, oracle, k_dim):
    """int32 [8192, 8192] -> f16 with g = 128 f32 scales along each row (kDim 1) or down the columns (kDim 0)"""
    _policy_case(ascq_gpu, seeded(20 + k_dim), 8192, 8192, "int32", O.F32, O.F16, O.PER_GROUP, k_dim, 128)
