"""numpy front-end of the CPU oracle (oracle/liboracle.so).

Test infrastructure only: used by tests/, the smoke check and bench.py's cpu_baseline leg as the
checker; the product path never calls it.  Arrays are numpy; f16 / bf16 travel as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_DIR = ROOT / "oracle"
ORACLE_SO = Path(os.environ.get("ASCQ_ORACLE_SO", ORACLE_DIR / "liboracle.so"))

INT8, UINT8, INT4, INT32, F16, BF16, F32, U64, FP8_E4M3, FP8_E5M2, FP4_E2M1, E8M0, INT64, FP4_E1M2, HIF8 = range(1, 16)
ROUND_NONE, ROUND_RINT, ROUND_FLOOR, ROUND_CEIL, ROUND_ROUND, ROUND_TRUNC = range(6)
PER_TENSOR, PER_CHANNEL, PER_TOKEN, PER_GROUP = range(4)
ARITH_F16, ARITH_F32, ARITH_BF16 = 0, 1, 2

_lib = None
_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build_if_missing() -> None:
    if not ORACLE_SO.exists():
        subprocess.run(["make", "-C", str(ORACLE_DIR)], check=True, capture_output=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        build_if_missing()
        L = ctypes.CDLL(str(ORACLE_SO))
        sig = {
            "oq_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float, ctypes.c_int]),
            "oq_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oq_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float, ctypes.c_int]),
            "oq_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oq_f64_to_f16": (ctypes.c_uint16, [ctypes.c_double, ctypes.c_int]),
            "oq_f64_to_bf16": (ctypes.c_uint16, [ctypes.c_double, ctypes.c_int]),
            "oq_quant_pre_m1": (ctypes.c_float, [ctypes.c_uint64]),
            "oq_pack_quant_pre": (ctypes.c_uint64, [ctypes.c_float, ctypes.c_int32, ctypes.c_int32]),
            "oq_round_to_int": (ctypes.c_int32, [ctypes.c_float, ctypes.c_int]),
            "oq_e2m1_decode": (ctypes.c_float, [ctypes.c_uint8]),
            "oq_e2m1_encode_rne": (ctypes.c_uint8, [ctypes.c_float]),
            "oq_e8m0_decode": (ctypes.c_float, [ctypes.c_uint8]),
            "oq_mx_shared_exp": (ctypes.c_uint8, [ctypes.c_float]),
            "oq_fp8_decode": (ctypes.c_float, [ctypes.c_uint8, ctypes.c_int]),
            "oq_f32_to_fp8": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_int]),
            "oq_requant8": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_uint64]),
            "oq_mm_requant": (None, [_P, _P, _I64, _I64, _P, ctypes.c_uint64]),
            "oq_requant4": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_uint64]),
            "oq_antiquant_policy": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int,
                                           _I64, _I64, _I64, ctypes.c_int, ctypes.c_int]),
            "oq_mm_requant4": (None, [_P, _P, _I64, _I64, _P, ctypes.c_uint64]),
            "oq_e2m1_encode": (ctypes.c_uint8, [ctypes.c_double, ctypes.c_int]),
            "oq_e1m2_encode": (ctypes.c_uint8, [ctypes.c_double, ctypes.c_int]),
            "oq_e1m2_decode": (ctypes.c_float, [ctypes.c_uint8]),
            "oq_f32_to_fp8_sat": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_int]),
            "oq_quant_policy": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int,
                                       ctypes.c_float, ctypes.c_int, _I64, _I64, _I64, ctypes.c_int, ctypes.c_int]),
            "oq_requant4_f32": (None, [_P, _P, _I64, _I64, _P, ctypes.c_uint64]),
            "oq_quantize": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int,
                                   ctypes.c_float, ctypes.c_float, ctypes.c_int, _I64, _I64, _I64, ctypes.c_int,
                                   ctypes.c_int]),
            "oq_dequantize": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int, ctypes.c_float,
                                     ctypes.c_int, _I64, _I64, _I64, ctypes.c_int]),
            "oq_antiquantize": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int,
                                       ctypes.c_float, ctypes.c_float, ctypes.c_int, _I64, _I64, _I64, ctypes.c_int]),
            "oq_matmul_i8": (None, [_P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int, ctypes.c_int]),
            "oq_mm_dequant": (None, [_P, _P, ctypes.c_int, _I64, _I64, _P, ctypes.c_uint64]),
            "oq_matmul_fp8": (None, [_P, _P, ctypes.c_int, ctypes.c_int, _P, _P, ctypes.c_int, _I64, _I64, _I64,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, ctypes.c_uint64, _P, _P, _P]),
            "oq_quant_per_token": (None, [_P, _P, ctypes.c_int, _P, _P, _I64, _I64, ctypes.c_int]),
            "oq_quant_dynamic_per_token": (None, [_P, _P, _P, ctypes.c_int, _I64, _I64, ctypes.c_int]),
            "oq_quant_legacy_f16": (None, [_P, _P, ctypes.c_int, _P, ctypes.c_uint16, _P, ctypes.c_uint16, _I64, _I64]),
            "oq_i32_to_f32_rna": (ctypes.c_float, [ctypes.c_int32]),
            "oq_hif8_decode": (ctypes.c_float, [ctypes.c_uint8]),
            "oq_hif8_encode": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_int]),
            "oq_quant_legacy": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, _P, ctypes.c_float, ctypes.c_float, _I64,
                                       _I64]),
            "oq_antiquant_scalar": (None, [_P, ctypes.c_int, _P, ctypes.c_int, ctypes.c_uint16, ctypes.c_uint16,
                                           ctypes.c_int, _I64]),
            "oq_dequant_legacy": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int, ctypes.c_float,
                                         ctypes.c_int, ctypes.c_int, _I64, _I64, _I64]),
            "oq_dequant_legacy_shape": (_I64, [ctypes.c_int, ctypes.c_int, ctypes.POINTER(_I64),
                                               ctypes.POINTER(_I64), _I64]),
            "oq_dequant_policy": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, _I64, _I64, _I64]),
            "oq_antiquant": (None, [_P, ctypes.c_int, _P, ctypes.c_int, _P, _P, _I64, _I64, _I64, ctypes.c_int,
                                    ctypes.c_int]),
            "oq_antiquant_matmul": (None, [_P, _P, _P, _P, _P, ctypes.c_int, _P, _P, _I64, _I64, _I64, _I64,
                                           ctypes.c_int]),
            "oq_group_matmul": (None, [_P, ctypes.c_int, _P, _P, _P, ctypes.c_int, _P, _P, ctypes.c_int, _I64, _I64,
                                       _I64, _I64, ctypes.c_int]),
            "oq_faster_gelu": (ctypes.c_float, [ctypes.c_float]),
            "oq_nz_to_nd": (None, [_P, _P, ctypes.c_int, _I64, _I64, _I64, ctypes.c_int]),
            "oq_nd_to_nz": (None, [_P, _P, ctypes.c_int, _I64, _I64, _I64]),
            "oq_mx_matmul": (None, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, _P, _I64, _P, _P]),
            "oq_c_combine": (None, [_P, _P, ctypes.c_int, ctypes.c_int, _I64]),
            "oq_mx_quantize_fp4": (None, [_P, _P, _P, _I64, _I64]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


# ---------------- scalar helpers (vectorised over numpy inputs) ----------------
def f32_to_f16(x, sat=True) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    f = lib().oq_f32_to_f16
    return np.array([f(float(v), int(sat)) for v in x], dtype=np.uint16)


def matmul_i8(A, B, bias=None, trans_a=False, trans_b=False):
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    M = A.shape[1] if trans_a else A.shape[0]
    K = A.shape[0] if trans_a else A.shape[1]
    N = B.shape[0] if trans_b else B.shape[1]
    C = np.empty((M, N), np.int32)
    b = None if bias is None else np.ascontiguousarray(bias, np.int32)
    lib().oq_matmul_i8(_p(A), _p(B), _p(b), _p(C), M, N, K, int(trans_a), int(trans_b))
    return C


def matmul_fp8(A, B, a_fmt, b_fmt, bias=None, out_type=F32, trans_a=False, trans_b=False, use_q=False, qvec=None,
               qscalar=0):
    """fp8 / hifloat8 Matmul (bytes in, codes FP8_E4M3 / FP8_E5M2, or HIF8 for both): returns (out, exact fp64
    sum + bias, sum |a b|, sum over 16-element K groups of the group's largest |a b|)."""
    A = np.ascontiguousarray(A, np.uint8)
    B = np.ascontiguousarray(B, np.uint8)
    M = A.shape[1] if trans_a else A.shape[0]
    K = A.shape[0] if trans_a else A.shape[1]
    N = B.shape[0] if trans_b else B.shape[1]
    odt = {F32: np.float32, INT8: np.int8, UINT8: np.uint8, FP8_E4M3: np.uint8, FP8_E5M2: np.uint8,
           HIF8: np.uint8}.get(out_type, np.uint16)
    out = np.empty((M, N), odt)
    exact = np.empty((M, N), np.float64)
    absd = np.empty((M, N), np.float64)
    bmax = np.empty((M, N), np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    qv = None if qvec is None else np.ascontiguousarray(qvec, np.uint64)
    lib().oq_matmul_fp8(_p(A), _p(B), a_fmt, b_fmt, _p(b), _p(out), out_type, M, N, K, int(trans_a), int(trans_b),
                        int(use_q), _p(qv), int(qscalar), _p(exact), _p(absd), _p(bmax))
    return out, exact, absd, bmax


def nz_size(esize, batch, rows, cols):
    return batch * ((cols * esize + 31) // 32) * ((rows + 15) // 16) * 512


def nz_to_nd(nz, esize, batch, rows, cols, transpose_out=False):
    nz = np.ascontiguousarray(nz, np.uint8).reshape(-1)
    out = np.empty(batch * rows * cols * esize, np.uint8)
    lib().oq_nz_to_nd(_p(out), _p(nz), esize, batch, rows, cols, int(transpose_out))
    return out.reshape((batch, cols, rows * esize) if transpose_out else (batch, rows, cols * esize))


def nd_to_nz(nd, esize, batch, rows, cols):
    nd = np.ascontiguousarray(nd).view(np.uint8).reshape(-1)
    out = np.empty(nz_size(esize, batch, rows, cols), np.uint8)
    lib().oq_nd_to_nz(_p(out), _p(nd), esize, batch, rows, cols)
    return out


def mm_requant(acc, qvec=None, qscalar=0):
    """(V)REQ8: int32 accumulators -> bytes (int8 or uint8 per the words' sign flag), returned as uint8"""
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    out = np.empty((M, N), np.uint8)
    qv = None if qvec is None else np.ascontiguousarray(qvec, np.uint64)
    lib().oq_mm_requant(_p(acc), _p(out), M, N, _p(qv), int(qscalar))
    return out


def antiquant_policy(src, src_type, scale, scale_type, dst_type, policy, m, n, group=0, offset=None, k_dim=0,
                     is_transpose=False):
    """AscendAntiQuant policy form over [m, n]: src int8 [m, n], fp8 bytes [m, n] or fp4 [m, n/2]; scale / offset
    arrays of scale_type (f16 / bf16 as uint16 bits, f32, E8M0 bytes); returns dst (uint16 bits or float32)"""
    out = np.empty((m, n), np.float32 if dst_type == F32 else np.uint16)
    src = np.ascontiguousarray(src)
    sc = np.ascontiguousarray(scale)
    of = None if offset is None else np.ascontiguousarray(offset)
    lib().oq_antiquant_policy(_p(out), dst_type, _p(src), src_type, _p(sc), _p(of), scale_type, policy, m, n, group,
                              k_dim, int(is_transpose))
    return out


def quant_policy(src, src_type, scale, scale_type, dst_type, policy, m, n, group=0, offset=None,
                 offset_scalar=None, k_dim=1, round_mode=ROUND_RINT):
    """AscendQuant policy form over [m, n]: src (uint16 bits or float32) [m, n]; scale / offset arrays of
    scale_type; offset_scalar a float (rounded to scale_type); returns int8 [m, n], fp8 bytes [m, n] or fp4
    codes packed [m, n/2]"""
    if dst_type in (FP4_E2M1, FP4_E1M2):
        out = np.empty((m, n // 2), np.uint8)
    else:
        out = np.empty((m, n), np.int8 if dst_type == INT8 else np.uint8)
    src = np.ascontiguousarray(src)
    sc = np.ascontiguousarray(scale)
    of = None if offset is None else np.ascontiguousarray(offset)
    has_off = offset is not None or offset_scalar is not None
    lib().oq_quant_policy(_p(out), dst_type, _p(src), src_type, _p(sc), scale_type, _p(of), int(has_off),
                          float(offset_scalar or 0.0), policy, m, n, group, k_dim, round_mode)
    return out


def quantize(src, src_type, dst_type, policy, m, n, scale=None, scale_type=F32, offset=None, scale_scalar=1.0,
             offset_scalar=None, group=0, k_dim=1, round_mode=ROUND_RINT):
    """Quantize (the newer interface) over [m, n]: src (uint16 bits or float32); scale / offset arrays of scale_type
    (PER_TENSOR: the scalars); returns int8 [m, n], byte codes [m, n] or fp4 codes packed [m, n/2]"""
    if dst_type in (FP4_E2M1, FP4_E1M2):
        out = np.empty((m, n // 2), np.uint8)
    else:
        out = np.empty((m, n), np.int8 if dst_type == INT8 else np.uint8)
    sc = None if scale is None else np.ascontiguousarray(scale)
    of = None if offset is None else np.ascontiguousarray(offset)
    has_off = offset is not None or offset_scalar is not None
    lib().oq_quantize(_p(out), dst_type, _p(np.ascontiguousarray(src)), src_type, _p(sc), scale_type, _p(of),
                      int(has_off), float(scale_scalar), float(offset_scalar or 0.0), policy, m, n, group, k_dim,
                      round_mode)
    return out


def dequantize(src, src_type, dst_type, policy, scale=None, scale_type=F32, scale_scalar=1.0, group=0, k_dim=1):
    """Dequantize (the newer interface) of src [m, n]; returns [m, n] (uint16 bits or float32)"""
    src = np.ascontiguousarray(src)
    m, n = src.shape
    dst = np.zeros((m, n), np.float32 if dst_type == F32 else np.uint16)
    sc = None if scale is None else np.ascontiguousarray(scale)
    lib().oq_dequantize(_p(dst), dst_type, _p(src), src_type, _p(sc), scale_type, float(scale_scalar), policy, m, n,
                        group, k_dim)
    return dst


def antiquantize(src, src_type, dst_type, policy, m, n, scale=None, scale_type=F16, offset=None, scale_scalar=1.0,
                 offset_scalar=None, group=0, k_dim=1):
    """AntiQuantize (the newer interface) over [m, n] (fp4: [m, n/2] bytes); returns [m, n] (uint16 bits or
    float32)"""
    dst = np.empty((m, n), np.float32 if dst_type == F32 else np.uint16)
    sc = None if scale is None else np.ascontiguousarray(scale)
    of = None if offset is None else np.ascontiguousarray(offset)
    has_off = offset is not None or offset_scalar is not None
    lib().oq_antiquantize(_p(dst), dst_type, _p(np.ascontiguousarray(src)), src_type, _p(sc), scale_type, _p(of),
                          int(has_off), float(scale_scalar), float(offset_scalar or 0.0), policy, m, n, group, k_dim)
    return dst


def mm_requant4(acc, qvec=None, qscalar=0):
    """(V)REQ4: int32 accumulators [M, N] (N even) -> int4 codes packed two per byte [M, N/2]"""
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    out = np.empty((M, N // 2), np.uint8)
    qv = None if qvec is None else np.ascontiguousarray(qvec, np.uint64)
    lib().oq_mm_requant4(_p(acc), _p(out), M, N, _p(qv), int(qscalar))
    return out


def requant4_f32(v, qvec=None, qscalar=0):
    """(V)QF322S4_PRE on fp32 values (acc + bias) [M, N] (N even) -> packed int4 codes [M, N/2]"""
    v = np.ascontiguousarray(v, np.float32)
    M, N = v.shape
    out = np.empty((M, N // 2), np.uint8)
    qv = None if qvec is None else np.ascontiguousarray(qvec, np.uint64)
    lib().oq_requant4_f32(_p(v), _p(out), M, N, _p(qv), int(qscalar))
    return out


def unpack_int4(packed, n):
    """[M, N/2] bytes -> [M, N] int8 values (even column in the low nibble, two's complement nibbles)"""
    lo = (packed & 0xF).astype(np.int8)
    hi = (packed >> 4).astype(np.int8)
    out = np.empty((packed.shape[0], n), np.int8)
    out[:, 0::2] = np.where(lo >= 8, lo - 16, lo)
    out[:, 1::2] = np.where(hi >= 8, hi - 16, hi)
    return out


def mm_dequant(acc, out_type=F16, qvec=None, qscalar=0):
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    out = np.empty((M, N), np.uint16)
    qv = None if qvec is None else np.ascontiguousarray(qvec, np.uint64)
    lib().oq_mm_dequant(_p(acc), _p(out), out_type, M, N, _p(qv), int(qscalar))
    return out


def quant_per_token(x, src_type, scale, offset=None, round_mode=ROUND_RINT):
    x = np.ascontiguousarray(x)
    m, n = x.shape
    q = np.empty((m, n), np.int8)
    s = np.ascontiguousarray(scale, np.float32)
    o = None if offset is None else np.ascontiguousarray(offset, np.float32)
    lib().oq_quant_per_token(_p(q), _p(x), src_type, _p(s), _p(o), m, n, round_mode)
    return q


def quant_dynamic_per_token(x, src_type, round_mode=ROUND_RINT):
    x = np.ascontiguousarray(x)
    m, n = x.shape
    q = np.empty((m, n), np.int8)
    s = np.empty((m,), np.float32)
    lib().oq_quant_dynamic_per_token(_p(q), _p(s), _p(x), src_type, m, n, round_mode)
    return q, s


def quant_legacy_f16(x, src_type, scale_vec=None, scale_scalar=0x3C00, offset_vec=None, offset_scalar=0,
                     scale_count=0):
    x = np.ascontiguousarray(x)
    q = np.empty(x.shape, np.int8)
    sv = None if scale_vec is None else np.ascontiguousarray(scale_vec, np.uint16)
    ov = None if offset_vec is None else np.ascontiguousarray(offset_vec, np.uint16)
    lib().oq_quant_legacy_f16(_p(q), _p(x), src_type, _p(sv), scale_scalar, _p(ov), offset_scalar, x.size,
                              scale_count)
    return q


def hif8_table():
    """float32 values of the 256 HiFloat8 codes"""
    L = lib()
    return np.array([L.oq_hif8_decode(c) for c in range(256)], np.float32)


def hif8_encode(x, sat=True):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    L = lib()
    return np.array([L.oq_hif8_encode(float(v), int(sat)) for v in x], np.uint8)


def quant_legacy(x, src_type, dst_type, scale=None, offset=None, scale_scalar=1.0, offset_scalar=0.0, scale_count=0):
    """Legacy AscendQuant (arch-3510 form): x raw array (f16 / bf16 as uint16 bits, or float32); scale / offset
    srcT arrays or None"""
    x = np.ascontiguousarray(x)
    q = np.empty(x.shape, np.uint8)
    sc = None if scale is None else np.ascontiguousarray(scale)
    of = None if offset is None else np.ascontiguousarray(offset)
    lib().oq_quant_legacy(_p(q), dst_type, _p(x), src_type, _p(sc), _p(of), float(scale_scalar), float(offset_scalar),
                          x.size, scale_count)
    return q.view(np.int8) if dst_type == INT8 else q


def antiquant_scalar(src, src_type, offset_bits, scale_bits, dst_type=F16, has_offset=True):
    """per-tensor AscendAntiQuant of every element of src (int4: two per byte)"""
    src = np.ascontiguousarray(src)
    count = src.size * (2 if src_type == INT4 else 1)
    dst = np.empty(count, np.uint16)
    lib().oq_antiquant_scalar(_p(dst), dst_type, _p(src), src_type, int(offset_bits), int(scale_bits),
                              int(has_offset), count)
    return dst


SINGLE_ROW, MULTI_ROW = 0, 1


def dequant_legacy_shape(dst_type, m, n, cal_count, mode=SINGLE_ROW):
    """(rows, cols, dst row stride) of the legacy form after the DEQUANT_WITH_SINGLE_ROW rule"""
    mm, nn = _I64(m), _I64(n)
    ldd = lib().oq_dequant_legacy_shape(dst_type, mode, ctypes.byref(mm), ctypes.byref(nn), cal_count)
    return mm.value, nn.value, ldd


def dequant_legacy(src, src_type, scale, scale_type, per_tensor=False, dst_type=F16, cal_count=None,
                   scale_scalar=1.0, mode=SINGLE_ROW, dst=None, m=None, n=None):
    """Legacy AscendDequant on DequantParams {m, n, calCount} (src holds m * n elements).  Returns dst as
    [rows, dst row stride] (the reference's padded layout); unwritten elements keep dst's initial values."""
    src = np.ascontiguousarray(src)
    if m is None:
        m, n = src.shape
    cal = n if cal_count is None else cal_count
    rows, _, ldd = dequant_legacy_shape(dst_type, m, n, cal, mode)
    if dst is None:
        dst = np.zeros((rows, ldd), np.float32 if dst_type == F32 else np.uint16)
    sc = None if scale is None else np.ascontiguousarray(scale)
    lib().oq_dequant_legacy(_p(dst), dst_type, _p(src), src_type, _p(sc), scale_type, float(scale_scalar),
                            int(per_tensor), mode, m, n, cal)
    return dst


def dequant_policy(src, src_type, scale, scale_type, policy, dst_type=F16, k_dim=1, group=0, cal_count=None,
                   dst=None):
    """AscendDequant policy form (PER_TOKEN / PER_GROUP) on src [rows, n]"""
    src = np.ascontiguousarray(src)
    rows, n = src.shape
    cal = rows * n if cal_count is None else cal_count
    if dst is None:
        dst = np.zeros((rows, n), np.float32 if dst_type == F32 else np.uint16)
    lib().oq_dequant_policy(_p(dst), dst_type, _p(src), src_type, _p(np.ascontiguousarray(scale)), scale_type, policy,
                            k_dim, n, cal, group)
    return dst


def antiquant(src, src_type, scale, offset, K, N, group_size=0, is_transpose=False, dst_type=F16, arith=ARITH_F16):
    src = np.ascontiguousarray(src)
    dst = np.empty((N, K) if is_transpose else (K, N), np.uint16)
    sc = np.ascontiguousarray(scale, np.uint16)
    of = None if offset is None else np.ascontiguousarray(offset, np.uint16)
    lib().oq_antiquant(_p(dst), dst_type, _p(src), src_type, _p(of), _p(sc), K, N, group_size, int(is_transpose),
                       arith)
    return dst


def antiquant_matmul(x_f16bits, w, w_type, scale, offset, group_size, M, N, K, w_transpose=False):
    x = np.ascontiguousarray(x_f16bits, np.uint16)
    w = np.ascontiguousarray(w)
    y = np.empty((M, N), np.uint16)
    ye = np.empty((M, N), np.float64)
    ya = np.empty((M, N), np.float64)
    sc = np.ascontiguousarray(scale, np.uint16)
    of = None if offset is None else np.ascontiguousarray(offset, np.uint16)
    lib().oq_antiquant_matmul(_p(y), _p(ye), _p(ya), _p(x), _p(w), w_type, _p(sc), _p(of), group_size, M, N, K,
                              int(w_transpose))
    return y, ye, ya


def group_matmul(x, pts, w, scale, group_list, list_type, G, M, K, N, out_type=BF16, w_trans=False, y=None, act=0):
    x = np.ascontiguousarray(x, np.int8)
    pts = np.ascontiguousarray(pts, np.float32)
    w = np.ascontiguousarray(w, np.int8)
    scale = np.ascontiguousarray(scale, np.float32)
    gl = np.ascontiguousarray(group_list, np.int64)
    if y is None:
        y = np.zeros((M, N), np.uint16)
    lib().oq_group_matmul(_p(y), out_type, _p(x), _p(pts), _p(w), int(w_trans), _p(scale), _p(gl), list_type, G, M, K,
                          N, int(act))
    return y


def mx_matmul(A, B, sA, sB, M, N, K, trans_b=False, sa_layout=0, sb_layout=0, elem_fmt=FP4_E2M1, rows=None,
              fmt_b=None, blockmax=False, bias=None):
    """returns (bf16 C, exact fp64 C, sum |a b| (+ |bias|)) and, with blockmax=True, the sum over 16-element K
    groups of the group's largest |a b| as a fourth array; bias: f32 [N] added to the sums"""
    A = np.ascontiguousarray(A, np.uint8)
    B = np.ascontiguousarray(B, np.uint8)
    sA = np.ascontiguousarray(sA, np.uint8)
    sB = np.ascontiguousarray(sB, np.uint8)
    C = np.zeros((M, N), np.uint16)
    Ce = np.zeros((M, N), np.float64)
    Ca = np.zeros((M, N), np.float64)
    Cb = np.zeros((M, N), np.float64) if blockmax else None
    r = None if rows is None else np.ascontiguousarray(rows, np.int64)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().oq_mx_matmul(_p(C), _p(Ce), _p(Ca), _p(A), _p(B), _p(sA), _p(sB), M, N, K, int(trans_b), sa_layout,
                       sb_layout, elem_fmt | ((fmt_b or 0) << 8), _p(r), 0 if r is None else r.size, _p(Cb), _p(bb))
    return (C, Ce, Ca, Cb) if blockmax else (C, Ce, Ca)


def c_combine(c, v, c_type, op):
    """IterateAll enAtomic on the host: returns op(c, v) element-wise in C's type (op 1 add, 2 max, 3 min);
    c / v: int32, float32, or uint16 bit patterns for F16 / BF16"""
    dt = {INT32: np.int32, F32: np.float32, F16: np.uint16, BF16: np.uint16}[c_type]
    out = np.ascontiguousarray(c, dt).copy()
    vv = np.ascontiguousarray(v, dt)
    assert out.shape == vv.shape
    lib().oq_c_combine(_p(out), _p(vv), c_type, op, out.size)
    return out


def mx_quantize_fp4(x):
    x = np.ascontiguousarray(x, np.float32)
    R, K = x.shape
    packed = np.empty((R, K // 2), np.uint8)
    scales = np.empty((R, K // 32), np.uint8)
    lib().oq_mx_quantize_fp4(_p(packed), _p(scales), _p(x), R, K)
    return packed, scales
