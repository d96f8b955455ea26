"""ascq -- Python binding of libascq.so (the gfx950 quantized-inference library).

Thin ctypes layer over the C ABI declared in include/ascq.h.  Tensors are torch tensors on the
GPU (torch is used for device memory and streams only); every compute call goes through the
C ABI into the HIP kernels.  There is no CPU fallback: if libascq.so is missing or a call fails,
an exception is raised.

The operator names and argument meanings mirror the reference's operator surface
(AscendC::Matmul SetTensorA/SetTensorB/SetBias/SetQuantScalar/SetQuantVector/IterateAll/End,
AscendQuant/AscendDequant/AscendAntiQuant, QuantGroupMatmul); see include/ascq.h for the
reference file:line each entry point replaces.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

_PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("ASCQ_LIB", _PKG_DIR / "libascq.so"))

# ascq_dtype
INT8, UINT8, INT4, INT32, F16, BF16, F32, U64, FP8_E4M3, FP8_E5M2, FP4_E2M1, E8M0, INT64, FP4_E1M2, HIF8 = range(1, 16)
# ascq_round_mode
ROUND_NONE, ROUND_RINT, ROUND_FLOOR, ROUND_CEIL, ROUND_ROUND, ROUND_TRUNC = range(6)
# ascq_policy
ACT_NONE, ACT_FASTER_GELU = 0, 1
PER_TENSOR, PER_CHANNEL, PER_TOKEN, PER_GROUP = range(4)
# IterateAll enAtomic (matmul_config_utils.h:53-55)
ATOMIC_NONE, ATOMIC_ADD, ATOMIC_MAX, ATOMIC_MIN = range(4)
# ascq_arith
ARITH_F16, ARITH_F32 = 0, 1
# ascq_dequant_mode (DeQuantMode)
DEQUANT_SINGLE_ROW, DEQUANT_MULTI_ROW = 0, 1
# ascq_format
FORMAT_ND, FORMAT_PACKED, FORMAT_NZ = 0, 1, 2

OK, E_INVALID_ARG, E_UNSUPPORTED, E_HIP, E_STATE = 0, -1, -2, -3, -4

_TORCH_OF = {INT8: torch.int8, INT32: torch.int32, F16: torch.float16, BF16: torch.bfloat16, F32: torch.float32}


class AscqError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"ascq error {status}: {message}")
        self.status = status


class _QuantParam(ctypes.Structure):
    _fields_ = [
        ("m", ctypes.c_uint32),
        ("n", ctypes.c_uint32),
        ("cal_count", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
        ("has_offset", ctypes.c_int32),
        ("kdim", ctypes.c_int32),
        ("round_mode", ctypes.c_int32),
    ]


class _DequantParam(ctypes.Structure):
    _fields_ = [("m", ctypes.c_uint32), ("n", ctypes.c_uint32), ("cal_count", ctypes.c_uint32)]


class _DequantPolicyParam(ctypes.Structure):
    _fields_ = [("m", ctypes.c_uint32), ("n", ctypes.c_uint32), ("cal_count", ctypes.c_uint32),
                ("group_size", ctypes.c_uint32), ("has_offset", ctypes.c_int32), ("kdim", ctypes.c_int32)]


class _QuantizeParam(ctypes.Structure):
    """ascq_quantize_param: QuantizeConfig{policy, hasOffset, roundMode, kDim} + QuantizeParams{m, n, groupSize}"""
    _fields_ = [("policy", ctypes.c_int32), ("has_offset", ctypes.c_int32), ("round_mode", ctypes.c_int32),
                ("kdim", ctypes.c_int32), ("m", ctypes.c_uint32), ("n", ctypes.c_uint32),
                ("group_size", ctypes.c_uint32)]


class _MatmulTypes(ctypes.Structure):
    _fields_ = [
        ("a_type", ctypes.c_int32),
        ("b_type", ctypes.c_int32),
        ("c_type", ctypes.c_int32),
        ("bias_type", ctypes.c_int32),
        ("scale_type", ctypes.c_int32),
        ("b_format", ctypes.c_int32),
    ]


CUBE_TILING_FIELDS = (
    "usedCoreNum M N Ka Kb singleCoreM singleCoreN singleCoreK baseM baseN baseK depthA1 depthB1 stepM stepN isBias "
    "transLength iterateOrder shareMode shareL1Size shareL0CSize shareUbSize batchM batchN singleBatchM singleBatchN "
    "stepKa stepKb depthAL1CacheUB depthBL1CacheUB dbL0A dbL0B dbL0C ALayoutInfoB ALayoutInfoS ALayoutInfoN "
    "ALayoutInfoG ALayoutInfoD BLayoutInfoB BLayoutInfoS BLayoutInfoN BLayoutInfoG BLayoutInfoD CLayoutInfoB "
    "CLayoutInfoS1 CLayoutInfoN CLayoutInfoG CLayoutInfoS2 BatchNum mxTypePara").split()


class CubeTiling(ctypes.Structure):
    """ascq_cube_tiling: the reference's TCubeTiling fields in their order (matmul_tilingdata.h:21-72)"""
    _fields_ = [(f, ctypes.c_int32) for f in CUBE_TILING_FIELDS]


_P = ctypes.c_void_p
_I32, _U32, _I64, _U64, _U16, _U8, _F32 = (ctypes.c_int32, ctypes.c_uint32, ctypes.c_int64, ctypes.c_uint64,
                                          ctypes.c_uint16, ctypes.c_uint8, ctypes.c_float)

# name -> (restype, argtypes)
SIGNATURES = {
    "ascq_last_error": (ctypes.c_char_p, []),
    "ascq_version": (ctypes.c_char_p, []),
    "ascq_device_count": (_I32, []),
    "ascq_set_launch_events": (_I32, [_P, _P]),
    "ascq_pack_quant_pre": (_U64, [_F32, _I32, _I32]),
    "ascq_matmul_create": (_I32, [ctypes.POINTER(_MatmulTypes), ctypes.POINTER(_P)]),
    "ascq_matmul_init": (_I32, [_P, ctypes.POINTER(CubeTiling)]),
    "ascq_matmul_set_org_shape": (_I32, [_P, _I64, _I64, _I64]),
    "ascq_matmul_set_single_shape": (_I32, [_P, _I64, _I64, _I64]),
    "ascq_matmul_set_tail": (_I32, [_P, _I64, _I64, _I64]),
    "ascq_matmul_set_tensor_a": (_I32, [_P, _P, _I32]),
    "ascq_matmul_set_tensor_b": (_I32, [_P, _P, _I32]),
    "ascq_matmul_set_bias": (_I32, [_P, _P]),
    "ascq_matmul_disable_bias": (_I32, [_P]),
    "ascq_matmul_set_quant_scalar": (_I32, [_P, _U64]),
    "ascq_matmul_set_quant_vector": (_I32, [_P, _P]),
    "ascq_matmul_set_antiquant_scalar": (_I32, [_P, _U16, _U16]),
    "ascq_matmul_set_antiquant_vector": (_I32, [_P, _P, _P, _I64]),
    "ascq_matmul_set_tensor_scale_a": (_I32, [_P, _P, _I32]),
    "ascq_matmul_set_tensor_scale_b": (_I32, [_P, _P, _I32]),
    "ascq_matmul_workspace_size": (_I32, [_P, ctypes.POINTER(ctypes.c_size_t)]),
    "ascq_matmul_set_workspace": (_I32, [_P, _P, ctypes.c_size_t]),
    "ascq_matmul_iterate_all": (_I32, [_P, _P, _U8, _P]),
    "ascq_matmul_iterate_all_noalloc": (_I32, [_P, _P, _U8, _P]),
    "ascq_matmul_end": (_I32, [_P]),
    "ascq_matmul_destroy": (_I32, [_P]),
    "ascq_ascend_quant_per_token": (_I32, [_P, _P, _I32, _P, _P, ctypes.POINTER(_QuantParam), _P]),
    "ascq_ascend_quant_dynamic_per_token": (_I32, [_P, _P, _P, _I32, _U32, _U32, _I32, _P]),
    "ascq_ascend_quant_policy": (_I32, [_P, _I32, _P, _I32, _P, _P, _F32, _I32, _I32, ctypes.POINTER(_QuantParam), _P]),
    "ascq_ascend_quant": (_I32, [_P, _I32, _P, _I32, _P, _P, _F32, _F32, _U32, _U32, _P]),
    "ascq_ascend_antiquant_scalar": (_I32, [_P, _I32, _P, _I32, _U16, _U16, _I32, _U64, _P]),
    "ascq_ascend_dequant": (_I32, [_P, _I32, _P, _I32, _P, _I32, _F32, _I32, _I32, ctypes.POINTER(_DequantParam),
                                   _P]),
    "ascq_ascend_dequant_dst_shape": (_I32, [_I32, _I32, ctypes.POINTER(_DequantParam), ctypes.POINTER(_U32),
                                             ctypes.POINTER(_U32)]),
    "ascq_ascend_dequant_policy": (_I32, [_P, _I32, _P, _I32, _P, _P, _I32, _I32, ctypes.POINTER(_DequantPolicyParam),
                                          _P]),
    "ascq_ascend_antiquant": (_I32, [_P, _I32, _P, _I32, _P, _P, _U32, _U32, _U32, _I32, _I32, _P]),
    "ascq_quantize": (_I32, [_P, _I32, _P, _I32, _P, _P, _F32, _F32, _I32, ctypes.POINTER(_QuantizeParam), _P]),
    "ascq_dequantize": (_I32, [_P, _I32, _P, _I32, _P, _F32, _I32, ctypes.POINTER(_QuantizeParam), _P]),
    "ascq_antiquantize": (_I32, [_P, _I32, _P, _I32, _P, _P, _F32, _F32, _I32, ctypes.POINTER(_QuantizeParam), _P]),
    "ascq_ascend_antiquant_policy": (_I32, [_P, _I32, _P, _I32, _P, _P, _I32, _I32, ctypes.c_int64, ctypes.c_int64,
                                            ctypes.c_int64, _I32, _I32, _P]),
    "ascq_weight_pack_size": (_I32, [_I32, _I64, _I64, ctypes.POINTER(ctypes.c_size_t)]),
    "ascq_weight_pack": (_I32, [_P, _P, _I32, _I64, _I64, _I32, _P]),
    "ascq_antiquant_matmul": (_I32, [_P, _P, _P, _I32, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "ascq_quant_group_matmul": (_I32, [_P, _I32, _P, _P, _P, _I32, _P, _P, _I32, _I64, _I64, _I64, _I64, _I32, _P]),
    "ascq_nz_size": (ctypes.c_size_t, [_I32, _I64, _I64, _I64]),
    "ascq_nz_to_nd": (_I32, [_P, _P, _I32, _I64, _I64, _I64, _I32, _P]),
    "ascq_nd_to_nz": (_I32, [_P, _P, _I32, _I64, _I64, _I64, _P]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libascq.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise AscqError(E_STATE, f"{LIB_PATH} not found: build it with python asc-devkit_clone_amd/build.py")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().ascq_last_error().decode()


def check(status: int, what: str) -> None:
    if status != OK:
        raise AscqError(status, f"{what}: {last_error()}")


def _ptr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    return torch.cuda.current_stream().cuda_stream


def _half_bits(v: float) -> int:
    return int(torch.tensor([v], dtype=torch.float16).view(torch.int16).item()) & 0xFFFF


def pack_quant_pre(m1: float, offset9: int = 0, sign: int = 0) -> int:
    return int(lib().ascq_pack_quant_pre(float(m1), offset9, sign))


# ------------------------------------------------------------------------------------------
# AscendQuant / AscendDequant / AscendAntiQuant
# ------------------------------------------------------------------------------------------
def quant_dynamic_per_token(x: torch.Tensor, round_mode: int = ROUND_RINT, out=None, scale_out=None, stream=None):
    """Per-row absmax -> int8 q and fp32 scale (= absmax/127).  x: [m, n] f16 / bf16 / f32."""
    m, n = x.shape
    src_type = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}[x.dtype]
    q = out if out is not None else torch.empty((m, n), dtype=torch.int8, device=x.device)
    s = scale_out if scale_out is not None else torch.empty((m,), dtype=torch.float32, device=x.device)
    check(lib().ascq_ascend_quant_dynamic_per_token(_ptr(q), _ptr(s), _ptr(x), src_type, m, n, round_mode,
                                                    _stream(stream)), "quant_dynamic_per_token")
    return q, s


def quant_per_token(x: torch.Tensor, scale: torch.Tensor, offset=None, round_mode: int = ROUND_RINT, out=None,
                    stream=None):
    """AscendQuant PER_TOKEN: q = sat_s8(round(f32(x) * scale[row] (+ offset[row])))."""
    m, n = x.shape
    src_type = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}[x.dtype]
    q = out if out is not None else torch.empty((m, n), dtype=torch.int8, device=x.device)
    p = _QuantParam(m, n, m * n, 0, 1 if offset is not None else 0, 1, round_mode)
    check(lib().ascq_ascend_quant_per_token(_ptr(q), _ptr(x), src_type, _ptr(scale), _ptr(offset), ctypes.byref(p),
                                            _stream(stream)), "quant_per_token")
    return q


def ascend_quant_policy(x: torch.Tensor, scale: torch.Tensor, policy: int, dst_type: int = INT8,
                        group_size: int = 0, offset=None, offset_scalar=None, k_dim: int = 1,
                        round_mode: int = ROUND_RINT, scale_type: int | None = None, out=None, stream=None):
    """AscendQuant policy form (PER_TOKEN / PER_GROUP) of x [m, n] (f16 / bf16 / f32) to int8, fp8 (e4m3 / e5m2;
    returned as uint8 codes) or fp4 E2M1 / E1M2 (two codes a byte, [m, n/2] uint8).  scale / offset f16 / bf16 / f32; a
    scalar offset_scalar applies when no offset tensor is given."""
    m, n = x.shape
    src_type = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}[x.dtype]
    if scale_type is None:
        scale_type = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}[scale.dtype]
    if out is not None:
        q = out
    elif dst_type in (FP4_E2M1, FP4_E1M2):
        q = torch.empty((m, n // 2), dtype=torch.uint8, device=x.device)
    else:
        q = torch.empty((m, n), dtype=torch.int8 if dst_type == INT8 else torch.uint8, device=x.device)
    has_off = offset is not None or offset_scalar is not None
    p = _QuantParam(m, n, m * n, group_size, int(has_off), k_dim, round_mode)
    check(lib().ascq_ascend_quant_policy(_ptr(q), dst_type, _ptr(x), src_type, _ptr(scale), _ptr(offset),
                                         float(offset_scalar or 0.0), scale_type, policy, ctypes.byref(p),
                                         _stream(stream)), "ascend_quant_policy")
    return q


def ascend_quant(x: torch.Tensor, dst_type: int = INT8, scale=None, offset=None, scale_scalar: float = 1.0,
                 offset_scalar: float = 0.0, scale_count: int = 0, out=None, stream=None):
    """Legacy AscendQuant (arch-3510 form): per tensor (float scalars) or per channel (scale / offset tensors of the
    source's type; offset None takes offset_scalar as a source-typed value).  dst INT8 / HIF8 (half arithmetic) or
    FP8_E4M3 / FP8_E5M2 (fp32 arithmetic); returns int8 (INT8) or uint8 codes of x's shape."""
    src_type = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}[x.dtype]
    q = out if out is not None else torch.empty(x.shape, dtype=torch.int8 if dst_type == INT8 else torch.uint8,
                                                device=x.device)
    if scale is not None:
        scale_count = scale_count or scale.numel()
    check(lib().ascq_ascend_quant(_ptr(q), dst_type, _ptr(x), src_type, _ptr(scale), _ptr(offset), float(scale_scalar),
                                  float(offset_scalar), x.numel(), scale_count, _stream(stream)), "ascend_quant")
    return q


def _dtype_code(t) -> int:
    return {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}[t]


def dequant_dst_shape(dst_dtype, m: int, n: int, cal_count: int, mode: int = DEQUANT_SINGLE_ROW):
    """(rows, row stride) of the legacy AscendDequant's dst after the DEQUANT_WITH_SINGLE_ROW rule"""
    rows, ldd = _U32(), _U32()
    p = _DequantParam(m, n, cal_count)
    check(lib().ascq_ascend_dequant_dst_shape(_dtype_code(dst_dtype), mode, ctypes.byref(p), ctypes.byref(rows),
                                              ctypes.byref(ldd)), "ascend_dequant_dst_shape")
    return rows.value, ldd.value


def ascend_dequant(src: torch.Tensor, scale, dst_dtype=torch.float16, cal_count=None, scale_scalar: float = 1.0,
                   scale_type: int | None = None, mode: int = DEQUANT_SINGLE_ROW, m: int | None = None,
                   n: int | None = None, out=None, stream=None):
    """Legacy AscendDequant<dstT, scaleT, mode>(dst, src, deqScale, {m, n, calCount}): `scale` a deqScale tensor
    (f32 / bf16, or int64 holding uint64 words) or None for the scalar `scale_scalar` (scale_type F32 or BF16).
    Returns dst as [rows, row stride] (rows of n padded to 32 bytes; unwritten elements keep `out`'s values)."""
    if m is None:
        m, n = src.shape
    cal = n if cal_count is None else cal_count
    src_type = {torch.int32: INT32, torch.int8: INT8}[src.dtype]
    dst_type = _dtype_code(dst_dtype)
    if scale_type is None:
        scale_type = F32 if scale is None else {torch.float32: F32, torch.bfloat16: BF16, torch.int64: U64}[scale.dtype]
    rows, ldd = dequant_dst_shape(dst_dtype, m, n, cal, mode)
    y = out if out is not None else torch.empty((rows, ldd), dtype=dst_dtype, device=src.device)
    p = _DequantParam(m, n, cal)
    check(lib().ascq_ascend_dequant(_ptr(y), dst_type, _ptr(src), src_type, _ptr(scale), scale_type,
                                    float(scale_scalar), PER_TENSOR if scale is None else PER_CHANNEL, mode,
                                    ctypes.byref(p), _stream(stream)), "ascend_dequant")
    return y


def ascend_dequant_policy(src: torch.Tensor, scale: torch.Tensor, policy: int, dst_dtype=torch.float16,
                          group_size: int = 0, kdim: int = 1, cal_count=None, offset=None, out=None, stream=None):
    """AscendDequant<dstT, srcT, scaleT, {hasOffset, kDim}, policy>(dst, src, scale, offset, {m, n, calCount,
    groupSize}): PER_TOKEN (scale[row]) or PER_GROUP (kdim 1: scale[row][col / g]; kdim 0: scale[row / g][col])
    on src [rows, n] int32 / f32 (or int8); scale f32 / f16 / bf16."""
    m, n = src.shape
    src_type = {torch.int32: INT32, torch.float32: F32, torch.int8: INT8}[src.dtype]
    scale_type = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[scale.dtype]
    y = out if out is not None else torch.empty((m, n), dtype=dst_dtype, device=src.device)
    p = _DequantPolicyParam(m, n, m * n if cal_count is None else cal_count, group_size, int(offset is not None), kdim)
    check(lib().ascq_ascend_dequant_policy(_ptr(y), _dtype_code(dst_dtype), _ptr(src), src_type, _ptr(scale),
                                           _ptr(offset), scale_type, policy, ctypes.byref(p), _stream(stream)),
          "ascend_dequant_policy")
    return y


def ascend_antiquant(src: torch.Tensor, src_type: int, scale: torch.Tensor, offset, k: int, n: int,
                     group_size: int = 0, is_transpose: bool = False, dst_dtype=torch.float16,
                     arith: int = ARITH_F16, out=None, stream=None):
    """AscendAntiQuant: dst = (src + offset) * scale.  Returns [K, N] (or [N, K] when is_transpose)."""
    dst_type = {torch.float16: F16, torch.bfloat16: BF16}[dst_dtype]
    shape = (n, k) if is_transpose else (k, n)
    y = out if out is not None else torch.empty(shape, dtype=dst_dtype, device=src.device)
    check(lib().ascq_ascend_antiquant(_ptr(y), dst_type, _ptr(src), src_type, _ptr(offset), _ptr(scale), k, n,
                                      group_size, int(is_transpose), arith, _stream(stream)), "ascend_antiquant")
    return y


def ascend_antiquant_scalar(src: torch.Tensor, src_type: int, offset: float | None, scale: float, count: int,
                            dst_dtype=torch.float16, out=None, stream=None):
    """AscendAntiQuant per tensor: dst[i] = (src[i] + offset) * scale with offset / scale of dst_dtype (offset None:
    scale only); count elements (int4 two per byte)."""
    dst_type = {torch.float16: F16, torch.bfloat16: BF16}[dst_dtype]
    bits = lambda v: int(torch.tensor([v], dtype=dst_dtype).view(torch.int16).item()) & 0xFFFF
    y = out if out is not None else torch.empty(count, dtype=dst_dtype, device=src.device)
    check(lib().ascq_ascend_antiquant_scalar(_ptr(y), dst_type, _ptr(src), src_type, bits(offset or 0.0), bits(scale),
                                             int(offset is not None), count, _stream(stream)), "ascend_antiquant_scalar")
    return y


def ascend_antiquant_policy(src: torch.Tensor, src_type: int, scale: torch.Tensor, scale_type: int, policy: int,
                            m: int, n: int, group_size: int = 0, offset=None, k_dim: int = 0,
                            is_transpose: bool = False, dst_dtype=torch.float16, out=None, stream=None):
    """AscendAntiQuant policy form (PER_TOKEN / PER_GROUP) over [m, n]: int8 / fp8 sources with f16 / bf16 / f32
    scales, fp4 E2M1 / E1M2 sources with E8M0 group scales.  Returns [m, n] of dst_dtype."""
    dst_type = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}[dst_dtype]
    y = out if out is not None else torch.empty((m, n), dtype=dst_dtype, device=src.device)
    check(lib().ascq_ascend_antiquant_policy(_ptr(y), dst_type, _ptr(src), src_type, _ptr(scale), _ptr(offset),
                                             scale_type, policy, m, n, group_size, k_dim, int(is_transpose),
                                             _stream(stream)), "ascend_antiquant_policy")
    return y


# ------------------------------------------------------------------------------------------
# Quantize / Dequantize / AntiQuantize (quantize.h / dequantize.h / antiquantize.h)
# ------------------------------------------------------------------------------------------
_FLOAT_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}


def quantize(x: torch.Tensor, policy: int, dst_type: int = INT8, scale=None, offset=None, scale_scalar: float = 1.0,
             offset_scalar=None, scale_type: int | None = None, group_size: int = 0, kdim: int = 1,
             round_mode: int = ROUND_RINT, out=None, stream=None):
    """Quantize<{policy, hasOffset, roundMode, kDim}>(dst, x, scale, offset, {m, n, groupSize}) of x [m, n] in fp32
    arithmetic.  PER_TENSOR: scale_scalar / offset_scalar (values of scale_type); the other policies: `scale` (and
    `offset`, or offset_scalar) tensors.  Returns int8 (INT8) or uint8 codes [m, n] ([m, n / 2] for fp4)."""
    m, n = x.shape
    if scale_type is None:
        scale_type = _FLOAT_CODE[scale.dtype] if scale is not None else F32
    if out is not None:
        q = out
    elif dst_type in (FP4_E2M1, FP4_E1M2):
        q = torch.empty((m, n // 2), dtype=torch.uint8, device=x.device)
    else:
        q = torch.empty((m, n), dtype=torch.int8 if dst_type == INT8 else torch.uint8, device=x.device)
    has_off = offset is not None or offset_scalar is not None
    p = _QuantizeParam(policy, int(has_off), round_mode, kdim, m, n, group_size)
    check(lib().ascq_quantize(_ptr(q), dst_type, _ptr(x), _FLOAT_CODE[x.dtype], _ptr(scale), _ptr(offset),
                              float(scale_scalar), float(offset_scalar or 0.0), scale_type, ctypes.byref(p),
                              _stream(stream)), "quantize")
    return q


def dequantize(src: torch.Tensor, policy: int, dst_dtype=torch.float32, scale=None, scale_scalar: float = 1.0,
               scale_type: int | None = None, group_size: int = 0, kdim: int = 1, out=None, stream=None):
    """Dequantize<{policy, false, kDim}>(dst, src, scale, {m, n, groupSize}): dst = cast(f32(src) * scale) over src
    [m, n] int32 (PER_TOKEN / PER_GROUP: int32 or f32).  PER_TENSOR: scale_scalar; PER_CHANNEL: scale [n] (f32, bf16,
    or int64 holding uint64 words)."""
    m, n = src.shape
    src_type = {torch.int32: INT32, torch.float32: F32}[src.dtype]
    if scale_type is None:
        scale_type = F32 if scale is None else {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
                                                torch.int64: U64}[scale.dtype]
    y = out if out is not None else torch.empty((m, n), dtype=dst_dtype, device=src.device)
    p = _QuantizeParam(policy, 0, ROUND_RINT, kdim, m, n, group_size)
    check(lib().ascq_dequantize(_ptr(y), _FLOAT_CODE[dst_dtype], _ptr(src), src_type, _ptr(scale), float(scale_scalar),
                                scale_type, ctypes.byref(p), _stream(stream)), "dequantize")
    return y


def antiquantize(src: torch.Tensor, src_type: int, policy: int, m: int, n: int, dst_dtype=torch.float16, scale=None,
                 offset=None, scale_scalar: float = 1.0, offset_scalar=None, scale_type: int | None = None,
                 group_size: int = 0, kdim: int = 1, out=None, stream=None):
    """AntiQuantize<{policy, hasOffset, kDim}>(dst, src, scale, offset, {m, n, groupSize}): dst = (src + offset) *
    scale in fp32, one cast, over [m, n] (int8 / hifloat8 / fp8 codes; fp4 [m, n / 2] bytes with E8M0 scales).
    PER_TENSOR: scale_scalar / offset_scalar (values of dst_dtype); the other policies: `scale` / `offset` tensors."""
    if scale_type is None:
        scale_type = _FLOAT_CODE[dst_dtype] if scale is None else {torch.float32: F32, torch.float16: F16,
                                                                   torch.bfloat16: BF16, torch.uint8: E8M0}[scale.dtype]
    y = out if out is not None else torch.empty((m, n), dtype=dst_dtype, device=src.device)
    has_off = offset is not None or offset_scalar is not None
    p = _QuantizeParam(policy, int(has_off), ROUND_RINT, kdim, m, n, group_size)
    check(lib().ascq_antiquantize(_ptr(y), _FLOAT_CODE[dst_dtype], _ptr(src), src_type, _ptr(scale), _ptr(offset),
                                  float(scale_scalar), float(offset_scalar or 0.0), scale_type, ctypes.byref(p),
                                  _stream(stream)), "antiquantize")
    return y


# ------------------------------------------------------------------------------------------
# weight-only antiquant matmul
# ------------------------------------------------------------------------------------------
def weight_pack_size(w_type: int, k: int, n: int) -> int:
    sz = ctypes.c_size_t(0)
    check(lib().ascq_weight_pack_size(w_type, k, n, ctypes.byref(sz)), "weight_pack_size")
    return sz.value


def weight_pack(w: torch.Tensor, w_type: int, k: int, n: int, is_transpose: bool = False, out=None, stream=None):
    nbytes = weight_pack_size(w_type, k, n)
    wp = out if out is not None else torch.empty((nbytes,), dtype=torch.uint8, device=w.device)
    check(lib().ascq_weight_pack(_ptr(wp), _ptr(w), w_type, k, n, int(is_transpose), _stream(stream)), "weight_pack")
    return wp


def antiquant_matmul(x: torch.Tensor, w_packed: torch.Tensor, w_type: int, scale: torch.Tensor, offset, group_size: int,
                     n: int, out=None, stream=None):
    m, k = x.shape
    y = out if out is not None else torch.empty((m, n), dtype=torch.float16, device=x.device)
    check(lib().ascq_antiquant_matmul(_ptr(y), _ptr(x), _ptr(w_packed), w_type, _ptr(scale), _ptr(offset), group_size,
                                      m, n, k, _stream(stream)), "antiquant_matmul")
    return y


# ------------------------------------------------------------------------------------------
# quantized group matmul (MoE)
# ------------------------------------------------------------------------------------------
def quant_group_matmul(x: torch.Tensor, per_token_scale: torch.Tensor, w: torch.Tensor, scale: torch.Tensor,
                       group_list: torch.Tensor, list_type: int = 0, w_trans: bool = False,
                       out_dtype=torch.bfloat16, out=None, stream=None, activation: int = 0):
    """activation: ACT_NONE or ACT_FASTER_GELU (the reference sample's epilogue)"""
    m, k = x.shape
    g = scale.shape[0]
    n = scale.shape[1]
    out_type = {torch.bfloat16: BF16, torch.float16: F16}[out_dtype]
    y = out if out is not None else torch.empty((m, n), dtype=out_dtype, device=x.device)
    check(lib().ascq_quant_group_matmul(_ptr(y), out_type, _ptr(x), _ptr(per_token_scale), _ptr(w), int(w_trans),
                                        _ptr(scale), _ptr(group_list), list_type, g, m, k, n, int(activation),
                                        _stream(stream)),
          "quant_group_matmul")
    return y


# ------------------------------------------------------------------------------------------
# NZ fractal <-> ND
# ------------------------------------------------------------------------------------------
def nz_size(dtype: int, batch: int, rows: int, cols: int) -> int:
    return int(lib().ascq_nz_size(dtype, batch, rows, cols))


def nz_to_nd(src: torch.Tensor, dtype: int, batch: int, rows: int, cols: int, transpose_out: bool = False, out=None,
             stream=None):
    """NZ bytes -> ND [batch, rows, cols] (transpose_out: [batch, cols, rows]) as a uint8 tensor of that shape
    times the element size"""
    esize = {INT8: 1, UINT8: 1, FP8_E4M3: 1, FP8_E5M2: 1, F16: 2, BF16: 2, INT32: 4, F32: 4}[dtype]
    shape = (batch, cols, rows * esize) if transpose_out else (batch, rows, cols * esize)
    y = out if out is not None else torch.empty(shape, dtype=torch.uint8, device=src.device)
    check(lib().ascq_nz_to_nd(_ptr(y), _ptr(src), dtype, batch, rows, cols, int(transpose_out), _stream(stream)),
          "nz_to_nd")
    return y


def nd_to_nz(src: torch.Tensor, dtype: int, batch: int, rows: int, cols: int, out=None, stream=None):
    y = out if out is not None else torch.empty(nz_size(dtype, batch, rows, cols), dtype=torch.uint8, device=src.device)
    check(lib().ascq_nd_to_nz(_ptr(y), _ptr(src), dtype, batch, rows, cols, _stream(stream)), "nd_to_nz")
    return y


# ------------------------------------------------------------------------------------------
# Matmul handle (mirrors AscendC::Matmul's call sequence)
# ------------------------------------------------------------------------------------------
class Matmul:
    """Matmul<A, B, C, Bias> handle: SetOrgShape / SetTensorA / SetTensorB / SetBias / SetQuant* /
    SetAntiQuant* / SetTensorScaleA/B / IterateAll / End, each a call into the C ABI."""

    def __init__(self, a_type: int, b_type: int, c_type: int, bias_type: int = 0, scale_type: int = 0,
                 b_format: int = FORMAT_ND):
        self._h = ctypes.c_void_p()
        t = _MatmulTypes(a_type, b_type, c_type, bias_type, scale_type, b_format)
        check(lib().ascq_matmul_create(ctypes.byref(t), ctypes.byref(self._h)), "matmul_create")
        self._keep = []

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value and _lib is not None:
            _lib.ascq_matmul_destroy(h)
            self._h = None

    def Init(self, tiling: CubeTiling):
        check(lib().ascq_matmul_init(self._h, ctypes.byref(tiling)), "Init")

    def SetOrgShape(self, m: int, n: int, k: int):
        check(lib().ascq_matmul_set_org_shape(self._h, m, n, k), "SetOrgShape")

    def SetSingleShape(self, m: int, n: int, k: int):
        check(lib().ascq_matmul_set_single_shape(self._h, m, n, k), "SetSingleShape")

    def SetTail(self, m: int = -1, n: int = -1, k: int = -1):
        check(lib().ascq_matmul_set_tail(self._h, m, n, k), "SetTail")

    def SetTensorA(self, a, is_transpose_a: bool = False):
        self._keep.append(a)
        check(lib().ascq_matmul_set_tensor_a(self._h, _ptr(a), int(is_transpose_a)), "SetTensorA")

    def SetTensorB(self, b, is_transpose_b: bool = False):
        self._keep.append(b)
        check(lib().ascq_matmul_set_tensor_b(self._h, _ptr(b), int(is_transpose_b)), "SetTensorB")

    def SetBias(self, bias):
        self._keep.append(bias)
        check(lib().ascq_matmul_set_bias(self._h, _ptr(bias)), "SetBias")

    def DisableBias(self):
        check(lib().ascq_matmul_disable_bias(self._h), "DisableBias")

    def SetQuantScalar(self, word: int):
        check(lib().ascq_matmul_set_quant_scalar(self._h, word & 0xFFFFFFFFFFFFFFFF), "SetQuantScalar")

    def SetQuantVector(self, words: torch.Tensor):
        self._keep.append(words)
        check(lib().ascq_matmul_set_quant_vector(self._h, _ptr(words)), "SetQuantVector")

    def SetAntiQuantScalar(self, offset: float, scale: float):
        check(lib().ascq_matmul_set_antiquant_scalar(self._h, _half_bits(offset), _half_bits(scale)),
              "SetAntiQuantScalar")

    def SetAntiQuantVector(self, offset, scale, group_size: int = 0):
        self._keep += [offset, scale]
        check(lib().ascq_matmul_set_antiquant_vector(self._h, _ptr(offset), _ptr(scale), group_size),
              "SetAntiQuantVector")

    def SetTensorScaleA(self, s, is_transpose_scale_a: bool = False):
        self._keep.append(s)
        check(lib().ascq_matmul_set_tensor_scale_a(self._h, _ptr(s), int(is_transpose_scale_a)), "SetTensorScaleA")

    def SetTensorScaleB(self, s, is_transpose_scale_b: bool = True):
        self._keep.append(s)
        check(lib().ascq_matmul_set_tensor_scale_b(self._h, _ptr(s), int(is_transpose_scale_b)), "SetTensorScaleB")

    def WorkspaceSize(self) -> int:
        sz = ctypes.c_size_t(0)
        check(lib().ascq_matmul_workspace_size(self._h, ctypes.byref(sz)), "WorkspaceSize")
        return sz.value

    def SetWorkspace(self, ws, nbytes: int):
        self._keep.append(ws)
        check(lib().ascq_matmul_set_workspace(self._h, _ptr(ws), nbytes), "SetWorkspace")

    def IterateAll(self, c, en_atomic: int = 0, stream=None):
        check(lib().ascq_matmul_iterate_all(self._h, _ptr(c), en_atomic, _stream(stream)), "IterateAll")

    def IterateAllNoAlloc(self, c, en_atomic: int = 0, stream=None):
        """IterateAll with the workspace taken from the library's static per-device scratch (allocates nothing)"""
        check(lib().ascq_matmul_iterate_all_noalloc(self._h, _ptr(c), en_atomic, _stream(stream)), "IterateAllNoAlloc")

    def End(self):
        check(lib().ascq_matmul_end(self._h), "End")
        self._keep = []
