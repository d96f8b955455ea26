"""CPU tests of the C ABI: libascq.so loads, exports every function include/ascq.h declares, and rejects
invalid arguments on the host (negative status, nothing launched) -- no GPU needed for any of these."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import tempfile
from pathlib import Path

import pytest
import torch

import ascq

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ascq.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(ascq_[a-z0-9_]+)\s*\(", text))


def test_library_loads():
    L = ascq.lib()
    assert L.ascq_version().decode().startswith("ascq")


def test_exports_every_declared_symbol():
    declared = declared_functions()
    assert len(declared) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", str(ascq.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = declared - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    # and the binding's signature table covers exactly the declared set
    assert set(ascq.SIGNATURES) == declared


def test_pack_quant_pre_matches_reference_packing():
    # (uint64)(*(uint32*)&f) for f = 0.1 (matmul_quant.asc:111-113)
    f = ctypes.c_float(0.1)
    bits = ctypes.cast(ctypes.pointer(f), ctypes.POINTER(ctypes.c_uint32)).contents.value
    assert ascq.pack_quant_pre(0.1) == bits
    w = ascq.pack_quant_pre(1.0, offset9=-3, sign=1)
    assert w & 0xFFFFFFFF == 0x3F800000
    assert (w >> 37) & 0x1FF == (-3) & 0x1FF
    assert (w >> 46) & 1 == 1


def _err(status, expect):
    assert status == expect, f"status {status}: {ascq.last_error()}"


def test_quant_argument_checks():
    L = ascq.lib()
    P = ascq._QuantParam(0, 7, 15, 0, 0, 1, ascq.ROUND_RINT)  # calCount not a multiple of n
    dummy = ctypes.c_void_p(0x1000)
    _err(L.ascq_ascend_quant_per_token(dummy, dummy, ascq.F16, dummy, None, ctypes.byref(P), None),
         ascq.E_INVALID_ARG)
    assert "multiple of n" in ascq.last_error()
    P = ascq._QuantParam(0, 8, 16, 0, 0, 1, 17)  # bad round mode
    _err(L.ascq_ascend_quant_per_token(dummy, dummy, ascq.F16, dummy, None, ctypes.byref(P), None),
         ascq.E_INVALID_ARG)
    P = ascq._QuantParam(0, 8, 16, 0, 1, 1, 1)  # has_offset without an offset tensor
    _err(L.ascq_ascend_quant_per_token(dummy, dummy, ascq.F16, dummy, None, ctypes.byref(P), None),
         ascq.E_INVALID_ARG)
    _err(L.ascq_ascend_quant_per_token(None, dummy, ascq.F16, dummy, None, ctypes.byref(P), None),
         ascq.E_INVALID_ARG)
    _err(L.ascq_ascend_quant_dynamic_per_token(dummy, dummy, dummy, ascq.INT32, 4, 4, 1, None), ascq.E_UNSUPPORTED)
    aq = lambda dst, src, sc, of, cal, cnt: L.ascq_ascend_quant(dummy, dst, dummy, src, sc, of, 1.0, 0.0, cal, cnt, None)
    _err(aq(ascq.INT8, ascq.F16, dummy, None, 96, 5), ascq.E_INVALID_ARG)        # calCount % scaleCount
    _err(aq(ascq.INT8, ascq.F16, dummy, None, 100, 4), ascq.E_INVALID_ARG)       # calCount % 32 (per channel)
    _err(aq(ascq.INT8, ascq.F16, None, dummy, 96, 4), ascq.E_INVALID_ARG)        # offset tensor without scales
    _err(aq(ascq.FP4_E2M1, ascq.F16, None, None, 96, 0), ascq.E_UNSUPPORTED)     # int8 / hif8 / fp8 outputs only
    _err(aq(ascq.INT8, ascq.INT8, None, None, 96, 0), ascq.E_UNSUPPORTED)        # float sources only
    _err(aq(ascq.HIF8, ascq.BF16, None, None, 0, 0), ascq.OK)                    # calCount 0: nothing to do
    _err(L.ascq_ascend_antiquant_scalar(dummy, ascq.F32, dummy, ascq.INT8, 0, 0, 1, 8, None), ascq.E_UNSUPPORTED)
    _err(L.ascq_ascend_antiquant_scalar(dummy, ascq.F16, dummy, ascq.INT4, 0, 0, 1, 7, None), ascq.E_INVALID_ARG)
    _err(L.ascq_ascend_antiquant(dummy, ascq.F16, dummy, ascq.HIF8, dummy, dummy, 64, 32, 32, 0, 0, None),
         ascq.E_UNSUPPORTED)                                                      # hif8 / fp8: per channel only
    # zero-sized work is a no-op that succeeds without touching the device
    _err(L.ascq_ascend_quant_dynamic_per_token(dummy, dummy, dummy, ascq.F16, 0, 16, 1, None), ascq.OK)


def test_policy_form_argument_checks():
    """AscendQuant / AscendAntiQuant policy forms reject what the reference's static_asserts and checks reject,
    before any device work (ascend_quant_per_group_3510_impl.h:1465-1498; ascend_antiquant_3510_impl.h:2175-2221)"""
    L = ascq.lib()
    d = ctypes.c_void_p(0x1000)
    P = ascq._QuantParam(4, 64, 256, 32, 0, 1, ascq.ROUND_RINT)
    qp = lambda dst, src, sc, pol, p=P: L.ascq_ascend_quant_policy(d, dst, d, src, d, None, 0.0, sc, pol, ctypes.byref(p), None)
    _err(qp(ascq.FP4_E2M1, ascq.F16, ascq.F16, ascq.PER_TOKEN), ascq.E_UNSUPPORTED)      # PER_TOKEN: int8 / fp8 only
    _err(qp(ascq.INT4, ascq.F16, ascq.F16, ascq.PER_GROUP), ascq.E_UNSUPPORTED)          # no int4 / hifloat8 output
    _err(qp(ascq.INT8, ascq.F32, ascq.F16, ascq.PER_GROUP), ascq.E_UNSUPPORTED)          # 16-bit scale, f32 source
    _err(qp(ascq.INT8, ascq.F16, ascq.F16, ascq.PER_CHANNEL), ascq.E_UNSUPPORTED)        # policy
    _err(qp(ascq.INT8, ascq.INT8, ascq.F16, ascq.PER_GROUP), ascq.E_UNSUPPORTED)         # source type
    for bad in (ascq._QuantParam(4, 64, 256, 48, 0, 1, 1),   # group not a multiple of 32
                ascq._QuantParam(4, 64, 256, 32, 0, 2, 1),   # kDim
                ascq._QuantParam(4, 64, 250, 32, 0, 1, 1),   # calCount not a multiple of n
                ascq._QuantParam(4, 64, 256, 32, 0, 1, 9)):  # round mode
        _err(qp(ascq.INT8, ascq.F16, ascq.F16, ascq.PER_GROUP, bad), ascq.E_INVALID_ARG)
    _err(qp(ascq.FP4_E2M1, ascq.F16, ascq.F16, ascq.PER_GROUP, ascq._QuantParam(4, 63, 252, 32, 0, 1, 1)),
         ascq.E_INVALID_ARG)  # E2M1 rows pack two a byte
    # calCount 0 is a no-op that succeeds without touching the device, even with null pointers
    z = ascq._QuantParam(0, 64, 0, 32, 0, 1, 1)
    _err(L.ascq_ascend_quant_policy(None, ascq.INT8, None, ascq.F16, None, None, 0.0, ascq.F16, ascq.PER_GROUP,
                                    ctypes.byref(z), None), ascq.OK)
    aq = lambda src, sc, dst, pol, g=32, off=None: L.ascq_ascend_antiquant_policy(d, dst, d, src, d, off, sc, pol, 4, 64,
                                                                                  g, 1, 0, None)
    _err(aq(ascq.FP4_E2M1, ascq.F16, ascq.BF16, ascq.PER_GROUP), ascq.E_UNSUPPORTED)    # fp4 needs E8M0 scales
    _err(aq(ascq.FP4_E2M1, ascq.E8M0, ascq.BF16, ascq.PER_GROUP, off=d), ascq.E_UNSUPPORTED)  # and no offset
    _err(aq(ascq.INT8, ascq.F16, ascq.BF16, ascq.PER_GROUP), ascq.E_UNSUPPORTED)        # half scale writes half
    _err(aq(ascq.INT4, ascq.F16, ascq.F16, ascq.PER_GROUP), ascq.E_UNSUPPORTED)         # no int4 in the policy form
    _err(aq(ascq.INT8, ascq.F16, ascq.F16, ascq.PER_GROUP, g=16), ascq.E_INVALID_ARG)   # group % 32
    _err(L.ascq_ascend_antiquant_policy(None, ascq.F16, None, ascq.INT8, None, None, ascq.F16, ascq.PER_GROUP, 0, 64,
                                        32, 1, 0, None), ascq.OK)                        # m = 0: no-op


def test_dequant_antiquant_argument_checks():
    L = ascq.lib()
    d = ctypes.c_void_p(0x1000)
    dq = lambda dst, sc, pol, p, mode=0, scale=d: L.ascq_ascend_dequant(d, dst, d, ascq.INT32, scale, sc, 1.0, pol,
                                                                        mode, ctypes.byref(p), None)
    p = ascq._DequantParam(4, 8, 9)  # calCount > n
    _err(dq(ascq.F32, ascq.F32, ascq.PER_CHANNEL, p), ascq.E_INVALID_ARG)
    _err(dq(ascq.F32, ascq.F32, ascq.PER_CHANNEL, ascq._DequantParam(4, 12, 8)), ascq.E_INVALID_ARG)  # n % 8
    _err(dq(ascq.F32, ascq.F32, ascq.PER_CHANNEL, ascq._DequantParam(4, 8, 0)), ascq.E_INVALID_ARG)   # calCount 0
    p = ascq._DequantParam(4, 8, 8)
    _err(dq(ascq.INT8, ascq.F32, ascq.PER_CHANNEL, p), ascq.E_UNSUPPORTED)
    _err(dq(ascq.F32, ascq.F32, ascq.PER_CHANNEL, p, mode=2), ascq.E_INVALID_ARG)
    _err(dq(ascq.F32, ascq.F32, ascq.PER_TOKEN, p), ascq.E_UNSUPPORTED)          # the policy form's entry point
    _err(dq(ascq.F32, ascq.F32, ascq.PER_CHANNEL, p, scale=None), ascq.E_INVALID_ARG)
    # IsTemplateValid: tensor (U64, F16) (F32, F32) (BF16, F32) (BF16, BF16) (F32, BF16); scalar without U64 / F16
    for sc, dst, ok in [(ascq.U64, ascq.F16, True), (ascq.F32, ascq.F16, False), (ascq.F16, ascq.F16, False),
                        (ascq.BF16, ascq.BF16, True), (ascq.U64, ascq.F32, False), (ascq.F32, ascq.BF16, True)]:
        _err(dq(dst, sc, ascq.PER_CHANNEL, ascq._DequantParam(0, 8, 8)), ascq.OK if ok else ascq.E_UNSUPPORTED)
    for sc, dst, ok in [(ascq.BF16, ascq.F32, True), (ascq.F32, ascq.F16, False), (ascq.U64, ascq.F16, False)]:
        _err(dq(dst, sc, ascq.PER_TENSOR, ascq._DequantParam(0, 8, 8)), ascq.OK if ok else ascq.E_UNSUPPORTED)
    rows, ldd = ascq.dequant_dst_shape(torch.float32, 1, 16, 8)
    assert (rows, ldd) == (2, 8)
    assert ascq.dequant_dst_shape(torch.bfloat16, 1, 16, 8) == (1, 16)
    assert ascq.dequant_dst_shape(torch.float16, 3, 24, 24) == (3, 32)
    assert ascq.dequant_dst_shape(torch.float32, 1, 16, 8, ascq.DEQUANT_MULTI_ROW) == (1, 16)
    pp = lambda g=32, k=1: ascq._DequantPolicyParam(4, 64, 256, g, 0, k)
    dqp = lambda src, sc, dst, pol, p: L.ascq_ascend_dequant_policy(d, dst, d, src, d, None, sc, pol, ctypes.byref(p),
                                                                    None)
    _err(dqp(ascq.INT32, ascq.F32, ascq.F16, ascq.PER_GROUP, pp(g=16)), ascq.E_INVALID_ARG)      # group % 32
    _err(dqp(ascq.INT32, ascq.F32, ascq.F16, ascq.PER_GROUP, pp(k=2)), ascq.E_INVALID_ARG)       # kDim 0 / 1
    _err(dqp(ascq.F16, ascq.F32, ascq.F16, ascq.PER_TOKEN, pp()), ascq.E_UNSUPPORTED)            # src int32 / f32
    _err(dqp(ascq.INT32, ascq.U64, ascq.F16, ascq.PER_TOKEN, pp()), ascq.E_UNSUPPORTED)          # scale 16/32-bit fp
    _err(dqp(ascq.INT32, ascq.F32, ascq.F16, ascq.PER_CHANNEL, pp()), ascq.E_UNSUPPORTED)
    _err(L.ascq_ascend_dequant_policy(None, ascq.F16, None, ascq.INT32, None, None, ascq.F32, ascq.PER_TOKEN,
                                      ctypes.byref(ascq._DequantPolicyParam(4, 64, 63, 0, 0, 1)), None), ascq.OK)
    _err(L.ascq_ascend_antiquant(d, ascq.F16, d, ascq.INT8, d, d, 100, 8, 32, 0, 0, None), ascq.E_INVALID_ARG)
    _err(L.ascq_ascend_antiquant(d, ascq.F32, d, ascq.INT8, d, d, 128, 8, 32, 0, 0, None), ascq.E_UNSUPPORTED)


def test_quantize_interface_argument_checks():
    """Quantize / Dequantize / AntiQuantize reject what the reference's static_asserts and asserts reject, before any
    device work (quantize_impl.h:33-61, 1006-1066; dequantize_impl.h:67-195; antiquantize_impl.h:46-226)"""
    L = ascq.lib()
    d = ctypes.c_void_p(0x1000)
    P = lambda pol, off=0, k=1, m=4, n=64, g=32, rm=ascq.ROUND_RINT: ascq._QuantizeParam(pol, off, rm, k, m, n, g)
    q = lambda dst, src, sc, p, scale=d, off=None: L.ascq_quantize(d, dst, d, src, scale, off, 1.0, 0.0, sc,
                                                                  ctypes.byref(p), None)
    _err(q(ascq.INT8, ascq.F32, ascq.F16, P(ascq.PER_TOKEN)), ascq.E_UNSUPPORTED)            # (f32, f16) pair
    _err(q(ascq.INT8, ascq.F16, ascq.BF16, P(ascq.PER_TOKEN)), ascq.E_UNSUPPORTED)           # (f16, bf16) pair
    _err(q(ascq.FP4_E2M1, ascq.F16, ascq.F16, P(ascq.PER_TOKEN)), ascq.E_UNSUPPORTED)        # fp4: PER_GROUP only
    _err(q(ascq.INT4, ascq.F16, ascq.F16, P(ascq.PER_GROUP)), ascq.E_UNSUPPORTED)            # no int4 output
    _err(q(ascq.INT8, ascq.F16, ascq.F16, P(ascq.PER_TOKEN, n=48)), ascq.E_INVALID_ARG)      # n % 32
    _err(q(ascq.INT8, ascq.F16, ascq.F16, P(ascq.PER_GROUP, g=48)), ascq.E_INVALID_ARG)      # group % 32
    _err(q(ascq.INT8, ascq.F16, ascq.F16, P(ascq.PER_GROUP, k=2)), ascq.E_INVALID_ARG)       # kDim
    _err(q(ascq.INT8, ascq.F16, ascq.F16, P(ascq.PER_TENSOR)), ascq.E_INVALID_ARG)           # PER_TENSOR: scalars
    _err(q(ascq.INT8, ascq.F16, ascq.F16, P(ascq.PER_TOKEN, rm=9)), ascq.E_INVALID_ARG)      # round mode
    _err(q(ascq.INT8, ascq.F16, ascq.F16, P(7)), ascq.E_INVALID_ARG)                         # policy
    _err(L.ascq_quantize(None, ascq.INT8, None, ascq.F16, None, None, 1.0, 0.0, ascq.F16,
                         ctypes.byref(P(ascq.PER_TOKEN, m=0)), None), ascq.OK)                # m = 0: no-op
    dq = lambda dst, src, sc, p: L.ascq_dequantize(d, dst, d, src, d, 1.0, sc, ctypes.byref(p), None)
    _err(dq(ascq.F32, ascq.INT32, ascq.F32, P(ascq.PER_CHANNEL, off=1)), ascq.E_UNSUPPORTED)  # no offset
    _err(dq(ascq.F16, ascq.INT32, ascq.F32, P(ascq.PER_CHANNEL)), ascq.E_UNSUPPORTED)         # (f32, f16) channel
    _err(dq(ascq.F16, ascq.INT32, ascq.F16, P(ascq.PER_TENSOR)), ascq.E_UNSUPPORTED)          # half scalar
    _err(dq(ascq.F32, ascq.F32, ascq.F32, P(ascq.PER_CHANNEL)), ascq.E_UNSUPPORTED)           # channel: int32 src
    _err(dq(ascq.F16, ascq.INT32, ascq.F16, P(ascq.PER_TOKEN, n=8)), ascq.E_INVALID_ARG)      # 16-byte f16 rows
    _err(dq(ascq.F16, ascq.INT32, ascq.BF16, P(ascq.PER_TOKEN)), ascq.E_UNSUPPORTED)          # (bf16, f16) pair
    _err(L.ascq_dequantize(None, ascq.F32, None, ascq.INT32, None, 1.0, ascq.F32,
                           ctypes.byref(P(ascq.PER_CHANNEL, m=0)), None), ascq.OK)
    aq = lambda dst, src, sc, p, scale=d, off=None: L.ascq_antiquantize(d, dst, d, src, scale, off, 1.0, 0.0, sc,
                                                                        ctypes.byref(p), None)
    _err(aq(ascq.F32, ascq.INT8, ascq.F32, P(ascq.PER_CHANNEL)), ascq.E_UNSUPPORTED)  # channel: f16 / bf16 scales
    _err(aq(ascq.F16, ascq.INT8, ascq.BF16, P(ascq.PER_CHANNEL)), ascq.E_UNSUPPORTED)  # of the dst type
    _err(aq(ascq.F16, ascq.INT4, ascq.F16, P(ascq.PER_TOKEN)), ascq.E_UNSUPPORTED)     # no int4
    _err(aq(ascq.BF16, ascq.INT8, ascq.F16, P(ascq.PER_GROUP)), ascq.E_UNSUPPORTED)    # (f16, bf16) pair
    _err(aq(ascq.BF16, ascq.FP4_E2M1, ascq.E8M0, P(ascq.PER_GROUP, off=1), off=d), ascq.E_UNSUPPORTED)  # fp4 offset
    _err(aq(ascq.BF16, ascq.FP4_E2M1, ascq.E8M0, P(ascq.PER_TOKEN)), ascq.E_UNSUPPORTED)  # fp4: PER_GROUP
    _err(aq(ascq.BF16, ascq.FP4_E2M1, ascq.E8M0, P(ascq.PER_GROUP, n=32)), ascq.E_INVALID_ARG)  # fp4 n % 64
    _err(aq(ascq.F16, ascq.INT8, ascq.F16, P(ascq.PER_TOKEN, off=1)), ascq.E_INVALID_ARG)  # has_offset, no tensor
    _err(aq(ascq.F16, ascq.INT8, ascq.F16, P(ascq.PER_TENSOR)), ascq.E_INVALID_ARG)        # PER_TENSOR: scalars
    _err(aq(ascq.F16, ascq.INT8, ascq.F16, P(ascq.PER_TOKEN, n=40)), ascq.E_INVALID_ARG)   # 32-byte rows
    _err(L.ascq_antiquantize(None, ascq.F16, None, ascq.INT8, None, None, 1.0, 0.0, ascq.F16,
                             ctypes.byref(P(ascq.PER_TENSOR, m=0)), None), ascq.OK)


def test_gemv_group_argument_checks():
    L = ascq.lib()
    d = ctypes.c_void_p(0x1000)
    sz = ctypes.c_size_t(0)
    _err(L.ascq_weight_pack_size(ascq.INT4, 4096, 11008, ctypes.byref(sz)), ascq.OK)
    assert sz.value == 4096 * 11008 // 2
    _err(L.ascq_weight_pack_size(ascq.INT8, 100, 16, ctypes.byref(sz)), ascq.E_INVALID_ARG)
    _err(L.ascq_antiquant_matmul(d, d, d, ascq.INT4, d, d, 48, 1, 64, 256, None), ascq.E_INVALID_ARG)  # g % 32
    _err(L.ascq_antiquant_matmul(d, d, d, ascq.INT4, d, d, 96, 1, 64, 256, None), ascq.E_INVALID_ARG)  # g !| K
    _err(L.ascq_antiquant_matmul(d, ctypes.c_void_p(0x1001), d, ascq.INT4, d, d, 128, 1, 64, 256, None),
         ascq.E_INVALID_ARG)  # misaligned x
    _err(L.ascq_quant_group_matmul(d, ascq.F32, d, d, d, 0, d, d, 0, 4, 8, 16, 16, 0, None), ascq.E_UNSUPPORTED)
    _err(L.ascq_quant_group_matmul(d, ascq.BF16, d, d, d, 0, d, d, 2, 4, 8, 16, 16, 0, None), ascq.E_INVALID_ARG)
    _err(L.ascq_quant_group_matmul(d, ascq.BF16, d, d, d, 0, d, d, 0, 4, 8, 16, 16, 7, None), ascq.E_INVALID_ARG)


def test_matmul_handle_state_machine():
    L = ascq.lib()
    h = ctypes.c_void_p()
    bad = ascq._MatmulTypes(ascq.F16, ascq.F16, ascq.F16, 0, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(bad), ctypes.byref(h)), ascq.E_UNSUPPORTED)
    t = ascq._MatmulTypes(ascq.INT8, ascq.INT8, ascq.F16, ascq.INT32, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)
    d = ctypes.c_void_p(0x1000)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_STATE)          # no tensors yet
    _err(L.ascq_matmul_set_tensor_a(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_tensor_b(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_STATE)          # no org shape
    _err(L.ascq_matmul_set_org_shape(h, 128, 256, 512), ascq.OK)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_STATE)          # f16 out without quant params
    _err(L.ascq_matmul_iterate_all(h, d, 4, None), ascq.E_INVALID_ARG)    # enAtomic > ATOMIC_MIN
    _err(L.ascq_matmul_set_antiquant_scalar(h, 0, 0), ascq.E_UNSUPPORTED)
    _err(L.ascq_matmul_set_tensor_scale_a(h, d, 0), ascq.E_UNSUPPORTED)
    _err(L.ascq_matmul_set_single_shape(h, 256, 256, 512), ascq.OK)
    _err(L.ascq_matmul_set_quant_scalar(h, 0x3F800000), ascq.OK)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_INVALID_ARG)   # single shape exceeds org shape
    _err(L.ascq_matmul_end(h), ascq.OK)
    _err(L.ascq_matmul_destroy(h), ascq.OK)
    mx = ascq._MatmulTypes(ascq.FP4_E2M1, ascq.FP4_E2M1, ascq.BF16, 0, ascq.E8M0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(mx), ctypes.byref(h)), ascq.OK)
    _err(L.ascq_matmul_set_org_shape(h, 128, 128, 96), ascq.OK)
    _err(L.ascq_matmul_set_tensor_a(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_tensor_b(h, d, 1), ascq.OK)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_STATE)          # no scales
    _err(L.ascq_matmul_set_tensor_scale_a(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_tensor_scale_b(h, d, 1), ascq.OK)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_UNSUPPORTED)    # K % 128
    _err(L.ascq_matmul_destroy(h), ascq.OK)


def test_mx_e1m2_and_bias_handle():
    """fp4x2_e1m2_t MX operands (either side, with E2M1 on the other) are accepted and need the fp6 planes of both
    operands in the workspace; the MX bias must be f32; an int8 C refuses enAtomic before any launch"""
    L = ascq.lib()
    h = ctypes.c_void_p()
    d = ctypes.c_void_p(0x1000)
    for fa, fb in ((ascq.FP4_E1M2, ascq.FP4_E1M2), (ascq.FP4_E1M2, ascq.FP4_E2M1), (ascq.FP4_E2M1, ascq.FP4_E1M2)):
        t = ascq._MatmulTypes(fa, fb, ascq.BF16, ascq.F32, ascq.E8M0, 0)
        _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)
        _err(L.ascq_matmul_set_org_shape(h, 256, 256, 256), ascq.OK)
        _err(L.ascq_matmul_set_tensor_b(h, d, 1), ascq.OK)
        ws = ctypes.c_size_t()
        _err(L.ascq_matmul_workspace_size(h, ctypes.byref(ws)), ascq.OK)
        scales = 2 * ((256 * 8 + 16 + 255) // 256 * 256)
        p_plane, q_plane = 256 * 128, (256 // 128) * (256 // 32) * 1024
        assert ws.value == scales + 2 * (p_plane + q_plane)
        _err(L.ascq_matmul_destroy(h), ascq.OK)
    for bt in (ascq.INT32, ascq.F16):
        t = ascq._MatmulTypes(ascq.FP4_E2M1, ascq.FP4_E1M2, ascq.F32, bt, ascq.E8M0, 0)
        _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.E_UNSUPPORTED)
    t = ascq._MatmulTypes(ascq.INT8, ascq.INT8, ascq.INT8, 0, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)
    _err(L.ascq_matmul_set_org_shape(h, 64, 64, 64), ascq.OK)
    _err(L.ascq_matmul_set_tensor_a(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_tensor_b(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_quant_scalar(h, 0x3F800000), ascq.OK)
    _err(L.ascq_matmul_iterate_all(h, d, ascq.ATOMIC_ADD, None), ascq.E_UNSUPPORTED)
    _err(L.ascq_matmul_destroy(h), ascq.OK)


def test_nz_b_format_handle():
    """B declared CubeFormat::NZ (ASCQ_FORMAT_NZ): accepted for int8 and fp8 B, whose workspace then holds the ND
    [N, K] copy of B (whatever the transpose flag, and in place of the [K, N] transpose); refused for int4, MX,
    hifloat8 and weight-only B, and an unknown format is refused everywhere"""
    L = ascq.lib()
    h = ctypes.c_void_p()
    d = ctypes.c_void_p(0x1000)
    ws = ctypes.c_size_t()
    for at, bt, ct in ((ascq.INT8, ascq.INT8, ascq.INT32), (ascq.FP8_E4M3, ascq.FP8_E5M2, ascq.F32)):
        t = ascq._MatmulTypes(at, bt, ct, 0, 0, ascq.FORMAT_NZ)
        _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)
        _err(L.ascq_matmul_set_org_shape(h, 2048, 1280, 512), ascq.OK)
        for tb in (0, 1):
            _err(L.ascq_matmul_set_tensor_b(h, d, tb), ascq.OK)
            _err(L.ascq_matmul_workspace_size(h, ctypes.byref(ws)), ascq.OK)
            assert ws.value == 1280 * 512
        _err(L.ascq_matmul_destroy(h), ascq.OK)
    refused = [ascq._MatmulTypes(ascq.INT4, ascq.INT4, ascq.INT32, 0, 0, ascq.FORMAT_NZ),
               ascq._MatmulTypes(ascq.FP4_E2M1, ascq.FP4_E2M1, ascq.BF16, 0, ascq.E8M0, ascq.FORMAT_NZ),
               ascq._MatmulTypes(ascq.HIF8, ascq.HIF8, ascq.F32, 0, 0, ascq.FORMAT_NZ),
               ascq._MatmulTypes(ascq.F16, ascq.INT8, ascq.F16, 0, 0, ascq.FORMAT_NZ),
               ascq._MatmulTypes(ascq.INT8, ascq.INT8, ascq.INT32, 0, 0, 7),
               ascq._MatmulTypes(ascq.F16, ascq.INT4, ascq.F16, 0, 0, 7)]
    for t in refused:
        _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.E_UNSUPPORTED)


def test_int4_operand_handle():
    """int4b_t A / B (matmul_int4): accepted with int32 / f16 C; the workspace holds both operands unpacked to
    int8, plus the nibble-transposed B when B is given [K, N]; a transposed A and odd K / N are rejected before
    any launch"""
    L = ascq.lib()
    h = ctypes.c_void_p()
    d = ctypes.c_void_p(0x1000)
    t = ascq._MatmulTypes(ascq.INT4, ascq.INT4, ascq.INT32, ascq.INT32, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)
    _err(L.ascq_matmul_set_org_shape(h, 256, 7680, 128), ascq.OK)
    _err(L.ascq_matmul_set_tensor_a(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_tensor_b(h, d, 0), ascq.OK)
    ws = ctypes.c_size_t()
    _err(L.ascq_matmul_workspace_size(h, ctypes.byref(ws)), ascq.OK)
    assert ws.value == 256 * 128 + 7680 * 128 + 7680 * 64
    _err(L.ascq_matmul_set_tensor_b(h, d, 1), ascq.OK)
    _err(L.ascq_matmul_workspace_size(h, ctypes.byref(ws)), ascq.OK)
    assert ws.value == 256 * 128 + 7680 * 128
    _err(L.ascq_matmul_set_tensor_a(h, d, 1), ascq.OK)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_UNSUPPORTED)   # transposed int4 A
    _err(L.ascq_matmul_set_tensor_a(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_org_shape(h, 16, 16, 15), ascq.OK)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_INVALID_ARG)   # odd K
    _err(L.ascq_matmul_destroy(h), ascq.OK)
    t = ascq._MatmulTypes(ascq.INT4, ascq.INT4, ascq.F32, 0, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.E_UNSUPPORTED)


def test_hif8_operand_handle():
    """hifloat8 A and B (matmul_fp8.asc:229; both the same type, matmul_fp8/README_en.md): accepted with every C of
    the fp8 Matmul plus hifloat8 C; the workspace holds both operands decoded to bf16 rows of K rounded up to 8;
    hifloat8 mixed with fp8 is refused; a hifloat8 C needs a quant word before IterateAll"""
    L = ascq.lib()
    h = ctypes.c_void_p()
    d = ctypes.c_void_p(0x1000)
    for ct in (ascq.F32, ascq.F16, ascq.BF16, ascq.INT8, ascq.UINT8, ascq.INT4, ascq.FP8_E4M3, ascq.FP8_E5M2,
               ascq.HIF8):
        t = ascq._MatmulTypes(ascq.HIF8, ascq.HIF8, ct, ascq.F32, 0, 0)
        _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)
        _err(L.ascq_matmul_destroy(h), ascq.OK)
    for fa, fb in ((ascq.HIF8, ascq.FP8_E4M3), (ascq.FP8_E5M2, ascq.HIF8)):
        t = ascq._MatmulTypes(fa, fb, ascq.F32, 0, 0, 0)
        _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.E_UNSUPPORTED)
    t = ascq._MatmulTypes(ascq.HIF8, ascq.HIF8, ascq.F32, ascq.INT32, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.E_UNSUPPORTED)  # bias must be f32
    t = ascq._MatmulTypes(ascq.FP8_E4M3, ascq.FP8_E4M3, ascq.HIF8, 0, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)               # QF322HIF8_PRE on fp8
    _err(L.ascq_matmul_destroy(h), ascq.OK)
    t = ascq._MatmulTypes(ascq.HIF8, ascq.HIF8, ascq.HIF8, 0, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)
    _err(L.ascq_matmul_set_org_shape(h, 428, 479, 158), ascq.OK)
    _err(L.ascq_matmul_set_tensor_a(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_tensor_b(h, d, 0), ascq.OK)
    ws = ctypes.c_size_t()
    _err(L.ascq_matmul_workspace_size(h, ctypes.byref(ws)), ascq.OK)
    rup = lambda b: (b + 255) // 256 * 256  # noqa: E731
    assert ws.value == rup(428 * 160 * 2) + rup(479 * 160 * 2)
    _err(L.ascq_matmul_iterate_all(h, d, 0, None), ascq.E_STATE)  # hifloat8 C without a quant word
    _err(L.ascq_matmul_destroy(h), ascq.OK)


def test_no_device_reports_zero_or_more():
    assert ascq.lib().ascq_device_count() >= 0


@pytest.mark.parametrize("name", sorted(declared_functions()))
def test_header_comment_cites_reference_or_is_library_utility(name):
    """Every Matmul / quant entry point's declaration block carries a reference citation (file:line)."""
    text = HEADER.read_text()
    idx = text.index(name + "(")
    block = text[max(0, idx - 900):idx]
    utility = {"ascq_last_error", "ascq_version", "ascq_device_count", "ascq_weight_pack_size",
               "ascq_matmul_workspace_size", "ascq_matmul_set_workspace", "ascq_matmul_destroy"}
    if name in utility:
        return
    if "no counterpart in the reference" in block[-900:]:  # library-only entry points say so instead of citing
        return
    assert re.search(r"\.(h|asc|md|cpp|py):\d+", block), f"{name}: no reference file:line nearby"


def test_tiling_shim_compiles_and_behaves(tmp_path):
    """include/ascq_matmul.hpp's TCubeTiling mirror, MultiCoreMatmulTiling and Matmul::Init, compiled with g++
    as reference-style host code and run on the CPU (tests/cpp/tiling_shim.cpp)"""
    exe = tmp_path / "tiling_shim"
    libdir = Path(ascq.LIB_PATH).parent
    subprocess.run(["g++", "-std=c++17", "-Wall", "-I", str(ROOT / "include"), str(ROOT / "tests" / "cpp" / "tiling_shim.cpp"),
                    "-L", str(libdir), "-lascq", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr


def test_cube_tiling_struct_matches_header():
    assert ctypes.sizeof(ascq.CubeTiling) == 200
    assert ascq.CubeTiling.Ka.offset == 12 and ascq.CubeTiling.mxTypePara.offset == 196


def test_nz_argument_checks():
    L = ascq.lib()
    d = ctypes.c_void_p(0x1000)
    _err(L.ascq_nz_to_nd(d, d, ascq.U64, 1, 16, 32, 0, None), ascq.E_UNSUPPORTED)
    _err(L.ascq_nz_to_nd(d, d, ascq.F16, 1, 16, 32, 1, None), ascq.E_UNSUPPORTED)  # transpose needs 1-byte
    _err(L.ascq_nd_to_nz(d, d, ascq.INT8, 1, 0, 32, None), ascq.E_INVALID_ARG)
    _err(L.ascq_nz_to_nd(None, d, ascq.INT8, 1, 16, 32, 0, None), ascq.E_INVALID_ARG)
    assert L.ascq_nz_size(ascq.INT8, 2, 17, 33) == 2 * 2 * 2 * 512
    assert L.ascq_nz_size(ascq.F16, 1, 16, 16) == 512
    assert L.ascq_nz_size(ascq.U64, 1, 16, 16) == 0


def test_noalloc_iterate_all_rejects_oversized_workspace():
    """ascq_matmul_iterate_all_noalloc refuses, before launching anything, a handle whose workspace exceeds the
    static scratch (int8 [K, N] B of 8192 x 16384 needs 128 MiB to be transposed), and checks its arguments"""
    L = ascq.lib()
    h = ctypes.c_void_p()
    d = ctypes.c_void_p(0x1000)
    t = ascq._MatmulTypes(ascq.INT8, ascq.INT8, ascq.INT32, 0, 0, 0)
    _err(L.ascq_matmul_create(ctypes.byref(t), ctypes.byref(h)), ascq.OK)
    _err(L.ascq_matmul_set_org_shape(h, 1024, 16384, 8192), ascq.OK)
    _err(L.ascq_matmul_set_tensor_a(h, d, 0), ascq.OK)
    _err(L.ascq_matmul_set_tensor_b(h, d, 0), ascq.OK)
    ws = ctypes.c_size_t()
    _err(L.ascq_matmul_workspace_size(h, ctypes.byref(ws)), ascq.OK)
    assert ws.value > (64 << 20)
    _err(L.ascq_matmul_iterate_all_noalloc(h, d, 0, None), ascq.E_UNSUPPORTED)
    assert b"static scratch" in L.ascq_last_error()
    _err(L.ascq_matmul_iterate_all_noalloc(h, None, 0, None), ascq.E_INVALID_ARG)
    _err(L.ascq_matmul_destroy(h), ascq.OK)


def test_no_fma_with_zero_addend_in_half_arithmetic(tmp_path):
    """The half-arithmetic paths of quant.hip must not round an fp32 product to half through v_fma_mix*_f16 a, b, 0:
    an fma with a +0 addend turns a -0 product into +0, which the reference's half multiply keeps (e.g.
    (3 + -3) * -1.3 = -0).  Compiles the kernels to gfx950 assembly (CPU only) and looks for that instruction form."""
    out = tmp_path / "quant.s"
    cmd = ["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang",
           "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S", "-x", "hip",
           str(ROOT / "asc-devkit_clone_amd" / "csrc" / "quant.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    bad = [ln for ln in out.read_text().splitlines() if re.search(r"v_fma_mix(lo|hi)?_f16 .*, 0( |$)", ln)]
    assert not bad, bad[:5]


def _kernel_private_segments():
    """{kernel name: private (scratch) bytes per lane} of every kernel in the built libascq.so: the .hip_fatbin section
    holds one offload bundle per translation unit; each bundle's gfx950 code object carries the kernel metadata"""
    llvm = Path("/opt/rocm/llvm/bin")
    so = ROOT / "asc-devkit_clone_amd" / "libascq.so"
    out = {}
    with tempfile.TemporaryDirectory() as d:
        fb = Path(d) / "fatbin"
        subprocess.run([str(llvm / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fb}", str(so), str(Path(d) / "x")],
                       check=True, capture_output=True)
        data = fb.read_bytes()
        starts = [m.start() for m in re.finditer(re.escape(b"__CLANG_OFFLOAD_BUNDLE__"), data)]
        for n, (a, b) in enumerate(zip(starts, starts[1:] + [len(data)])):
            piece, co = Path(d) / f"b{n}", Path(d) / f"c{n}.o"
            piece.write_bytes(data[a:b])
            subprocess.run([str(llvm / "clang-offload-bundler"), "--unbundle", "--type=o", f"--input={piece}",
                            "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True,
                           capture_output=True)
            notes = subprocess.run([str(llvm / "llvm-readelf"), "--notes", str(co)], check=True, capture_output=True,
                                   text=True).stdout
            names = re.findall(r"\.name:\s+(\S+)", notes)
            sizes = re.findall(r"\.private_segment_fixed_size:\s+(\d+)", notes)
            assert len(names) == len(sizes)
            out.update(zip(names, map(int, sizes)))
    return out


def test_matmul_kernels_use_no_scratch():
    """The GEMM, group-matmul, MX and antiquant-GEMV kernels keep their accumulators and operands in registers: a
    kernel that needs private (scratch) memory has had its accumulator array or argument block demoted to memory by
    the compiler, which costs several times the kernel's time (an fp8 GEMM with an extra unrolled epilogue ran 13x
    slower that way).  Reads the kernel metadata of the built library's code objects (CPU only)."""
    seg = _kernel_private_segments()
    hot = {k: v for k, v in seg.items() if re.search(r"gemm|aq_|antiquant_gemm", k)}
    assert len(hot) > 50
    bad = {k: v for k, v in hot.items() if v}
    assert not bad, bad


def test_env_gated_host_log():
    """ASCQ_LOG=1 prints the message of a failed call on stderr; unset, the library is silent"""
    import subprocess
    import sys

    code = ("import sys; sys.path.insert(0, %r); import ascq; "
            "print(ascq.lib().ascq_quant_group_matmul(None, 0, None, None, None, 0, None, None, 0, 0, 0, 0, 0, 0, None))"
            % str(ROOT / "asc-devkit_clone_amd"))
    for env_val, expect in (("1", True), ("0", False)):
        env = dict(os.environ, ASCQ_LOG=env_val)
        r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        assert ("ascq: error" in r.stderr and "null argument" in r.stderr) == expect, r.stderr
