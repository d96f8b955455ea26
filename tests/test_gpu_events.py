"""Launch-event hook (ascq_set_launch_events): armed events time the next entry point's main kernel, and an entry
point that fails its argument checks disarms them, so they never time a later, unrelated call."""
from __future__ import annotations

import ctypes
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu


def _hip():
    p = Path(torch.__file__).resolve().parent / "lib" / "libamdhip64.so"
    hip = ctypes.CDLL(str(p) if p.exists() else "libamdhip64.so.7")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipGetLastError.argtypes = []
    return hip


def _events(hip):
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipEventCreate(ctypes.byref(a)) == 0 and hip.hipEventCreate(ctypes.byref(b)) == 0
    return a, b


def _elapsed(hip, a, b):
    ms = ctypes.c_float()
    rc = hip.hipEventElapsedTime(ctypes.byref(ms), a, b)
    return rc, ms.value


def test_events_time_the_next_call(ascq_gpu):
    hip = _hip()
    a, b = _events(hip)
    x = torch.randn(256, 1024, device="cuda").half()
    ascq_gpu.check(ascq_gpu.lib().ascq_set_launch_events(a, b), "set_launch_events")
    ascq_gpu.quant_dynamic_per_token(x)
    torch.cuda.synchronize()
    rc, ms = _elapsed(hip, a, b)
    assert rc == 0 and ms > 0.0
    hip.hipEventDestroy(a)
    hip.hipEventDestroy(b)


def test_failed_call_disarms_events(ascq_gpu):
    hip = _hip()
    a, b = _events(hip)
    x = torch.randn(256, 1024, device="cuda").half()
    lib = ascq_gpu.lib()
    ascq_gpu.check(lib.ascq_set_launch_events(a, b), "set_launch_events")
    # a null destination fails the argument checks before anything is launched
    st = lib.ascq_ascend_quant_dynamic_per_token(None, None, x.data_ptr(), ascq_gpu.F16, 256, 1024,
                                                 ascq_gpu.ROUND_RINT, torch.cuda.current_stream().cuda_stream)
    assert st != ascq_gpu.OK
    # the next, valid call must not record the events any more
    ascq_gpu.quant_dynamic_per_token(x)
    torch.cuda.synchronize()
    rc, _ = _elapsed(hip, a, b)
    # the query of unrecorded events leaves its error as the thread's last HIP error: clear it, or the next HIP
    # call of another test (torch's included) reports it as its own
    hip.hipGetLastError()
    assert rc != 0, "events armed before a failed call still timed the next call"
    hip.hipEventDestroy(a)
    hip.hipEventDestroy(b)
