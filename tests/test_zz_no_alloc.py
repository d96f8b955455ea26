"""ascq_matmul_iterate_all_noalloc (IterateAll with the workspace taken from the library's static per-device
scratch, allocating nothing) against ascq_matmul_iterate_all, bit-exact, on two calls in a row -- the second with a
smaller problem -- for each kind of handle that uses a workspace: int8 with a [K, N] B transposed into it, int8 at
decode-sized batches keeping K-split partials in it, MX-FP4
with its scales rearranged (and a [K, N] B transposed) into it, and int4 operands unpacked into it.  The handle
keeps its own workspace across the allocation-free calls.  A fresh handle that only calls the allocation-free entry
leaves the device's free memory unchanged and owns no workspace afterwards, and the call replays correctly from a
captured HIP graph."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import seeded

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _both(ascq, mm, shape, dtype):
    """IterateAll into one buffer and IterateAllNoAlloc into another (both pre-filled with different garbage);
    returns the two outputs"""
    c1 = torch.full(shape, 3, dtype=dtype, device="cuda")
    c2 = torch.full(shape, 5, dtype=dtype, device="cuda")
    mm.IterateAll(c1)
    mm.IterateAllNoAlloc(c2)
    torch.cuda.synchronize()
    return c1, c2


def _same(c1, c2):
    a, b = c1.cpu(), c2.cpu()
    if a.dtype in (torch.float16, torch.bfloat16):
        a, b = a.view(torch.int16), b.view(torch.int16)
    elif a.dtype == torch.float32:
        a, b = a.view(torch.int32), b.view(torch.int32)
    assert torch.equal(a, b)


def test_noalloc_int8_kn_b(ascq_gpu, oracle):
    """int8 x int8 -> f16 (VDEQF16), B given [K, N] with M, N >= 1024 (the 256 x 256 tile sizes): B is transposed
    into the workspace (smaller [K, N] problems read it in place with LDS transpose reads)"""
    ascq = ascq_gpu
    mm = ascq.Matmul(ascq.INT8, ascq.INT8, ascq.F16, ascq.INT32)
    for i, (M, N, K) in enumerate([(1024, 1024, 512), (1024, 1024, 256)]):
        rng = seeded(300 + i)
        A = rng.integers(-127, 128, (M, K), dtype=np.int8)
        B = rng.integers(-127, 128, (K, N), dtype=np.int8)
        bias = rng.integers(-(1 << 15), 1 << 15, N, dtype=np.int32)
        sc = np.exp(rng.uniform(np.log(2.0 ** -12), np.log(2.0 ** -6), N)).astype(np.float32)
        words = sc.view(np.uint32).astype(np.uint64)
        mm.SetOrgShape(M, N, K)
        assert mm.WorkspaceSize() > 0
        mm.SetQuantVector(_dev(words.view(np.int64)))
        mm.SetTensorA(_dev(A))
        mm.SetTensorB(_dev(B), False)
        mm.SetBias(_dev(bias))
        c1, c2 = _both(ascq, mm, (M, N), torch.float16)
        _same(c1, c2)
        ref = O.mm_dequant(O.matmul_i8(A, B, bias), O.F16, qvec=words)
        np.testing.assert_array_equal(c2.cpu().view(torch.int16).numpy().view(np.uint16), ref)
        mm.End()


def test_noalloc_int8_decode_split(ascq_gpu, oracle):
    """int8 x int8 -> f16 at decode-sized batches with B given [K, N] and long K: the K split across workgroups keeps
    its partials in the workspace (the static scratch for the allocation-free call); then a smaller problem"""
    ascq = ascq_gpu
    mm = ascq.Matmul(ascq.INT8, ascq.INT8, ascq.F16, ascq.INT32)
    for i, (M, N, K) in enumerate([(8, 4096, 8192), (1, 2048, 8192)]):
        rng = seeded(320 + i)
        A = rng.integers(-127, 128, (M, K), dtype=np.int8)
        B = rng.integers(-127, 128, (K, N), dtype=np.int8)
        bias = rng.integers(-(1 << 15), 1 << 15, N, dtype=np.int32)
        sc = np.exp(rng.uniform(np.log(2.0 ** -12), np.log(2.0 ** -6), N)).astype(np.float32)
        words = sc.view(np.uint32).astype(np.uint64)
        mm.SetOrgShape(M, N, K)
        assert mm.WorkspaceSize() > 0
        mm.SetQuantVector(_dev(words.view(np.int64)))
        mm.SetTensorA(_dev(A))
        mm.SetTensorB(_dev(B), False)
        mm.SetBias(_dev(bias))
        c1, c2 = _both(ascq, mm, (M, N), torch.float16)
        _same(c1, c2)
        ref = O.mm_dequant(O.matmul_i8(A, B, bias), O.F16, qvec=words)
        np.testing.assert_array_equal(c2.cpu().view(torch.int16).numpy().view(np.uint16), ref)
        mm.End()


def test_noalloc_mx_fp4(ascq_gpu, oracle):
    """MX-FP4 -> bf16 with a [K, N] B: B transposed and both scale tensors rearranged in the workspace"""
    from test_gpu_mx import mx_inputs, scale_pairs, to_kn

    ascq = ascq_gpu
    mm = ascq.Matmul(ascq.FP4_E2M1, ascq.FP4_E2M1, ascq.BF16, 0, ascq.E8M0)
    for i, (M, N, K) in enumerate([(256, 384, 512), (128, 128, 256)]):
        A, sA, Bt, sBt = mx_inputs(seeded(310 + i), M, N, K)
        mm.SetOrgShape(M, N, K)
        assert mm.WorkspaceSize() > 0
        mm.SetTensorA(_dev(A))
        mm.SetTensorB(_dev(to_kn(Bt, N, K)), False)
        mm.SetTensorScaleA(_dev(sA), 0)
        mm.SetTensorScaleB(_dev(scale_pairs(sBt)), 0)
        c1, c2 = _both(ascq, mm, (M, N), torch.bfloat16)
        _same(c1, c2)
        mm.End()


def test_noalloc_int4(ascq_gpu, oracle):
    """int4 x int4 -> int32: both operands unpacked to int8 in the workspace (B given [K, N], nibble-transposed)"""
    ascq = ascq_gpu
    mm = ascq.Matmul(ascq.INT4, ascq.INT4, ascq.INT32, ascq.INT32)
    for i, (M, N, K) in enumerate([(256, 512, 256), (64, 128, 128)]):
        rng = seeded(320 + i)
        a = rng.integers(-8, 8, (M, K), dtype=np.int8)
        b = rng.integers(-8, 8, (K, N), dtype=np.int8)
        pa = ((a[:, 0::2] & 0xF) | ((a[:, 1::2] & 0xF) << 4)).astype(np.uint8)
        pb = ((b[:, 0::2] & 0xF) | ((b[:, 1::2] & 0xF) << 4)).astype(np.uint8)
        mm.SetOrgShape(M, N, K)
        assert mm.WorkspaceSize() > 0
        mm.SetTensorA(_dev(pa))
        mm.SetTensorB(_dev(pb), False)
        c1, c2 = _both(ascq, mm, (M, N), torch.int32)
        _same(c1, c2)
        np.testing.assert_array_equal(c2.cpu().numpy(), O.matmul_i8(a, b))
        mm.End()


def _int8_kn_handle(ascq, M, N, K, seed):
    """an int8 -> f16 handle with B given [K, N] (M, N >= 1024: B is transposed into the workspace) and its inputs"""
    rng = seeded(seed)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-127, 128, (K, N), dtype=np.int8)
    words = np.full(N, np.float32(2.0 ** -10).view(np.uint32), np.uint64)
    mm = ascq.Matmul(ascq.INT8, ascq.INT8, ascq.F16, 0)
    mm.SetOrgShape(M, N, K)
    mm.SetQuantVector(_dev(words.view(np.int64)))
    mm.SetTensorA(_dev(A))
    mm.SetTensorB(_dev(B), False)
    return mm, A, B, words


def test_noalloc_fresh_handle_allocates_nothing(ascq_gpu, oracle):
    """A fresh handle that only ever calls IterateAllNoAlloc: the output matches the oracle and the device's free
    memory does not move (a workspace of its own would take >= 8 MiB); the first IterateAll on the same handle then
    allocates that workspace -- so the handle had none of its own before"""
    ascq = ascq_gpu
    M, N, K = 1024, 2048, 4096
    warm, _, _, _ = _int8_kn_handle(ascq, M, N, K, 330)  # loads the kernels and the scratch address first
    c = torch.empty((M, N), dtype=torch.float16, device="cuda")
    warm.IterateAllNoAlloc(c)
    torch.cuda.synchronize()
    mm, A, B, words = _int8_kn_handle(ascq, M, N, K, 331)
    need = mm.WorkspaceSize()
    assert need >= 8 << 20
    free0 = torch.cuda.mem_get_info()[0]
    mm.IterateAllNoAlloc(c)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert abs(free0 - free1) < (2 << 20), (free0, free1)
    ref = O.mm_dequant(O.matmul_i8(A, B), O.F16, qvec=words)
    np.testing.assert_array_equal(c.cpu().view(torch.int16).numpy().view(np.uint16), ref)
    c2 = torch.empty_like(c)
    free2 = torch.cuda.mem_get_info()[0]
    mm.IterateAll(c2)
    torch.cuda.synchronize()
    assert free2 - torch.cuda.mem_get_info()[0] >= need - (2 << 20)
    assert torch.equal(c.view(torch.int16), c2.view(torch.int16))
    mm.End()
    warm.End()


def test_noalloc_graph_capture_replays(ascq_gpu, oracle):
    """IterateAllNoAlloc captured in a HIP graph (the transpose of B into the scratch and the GEMM: kernel nodes only,
    no memset, no allocation): every replay, with eager allocation-free calls of another handle on the same scratch
    between the replays, equals the eager call bit for bit"""
    ascq = ascq_gpu
    M, N, K = 1024, 1024, 512
    mm, A, B, words = _int8_kn_handle(ascq, M, N, K, 340)
    other, _, _, _ = _int8_kn_handle(ascq, M, N, 256, 341)
    eager = torch.empty((M, N), dtype=torch.float16, device="cuda")
    mm.IterateAllNoAlloc(eager)
    junk = torch.empty_like(eager)
    other.IterateAllNoAlloc(junk)
    torch.cuda.synchronize()
    ref = O.mm_dequant(O.matmul_i8(A, B), O.F16, qvec=words)
    np.testing.assert_array_equal(eager.cpu().view(torch.int16).numpy().view(np.uint16), ref)
    out = torch.empty_like(eager)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(graph, stream=st):
            mm.IterateAllNoAlloc(out)
    torch.cuda.current_stream().wait_stream(st)
    for rep in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {rep} differs from the eager call"
        other.IterateAllNoAlloc(junk)  # overwrites the shared scratch between replays
        torch.cuda.synchronize()
    del graph
    mm.End()
    other.End()
