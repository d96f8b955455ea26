"""Benchmark of the MI355X quantized-inference hot path (one GPU).

Headline (the JSON line's value): AscendQuant per-token dynamic quant f16 [8192, 8192] -> int8 + fp32 scale,
then AscendDequant back to f16 -- one step = both ops over one batch, inputs resident in HBM.  value = whole-job
algorithmic GB/s (6*M*N + 8*M bytes per step).  Buffers are rotated over more than the 256 MB Infinity Cache so
the figure is HBM, not MALL, bandwidth.

Also measured and reported under "other_configs": the W8A8 int8 Matmul + per-channel DEQF16 (128x512x256 and the
8192^3 throughput shape), the W4A16 / W8A16 decode GEMV (M in {1, 16, 64}), the MoE group matmul (both weight
layouts), the MX-FP4 8192^3 GEMM and the fp8 / MX-FP8 8192^3 GEMMs, and -- for scale, not this library -- the
vendor BLAS (hipBLASLt through torch) on the int8 and fp8 8192^3 shapes.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                  [--only all|headline|quant|w8a8|gemv|group|mx|fp8|vendor|traffic|shapes|decode]

`--only shapes` (not part of the default run) times the weight-only matmul over model shapes (attention and MLP
projections of 7B / 13B / 70B-class models) at M = 1 / 16 / 64 / 512; `--only decode` (not part of the default run
either) times the int8, fp8 and MX-FP4 Matmuls at decode-sized batches (M = 1 / 16 / 64, B [N, K] streamed once; int8
and fp8 also with B given [K, N] at M = 1 / 64) and the MoE group matmul at 16 / 64 / 256 tokens.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "asc-devkit_clone_amd"))

METRIC = "int8/MXFP4 GEMM TOPS (%MFMA peak); antiquant GEMV + quant op HBM GB/s (%peak)"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0      # dense int8 MFMA, MI355X
MXFP4_PEAK_TFLOPS = 10100.0  # dense fp4 MFMA, MI355X
FP8_PEAK_TFLOPS = 5000.0     # dense fp8 MFMA, MI355X
F16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 * 2 ** 20


def rotation(bytes_per_set: int, minimum: int = 2) -> int:
    return max(minimum, int(np.ceil(2.5 * MALL_BYTES / bytes_per_set)))


def parse_traffic() -> dict:
    """Per-launch HBM bytes measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (profiles/pmc_traffic.txt:
    '<kernel-key> <bytes>' lines, copy-kernel calibrated)."""
    p = ROOT / "profiles" / "pmc_traffic.txt"
    out = {}
    if p.exists():
        for ln in p.read_text().splitlines():
            ln = ln.strip()
            if not ln or ln.startswith("#"):
                continue
            parts = ln.split()
            if len(parts) >= 2:
                try:
                    out[parts[0]] = float(parts[1])
                except ValueError:
                    pass
    return out


def bench_headline(torch, ascq, steps, warmup):
    M = N = 8192
    bytes_quant = 2 * M * N + M * N + 4 * M
    bytes_dequant = M * N + 4 * M + 2 * M * N
    per_set = 2 * M * N + M * N + 4 * M + 2 * M * N
    # four sets at least: the kernel-alone loops below touch x and q (quant) or q and y (dequant) of a set, 201 MB,
    # so four sets keep them above 3 x the 256 MB Infinity Cache
    R = rotation(per_set, 4)
    g = torch.Generator(device="cuda")
    g.manual_seed(20261201)
    xs, qs, ss, ys = [], [], [], []
    for _ in range(R):
        x = torch.randn((M, N), generator=g, device="cuda", dtype=torch.float32)
        mask = torch.rand((M, N), generator=g, device="cuda") < 0.001
        x = torch.where(mask, x * 50.0, x).to(torch.float16)
        xs.append(x)
        qs.append(torch.empty((M, N), dtype=torch.int8, device="cuda"))
        ss.append(torch.empty((M,), dtype=torch.float32, device="cuda"))
        ys.append(torch.empty((M, N), dtype=torch.float16, device="cuda"))
    stream = torch.cuda.current_stream()

    def quant(i):
        r = i % R
        ascq.quant_dynamic_per_token(xs[r], out=qs[r], scale_out=ss[r])

    def dequant(i):
        r = i % R
        ascq.ascend_dequant_policy(qs[r], ss[r], ascq.PER_TOKEN, torch.float16, out=ys[r])

    for i in range(warmup):
        quant(i)
        dequant(i)
    torch.cuda.synchronize()

    def timed(fn, n):
        """events on the launch stream around n back-to-back calls (queued ahead, so the GPU runs them without
        host gaps); returns the elapsed ms"""
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(n):
            fn(i)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end)

    # whole job: `steps` steps of quant then dequant, nothing else in the timed region
    t0 = time.perf_counter()
    total_ms = timed(lambda i: (quant(warmup + i), dequant(warmup + i)), steps)
    wall = time.perf_counter() - t0
    # each kernel on its own: n launches in a row (rotating buffers, so every launch reads from HBM); the average
    # includes the small gap between consecutive dispatches
    n_k = max(steps // 2, 10)
    q_ms = timed(quant, n_k) / n_k
    d_ms = timed(dequant, n_k) / n_k
    return dict(M=M, N=N, R=R, total_ms=total_ms, wall_s=wall, q_ms=q_ms, d_ms=d_ms, bytes_quant=bytes_quant,
                bytes_dequant=bytes_dequant, q_samples=n_k, d_samples=n_k)


def _cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    threads = int(os.environ.get("OMP_NUM_THREADS", nproc))
    return model, nproc, threads


def _median_s(fn, runs=5, warmup=1):
    """median wall time of `runs` calls after `warmup` untimed ones"""
    for _ in range(warmup):
        fn()
    t = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        t.append(time.perf_counter() - t0)
    return float(np.median(t)), t


def _cpu_record(value, unit, sample, secs, runs):
    model, nproc, threads = _cpu_info()
    return dict(value=value, unit=unit, cores=threads, kind="port", sample=sample, cpu_model=model, nproc=nproc,
                omp_threads=threads, median_s=round(secs, 5), runs=[round(x, 5) for x in runs],
                method="median of 5 timed runs after 1 untimed warm-up; oracle/ascq_oracle.c at -O3 "
                       "-march=x86-64-v3 with OpenMP")


def _oracle():
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    return O


def cpu_baseline_headline():
    """The oracle (C restatement, OpenMP) on the host: dynamic per-token quant + dequant over the full
    8192 x 8192 workload."""
    O = _oracle()
    M = N = 8192
    rng = np.random.default_rng(7)
    x = rng.standard_normal((M, N), dtype=np.float32).astype(np.float16).view(np.uint16)

    def run():
        q, s = O.quant_dynamic_per_token(x, O.F16)
        O.dequant_policy(q, O.INT8, s, O.F32, O.PER_TOKEN, O.F16)

    secs, runs = _median_s(run)
    return _cpu_record((6 * M * N + 8 * M) / secs / 1e9, "GB/s", "full 8192x8192 f16 workload (quant + dequant)",
                       secs, runs)


def cpu_baseline_w8a8(M, N, K):
    """int32 GEMM + bias + per-channel DEQF16 on the host; the 8192^3 shape on a 64-row sample"""
    O = _oracle()
    rng = np.random.default_rng(1)
    rows = M if M <= 1024 else 64
    A = rng.integers(-127, 128, (rows, K), dtype=np.int8)
    B = rng.integers(-127, 128, (K, N), dtype=np.int8)
    bias = rng.integers(-(1 << 15), 1 << 15, N, dtype=np.int32)
    words = np.full(N, np.float32(2.0 ** -9).view(np.uint32), np.uint64)
    secs, runs = _median_s(lambda: O.mm_dequant(O.matmul_i8(A, B, bias), O.F16, qvec=words))
    return _cpu_record(2 * rows * N * K / secs / 1e12, "TOPS", f"{rows} of {M} rows x N={N} x K={K}", secs, runs)


def cpu_baseline_gemv(bits, M):
    """dequant-on-the-fly dot products (oracle antiquant_matmul) at K = 4096, N = 11008, group 128"""
    O = _oracle()
    K, N, g = 4096, 11008, 128
    rng = np.random.default_rng(3)
    rows = min(M, 4)
    x = rng.standard_normal((rows, K)).astype(np.float16).view(np.uint16)
    if bits == 4:
        w = rng.integers(0, 256, (K, N // 2), dtype=np.uint8)
    else:
        w = rng.integers(-128, 128, (K, N), dtype=np.int8)
    sc = np.full((K // g, N), np.float16(0.01).view(np.uint16), np.uint16)
    of = np.full((K // g, N), np.float16(1.0).view(np.uint16), np.uint16)
    secs, runs = _median_s(lambda: O.antiquant_matmul(x, w, O.INT4 if bits == 4 else O.INT8, sc, of, g, rows, N, K))
    nbytes = K * N * bits // 8 + 2 * (K // g) * N * 2 + 2 * rows * K + 2 * rows * N
    return _cpu_record(nbytes / secs / 1e9, "GB/s", f"M={rows} (of {M}) x K={K} x N={N}; bytes as the GPU line "
                       "counts them for that M", secs, runs)


def cpu_baseline_group():
    """the MoE group matmul on a 512-token, 2-expert sample of the 4096-token, 16-expert workload (same K, N)"""
    O = _oracle()
    G, T, K, N = 2, 512, 4096, 1408
    rng = np.random.default_rng(4)
    x = rng.integers(-127, 128, (T, K), dtype=np.int8)
    w = rng.integers(-127, 128, (G, K, N), dtype=np.int8)
    pts = np.full(T, 0.01, np.float32)
    scale = np.full((G, N), 0.01, np.float32)
    gl = np.array([0, 300, T], np.int64)
    secs, runs = _median_s(lambda: O.group_matmul(x, pts, w, scale, gl, 0, G, T, K, N))
    return _cpu_record(2 * T * K * N / secs / 1e12, "TOPS", f"T={T} tokens in {G} groups, K={K}, N={N}", secs, runs)


def cpu_baseline_mx():
    """the MX-FP4 8192^3 GEMM (fp64 dequant-then-matmul, the reference golden) on 4 output rows"""
    O = _oracle()
    M = N = K = 8192
    rng = np.random.default_rng(5)
    rows = np.arange(4, dtype=np.int64)
    A = rng.integers(0, 256, (M, K // 2), dtype=np.uint8)
    Bt = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sA = np.full((M, K // 32), 127, np.uint8)
    sB = np.full((N, K // 32), 127, np.uint8)
    secs, runs = _median_s(lambda: O.mx_matmul(A, Bt, sA, sB, M, N, K, trans_b=True, sa_layout=0, sb_layout=1,
                                                rows=rows), runs=5, warmup=1)
    return _cpu_record(2 * len(rows) * N * K / secs / 1e12, "TFLOPS", f"{len(rows)} of {M} rows x N={N} x K={K}",
                       secs, runs)


def _roof(bound, achieved, peak, unit):
    return dict(bound=bound, achieved=round(achieved, 3), peak=peak, unit=unit, frac=round(achieved / peak, 4))


# ----------------------------------------------------------------------------------------------
# other configs (GPU only)
# ----------------------------------------------------------------------------------------------
def bench_prefill(torch, ascq, w_type, M, iters):
    """weight-only antiquant matmul at a prefill batch: x f16 [M, 4096] against the config-3 weight (int4 / int8
    [4096, 11008], g = 128 f16 scale + offset), fp32 accumulation, f16 out -- the LDS-ring kernel over 128-row blocks"""
    K, N, grp = 4096, 11008, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    wb = K * N // (2 if w_type == ascq.INT4 else 1)
    R = rotation(wb + 2 * 2 * (K // grp) * N + 2 * M * K + 2 * M * N)
    wps, scs, ofs, xs, ys = [], [], [], [], []
    for _ in range(R):
        wps.append(torch.randint(0, 256, (wb,), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8))
        scs.append(torch.exp(torch.empty((K // grp, N), device="cuda").uniform_(np.log(1e-3), np.log(1e-1),
                                                                                 generator=g)).half())
        ofs.append(torch.empty((K // grp, N), device="cuda").uniform_(-8, 8, generator=g).half())
        xs.append(torch.randn((M, K), generator=g, device="cuda").half())
        ys.append(torch.empty((M, N), dtype=torch.float16, device="cuda"))

    def fn(i):
        r = i % R
        ascq.antiquant_matmul(xs[r], wps[r], w_type, scs[r], ofs[r], grp, N, out=ys[r])

    ms = _time_loop(torch, fn, iters)
    bits = 4 if w_type == ascq.INT4 else 8
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    return dict(workload=f"W{bits}A16 antiquant matmul (prefill), M={M} K={K} N={N} g={grp}", ms=ms, value=tf,
                unit="TFLOPS", frac_of_peak=tf / F16_PEAK_TFLOPS)


def _time_loop(torch, fn, iters, warmup=3, reps=3):
    """ms per call: the median over `reps` timed loops of `iters` back-to-back calls (events around each loop)"""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    res = []
    for _ in range(reps):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(iters):
            fn(i)
        e.record()
        torch.cuda.synchronize()
        res.append(s.elapsed_time(e) / iters)
    return sorted(res)[len(res) // 2]


USE_GRAPH = True  # --no-graph: eager timing only (counter passes of rocprofv3)


def _time_graph(torch, fn, iters, out):
    """Device time per call of `iters` calls captured in one HIP graph and replayed (the host's per-call overhead,
    ~6.5 us through the Python binding, is outside the graph).  The graph's last output must equal an eager call's
    bit for bit.  Returns (ms per call in the graph, ms per call eager)."""
    eager = _time_loop(torch, fn, iters)
    if not USE_GRAPH:
        return eager, eager
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(graph, stream=st):
            for i in range(iters):
                fn(i)
    torch.cuda.current_stream().wait_stream(st)
    out.zero_()
    graph.replay()
    torch.cuda.synchronize()
    replayed = out.clone()
    fn(iters - 1)
    torch.cuda.synchronize()
    if not torch.equal(replayed, out):
        raise RuntimeError("graph replay differs from the eager call")
    best = float("inf")
    for _ in range(3):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        graph.replay()
        e.record()
        torch.cuda.synchronize()
        best = min(best, s.elapsed_time(e) / iters)
    del graph
    return best, eager


def bench_w8a8(torch, ascq, M, N, K, iters):
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    per = M * K + K * N + 2 * M * N
    R = rotation(per, 1) if M * N * K > 1e9 else 1
    A = [torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8) for _ in range(R)]
    B = [torch.randint(-127, 128, (K, N), generator=g, device="cuda", dtype=torch.int8) for _ in range(R)]
    bias = torch.randint(-(1 << 15), 1 << 15, (N,), generator=g, device="cuda", dtype=torch.int32)
    sc = torch.exp(torch.empty(N, device="cuda").uniform_(np.log(2.0 ** -12), np.log(2.0 ** -6), generator=g))
    words = sc.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    C = [torch.empty((M, N), dtype=torch.float16, device="cuda") for _ in range(R)]
    mm = ascq.Matmul(ascq.INT8, ascq.INT8, ascq.F16, ascq.INT32)
    mm.SetOrgShape(M, N, K)
    mm.SetQuantVector(words)
    mm.SetBias(bias)

    def fn(i):
        r = i % R
        mm.SetTensorA(A[r])
        mm.SetTensorB(B[r])
        mm.IterateAll(C[r])

    extra = {}
    if R == 1:  # launch-bound sample shape: device time from a graph of the calls
        ms, eager = _time_graph(torch, fn, iters, C[0])
        extra = dict(timing="HIP graph of the calls, replayed" if USE_GRAPH else "eager calls", eager_ms=eager)
    else:
        ms = _time_loop(torch, fn, iters)
    tops = 2 * M * N * K / (ms * 1e-3) / 1e12
    return dict(workload=f"W8A8 int8 Matmul + bias + per-channel DEQF16 -> f16, M={M} N={N} K={K}",
                ms=ms, value=tops, unit="TOPS", frac_of_peak=tops / INT8_PEAK_TOPS, **extra)


def bench_gemv(torch, ascq, w_type, M, iters):
    K, N, grp = 4096, 11008, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    wb = K * N // (2 if w_type == ascq.INT4 else 1)
    R = rotation(wb + 2 * 2 * (K // grp) * N)
    # weights, scales and offsets all rotate, so every call reads each of them from HBM
    wps, scs, ofs = [], [], []
    for _ in range(R):
        wps.append(torch.randint(0, 256, (wb,), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8))
        scs.append(torch.exp(torch.empty((K // grp, N), device="cuda").uniform_(np.log(1e-3), np.log(1e-1),
                                                                                 generator=g)).half())
        ofs.append(torch.empty((K // grp, N), device="cuda").uniform_(-8, 8, generator=g).half())
    x = torch.randn((M, K), generator=g, device="cuda").half()
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")

    def fn(i):
        r = i % R
        ascq.antiquant_matmul(x, wps[r], w_type, scs[r], ofs[r], grp, N, out=y)

    ms, eager = _time_graph(torch, fn, iters, y)
    bits = 4 if w_type == ascq.INT4 else 8
    nbytes = K * N * bits // 8 + 2 * (K // grp) * N * 2 + 2 * M * K + 2 * M * N
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(workload=f"W{bits}A16 antiquant GEMV, M={M} K={K} N={N} g={grp}", ms=ms, value=gbs, unit="GB/s",
                frac_of_peak=gbs / HBM_PEAK_GBS, tflops=2 * M * N * K / (ms * 1e-3) / 1e12,
                timing="HIP graph of the calls (weights rotating), replayed" if USE_GRAPH else "eager calls",
                eager_ms=eager)


def bench_wo_shape(torch, ascq, K, N, M, iters, grp=128, w_type=None):
    """weight-only matmul (int4, g = 128 f16 scale + offset) at one model shape: the same call as the decode GEMV and
    prefill lines, weights rotating past the Infinity Cache, timed as a HIP graph of the calls replayed"""
    w_type = ascq.INT4 if w_type is None else w_type
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    G = K // grp
    wb = K * N // (2 if w_type == ascq.INT4 else 1)
    R = rotation(wb + 4 * G * N)
    wps = [torch.randint(0, 256, (wb,), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8)
           for _ in range(R)]
    sc = torch.exp(torch.empty((G, N), device="cuda").uniform_(np.log(1e-3), np.log(1e-1), generator=g)).half()
    of = torch.empty((G, N), device="cuda").uniform_(-8, 8, generator=g).half()
    x = torch.randn((M, K), generator=g, device="cuda").half()
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")

    def fn(i):
        ascq.antiquant_matmul(x, wps[i % R], w_type, sc, of, grp, N, out=y)

    ms, eager = _time_graph(torch, fn, iters, y)
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    gbs = (K * N // 2 + 4 * G * N + 2 * M * K + 2 * M * N) / (ms * 1e-3) / 1e9
    return dict(workload=f"W4A16 weight-only matmul K={K} N={N} M={M} g={grp}", ms=ms, value=tf, unit="TFLOPS",
                frac_of_peak=tf / F16_PEAK_TFLOPS, gbs=round(gbs, 1), eager_ms=eager)


def bench_decode_matmul(torch, ascq, kind, K, N, M, iters=50, trans_b=True):
    """a quantized Matmul at a decode-sized batch (B [N, K] streamed once per call: the weight stream is the roofline),
    weights rotating past the Infinity Cache, timed as a HIP graph of the calls replayed.  kind: "int8" (W8A8,
    per-channel DEQF16 -> f16), "fp8" (e4m3, per-channel QF322BF16 -> bf16), "mxfp4" (E2M1 / E8M0 -> bf16; the
    call includes the scale rearrangement launch)"""
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    if kind == "int8":
        wb = K * N
        R = rotation(wb)
        A = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
        Bs = [(torch.randint(-127, 128, (N, K) if trans_b else (K, N), generator=g, device="cuda", dtype=torch.int8), None)
              for _ in range(R)]
        C = torch.empty((M, N), dtype=torch.float16, device="cuda")
        mm = ascq.Matmul(ascq.INT8, ascq.INT8, ascq.F16)
        mm.SetQuantVector(torch.full((N,), 0x3A800000, dtype=torch.int64, device="cuda"))
        what = "W8A8 int8 Matmul, per-channel DEQF16 -> f16"
    elif kind == "fp8":
        wb = K * N
        R = rotation(wb)
        A = _fp8_bytes(torch, (M, K), g, torch.float8_e4m3fn)
        Bs = [(_fp8_bytes(torch, (N, K) if trans_b else (K, N), g, torch.float8_e4m3fn), None) for _ in range(R)]
        C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        mm = ascq.Matmul(ascq.FP8_E4M3, ascq.FP8_E4M3, ascq.BF16)
        mm.SetQuantVector(torch.full((N,), 0x3C000000, dtype=torch.int64, device="cuda"))
        what = "fp8 e4m3 Matmul, per-channel QF322BF16 -> bf16"
    else:
        wb = K * N // 2 + K * N // 32
        R = rotation(wb)
        A, sA = _mx_fp4_normal(torch, M, K, g)
        Bs = [_mx_fp4_normal(torch, N, K, g) for _ in range(R)]
        C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        mm = ascq.Matmul(ascq.FP4_E2M1, ascq.FP4_E2M1, ascq.BF16, 0, ascq.E8M0)
        what = "MX-FP4 Matmul (E2M1, E8M0 per 32) -> bf16"
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(A)
    if kind == "mxfp4":
        mm.SetTensorScaleA(sA, False)

    def fn(i):
        B, sB = Bs[i % R]
        mm.SetTensorB(B, trans_b)
        if sB is not None:
            mm.SetTensorScaleB(sB, True)
        mm.IterateAll(C)

    ms, eager = _time_graph(torch, fn, iters, C)
    gbs = wb / (ms * 1e-3) / 1e9
    return dict(workload=f"{what}, decode batch M={M}, K={K}, N={N}, B given " + ("[N,K]" if trans_b else "[K,N]"),
                ms=ms, value=round(gbs, 1),
                unit="GB/s", frac_of_peak=gbs / HBM_PEAK_GBS, tops=round(2 * M * N * K / (ms * 1e-3) / 1e12, 1),
                timing="HIP graph of the calls (weights rotating), replayed" if USE_GRAPH else "eager calls",
                eager_ms=eager)


def bench_group_decode(torch, ascq, T, iters=30, G=16, K=4096, N=1408):
    """the MoE group matmul at a decode-sized batch: T tokens routed Zipf(1.1) over G experts, W [G, N, K] rotating;
    rate = the used experts' weight bytes per call"""
    rng = np.random.default_rng(4)
    p = 1.0 / (np.arange(1, G + 1) ** 1.1)
    counts = rng.multinomial(T, p / p.sum())
    offsets = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    R = rotation(G * K * N)
    x = torch.randint(-127, 128, (T, K), generator=g, device="cuda", dtype=torch.int8)
    ws = [torch.randint(-127, 128, (G, N, K), generator=g, device="cuda", dtype=torch.int8) for _ in range(R)]
    pts = torch.rand(T, generator=g, device="cuda") * 0.01
    scale = torch.rand((G, N), generator=g, device="cuda") * 0.01
    y = torch.empty((T, N), dtype=torch.bfloat16, device="cuda")

    def fn(i):
        ascq.quant_group_matmul(x, pts, ws[i % R], scale, offsets, 0, out=y, w_trans=True)

    ms, eager = _time_graph(torch, fn, iters, y)
    used = int((counts > 0).sum())
    gbs = used * K * N / (ms * 1e-3) / 1e9
    return dict(workload=f"MoE quant group matmul, decode batch: {T} tokens over {G} experts Zipf(1.1) ({used} used), "
                         f"K={K} N={N}, W [G,N,K], bf16 out", ms=ms, value=round(gbs, 1), unit="GB/s",
                frac_of_peak=gbs / HBM_PEAK_GBS, timing="HIP graph of the calls (weights rotating), replayed"
                if USE_GRAPH else "eager calls", eager_ms=eager)


DECODE_SHAPES = [(4096, 11008), (11008, 4096), (8192, 8192)]


# model shapes of the weight-only matmul (attention and MLP projections of 7B / 13B / 70B-class models), opt-in:
# `--only shapes`
WO_SHAPES = [(4096, 4096), (4096, 11008), (11008, 4096), (5120, 13824), (13824, 5120), (8192, 8192), (8192, 28672),
             (28672, 8192)]


def bench_group(torch, ascq, iters, w_trans=False):
    G, T, K, N = 16, 4096, 4096, 1408
    rng = np.random.default_rng(4)
    p = 1.0 / (np.arange(1, G + 1) ** 1.1)
    counts = rng.multinomial(T, p / p.sum())
    offsets = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    per = T * K + G * K * N + 2 * T * N
    R = rotation(per)
    xs = [torch.randint(-127, 128, (T, K), generator=g, device="cuda", dtype=torch.int8) for _ in range(R)]
    wshape = (G, N, K) if w_trans else (G, K, N)
    ws = [torch.randint(-127, 128, wshape, generator=g, device="cuda", dtype=torch.int8) for _ in range(R)]
    pts = torch.rand(T, generator=g, device="cuda") * 0.01
    scale = torch.rand((G, N), generator=g, device="cuda") * 0.01
    y = torch.empty((T, N), dtype=torch.bfloat16, device="cuda")

    def fn(i):
        r = i % R
        ascq.quant_group_matmul(xs[r], pts, ws[r], scale, offsets, 0, out=y, w_trans=w_trans)

    ms = _time_loop(torch, fn, iters)
    ops = 2 * T * K * N
    nbytes = T * K + 4 * T + G * K * N + 4 * G * N + 2 * T * N + 8 * (G + 1)
    tops = ops / (ms * 1e-3) / 1e12
    attainable = min(INT8_PEAK_TOPS, ops / nbytes * HBM_PEAK_GBS / 1e3)
    return dict(workload=f"MoE quant group matmul, {G} experts Zipf(1.1), T={T} K={K} N={N}, bf16 out, W given "
                         + ("[G,N,K] (K-contiguous, pre-formatted)" if w_trans else "[G,K,N]"),
                ms=ms, value=tops, unit="TOPS", frac_of_peak=tops / INT8_PEAK_TOPS,
                frac_of_attainable=tops / attainable, gbs=nbytes / (ms * 1e-3) / 1e9,
                group_counts=[int(c) for c in counts])


def _mx_fp4_normal(torch, R, K, g):
    """N(0, 1) [R, K] MX-quantised on the GPU with torch ops (data generation only): per 32-element block the
    shared exponent e = floor(log2(absmax)) - 2 (E2M1's largest binade), codes = E2M1 nearest of x / 2^e (ties
    to the even code), clamped to 6.  Returns packed [R, K/2] codes (even k low nibble) and scales [R, K/32]."""
    x = torch.randn((R, K // 32, 32), generator=g, device="cuda")
    amax = x.abs().amax(-1, keepdim=True).clamp_min(2.0 ** -126)
    e = torch.floor(torch.log2(amax)) - 2
    v = (x / torch.exp2(e)).abs().clamp_max(6.0)
    mags = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], device="cuda")
    mids = (mags[1:] + mags[:-1]) / 2
    idx = torch.bucketize(v, mids)  # v on midpoint j gets the lower code j ...
    tie = (idx < 7) & (v == mids[idx.clamp_max(6)])
    idx = torch.where(tie & (idx % 2 == 1), idx + 1, idx)  # ... or j + 1 when that is the even one
    code = (idx | torch.where(x < 0, 8, 0)).to(torch.uint8).reshape(R, K)
    packed = (code[:, 0::2] | (code[:, 1::2] << 4)).contiguous()
    scales = (e.reshape(R, K // 32) + 127).to(torch.uint8).contiguous()
    return packed, scales


def bench_mx(torch, ascq, iters, trans_b=True):
    M = N = K = 8192
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    A, sA = _mx_fp4_normal(torch, M, K, g)
    B, sB = _mx_fp4_normal(torch, N, K, g)
    if not trans_b:  # [N, K/2] packed along K -> [K, N/2] packed along N
        nib = torch.stack([B & 0xF, B >> 4], -1).reshape(N, K).t().contiguous()
        B = (nib[:, 0::2] | (nib[:, 1::2] << 4)).contiguous()
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    mm = ascq.Matmul(ascq.FP4_E2M1, ascq.FP4_E2M1, ascq.BF16, 0, ascq.E8M0)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(A)
    mm.SetTensorB(B, trans_b)
    mm.SetTensorScaleA(sA, False)
    mm.SetTensorScaleB(sB, True)

    def fn(i):
        mm.IterateAll(C)

    ms = _time_loop(torch, fn, iters, warmup=2)
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    return dict(workload=f"MX-FP4 E2M1/E8M0 GEMM {M}x{N}x{K}, N(0,1) MX-quantised, fp32 acc, bf16 out, B given "
                         + ("[N,K] (isTransposeB)" if trans_b else "[K,N] (transposed on the fly)"),
                ms=ms, value=tf, unit="TFLOPS", frac_of_peak=tf / MXFP4_PEAK_TFLOPS)


# the reference's published figures for its own two high-performance samples (Ascend 950PR, msprof)
REF_MX_E1M2_US = 693.283      # matmul_mxfp4_high_performance/README_en.md:177 (Case 2)
REF_GROUP_GELU_US = 204.129   # quant_group_matmul_high_performance/README_en.md:368 (scenario 2)


def bench_mx_e1m2_sample(torch, ascq, iters):
    """The reference's high-performance MX sample (matmul_mxfp4_high_performance): A [8192, 8192] and B given
    [K, N] = [8192, 8192], fp4x2_e1m2_t from randint(-1, 2), E8M0 scales randint(127, 130) (B's [sK/2, N, 2]),
    fp32 accumulation, bf16 out.  One IterateAll: B transpose, fp4 -> fp6 planes of both operands, scale
    rearrangement and the fp6 MFMA GEMM."""
    M = N = K = 8192
    g = torch.Generator(device="cuda")
    g.manual_seed(8)
    lut = torch.tensor([0xC, 0x0, 0x4], dtype=torch.uint8, device="cuda")  # e1m2 codes of -1, 0, 1
    a = lut[torch.randint(0, 3, (M, K), generator=g, device="cuda")]
    b = lut[torch.randint(0, 3, (K, N), generator=g, device="cuda")]
    A = (a[:, 0::2] | (a[:, 1::2] << 4)).contiguous()
    B = (b[:, 0::2] | (b[:, 1::2] << 4)).contiguous()
    del a, b
    sK = K // 32
    sA = torch.randint(127, 130, (M, sK), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8)
    sB = torch.randint(127, 130, (sK // 2, N, 2), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8)
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    mm = ascq.Matmul(ascq.FP4_E1M2, ascq.FP4_E1M2, ascq.BF16, 0, ascq.E8M0)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(A)
    mm.SetTensorB(B, False)
    mm.SetTensorScaleA(sA, False)
    mm.SetTensorScaleB(sB, False)

    def fn(i):
        mm.IterateAll(C)

    ms = _time_loop(torch, fn, iters, warmup=2)
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    return dict(workload=f"reference MX sample: fp4x2_e1m2 MX GEMM {M}x{N}x{K} (randint(-1,2) elements, scales "
                         "127-129), B given [K,N], bf16 out; the whole IterateAll (B transpose, fp6 planes, scales, "
                         "GEMM)", ms=ms, value=tf, unit="TFLOPS", frac_of_peak=tf / MXFP4_PEAK_TFLOPS,
                reference_us=REF_MX_E1M2_US, speedup_vs_reference=REF_MX_E1M2_US / (ms * 1e3))


def bench_group_sample(torch, ascq, iters):
    """The reference's QuantGroupMatmul sample (quant_group_matmul_high_performance, scenario 2): M = 8192 tokens
    in 8 equal groups, K = 1024, N = 8192, int8 x and NZ int8 weights [8, 1024, 8192], f32 per-token and
    per-channel scales, FasterGelu, f16 out.  The NZ weights are re-laid [G, N, K] once outside the timed loop
    (weights are static; the reference's NZ layout is itself prepared offline)."""
    G, M, K, N = 8, 8192, 1024, 8192
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    x = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
    w = torch.randint(-127, 128, (G, K, N), generator=g, device="cuda", dtype=torch.int8)
    w_nz = w.reshape(G, K // 16, 16, N // 32, 32).permute(0, 3, 1, 2, 4).contiguous()  # gen_data.py:62
    del w
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    wt = ascq.nz_to_nd(w_nz.view(torch.uint8).reshape(-1), ascq.INT8, G, K, N, transpose_out=True).view(torch.int8)
    torch.cuda.synchronize()
    relayout_ms = (time.perf_counter() - t0) * 1e3
    pts = torch.rand(M, generator=g, device="cuda") * 0.01
    scale = torch.rand((G, N), generator=g, device="cuda") * 0.01
    counts = torch.full((G,), M // G, dtype=torch.int64, device="cuda")
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")

    def fn(i):
        ascq.quant_group_matmul(x, pts, wt, scale, counts, 1, out=y, w_trans=True, out_dtype=torch.float16,
                                activation=ascq.ACT_FASTER_GELU)

    ms = _time_loop(torch, fn, iters)
    ops = 2 * M * K * N
    tops = ops / (ms * 1e-3) / 1e12
    nbytes = M * K + 4 * M + G * K * N + 4 * G * N + 2 * M * N + 8 * G
    attainable = min(INT8_PEAK_TOPS, ops / nbytes * HBM_PEAK_GBS / 1e3)
    return dict(workload=f"reference QuantGroupMatmul sample: M={M} in {G} equal groups, K={K}, N={N}, NZ int8 "
                         "weights (re-laid [G,N,K] once), per-token x per-channel f32 scales, FasterGelu, f16 out",
                ms=ms, value=tops, unit="TOPS", frac_of_peak=tops / INT8_PEAK_TOPS,
                frac_of_attainable=tops / attainable, nz_relayout_ms_once=relayout_ms,
                reference_us=REF_GROUP_GELU_US, speedup_vs_reference=REF_GROUP_GELU_US / (ms * 1e3))


def _fp8_bytes(torch, shape, g, dt):
    """N(0, 1) cast to fp8 (no NaN codes), as raw bytes"""
    return torch.randn(shape, generator=g, device="cuda").to(dt).view(torch.uint8)


def bench_fp8(torch, ascq, iters, trans_b=True):
    """fp8 e4m3 x e4m3 Matmul 8192^3, fp32 accumulation, per-channel QF322BF16_PRE -> bf16"""
    M = N = K = 8192
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    A = _fp8_bytes(torch, (M, K), g, torch.float8_e4m3fn)
    B = _fp8_bytes(torch, (N, K) if trans_b else (K, N), g, torch.float8_e4m3fn)
    words = torch.full((N,), 0x3C000000, dtype=torch.int64, device="cuda")  # M1 = 2^-7
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    mm = ascq.Matmul(ascq.FP8_E4M3, ascq.FP8_E4M3, ascq.BF16)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(A)
    mm.SetTensorB(B, trans_b)
    mm.SetQuantVector(words)

    def fn(i):
        mm.IterateAll(C)

    ms = _time_loop(torch, fn, iters, warmup=2)
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    return dict(workload=f"fp8 e4m3 Matmul {M}x{N}x{K}, fp32 acc, per-channel QF322BF16_PRE -> bf16, B given "
                         + ("[N,K] (isTransposeB)" if trans_b else "[K,N] (transposed into the workspace)"),
                ms=ms, value=tf, unit="TFLOPS", frac_of_peak=tf / FP8_PEAK_TFLOPS)


def bench_vendor(torch, kind, iters):
    """The vendor BLAS on the same box and shape, for scale (not this library): hipBLASLt through torch._int_mm (int8,
    int32 out) and torch._scaled_mm (fp8 e4m3, per-tensor scales, bf16 out), M = N = K = 8192, B given [N, K]."""
    M = N = K = 8192
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    if kind == "int8":
        A = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
        B = torch.randint(-127, 128, (N, K), generator=g, device="cuda", dtype=torch.int8)

        def fn(i):
            torch._int_mm(A, B.t())

        name, peak, unit = "hipBLASLt int8 GEMM (torch._int_mm)", INT8_PEAK_TOPS, "TOPS"
    else:
        A = torch.randn((M, K), generator=g, device="cuda").to(torch.float8_e4m3fn)
        B = torch.randn((N, K), generator=g, device="cuda").to(torch.float8_e4m3fn)
        one = torch.ones((), device="cuda")

        def fn(i):
            torch._scaled_mm(A, B.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)

        name, peak, unit = "hipBLASLt fp8 e4m3 GEMM (torch._scaled_mm), bf16 out", FP8_PEAK_TFLOPS, "TFLOPS"
    ms = _time_loop(torch, fn, iters, warmup=2)
    v = 2 * M * N * K / (ms * 1e-3) / 1e12
    return dict(workload=f"vendor reference: {name} {M}x{N}x{K}, B given [N,K]", ms=ms, value=v, unit=unit,
                frac_of_peak=v / peak)


def bench_mxfp8(torch, ascq, iters):
    """MX-FP8 (e4m3 elements, E8M0 per 32 K) GEMM 8192^3 -> bf16"""
    M = N = K = 8192
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    A = _fp8_bytes(torch, (M, K), g, torch.float8_e4m3fn)
    B = _fp8_bytes(torch, (N, K), g, torch.float8_e4m3fn)
    sA = torch.randint(124, 129, (M, K // 32), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8)
    sB = torch.randint(124, 129, (N, K // 32), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8)
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    mm = ascq.Matmul(ascq.FP8_E4M3, ascq.FP8_E4M3, ascq.BF16, 0, ascq.E8M0)
    mm.SetOrgShape(M, N, K)
    mm.SetTensorA(A)
    mm.SetTensorB(B, True)
    mm.SetTensorScaleA(sA, False)
    mm.SetTensorScaleB(sB, True)

    def fn(i):
        mm.IterateAll(C)

    ms = _time_loop(torch, fn, iters, warmup=2)
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    return dict(workload=f"MX-FP8 e4m3/E8M0 GEMM {M}x{N}x{K}, fp32 acc, bf16 out, B given [N,K]",
                ms=ms, value=tf, unit="TFLOPS", frac_of_peak=tf / FP8_PEAK_TFLOPS)


def traffic_probe(torch, ascq):
    """One launch each of a plain 256 MiB copy (the calibration for FETCH_SIZE / WRITE_SIZE), the dynamic
    quant kernel and the dequant kernel on the 8192 x 8192 f16 workload, with a 1 GiB fill between them so
    the Infinity Cache holds none of the next kernel's inputs.  Meant to run under rocprofv3 --pmc."""
    M = N = 8192
    x = torch.randn((M, N), device="cuda").half()
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    src = torch.randint(0, 255, (256 << 20,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    flush.fill_(1)
    dst.copy_(src)
    flush.fill_(2)
    q, s = ascq.quant_dynamic_per_token(x)
    flush.fill_(3)
    ascq.ascend_dequant_policy(q, s, ascq.PER_TOKEN, torch.float16)
    torch.cuda.synchronize()
    return {"traffic_probe": "copy 268435456 B, quant f16 8192x8192, dequant int8 8192x8192 -> f16"}


def bench_quant_policy(torch, ascq, dst_type, policy, iters, k_dim=1, g=128, round_mode=None):
    """AscendQuant policy form over an f16 [8192, 8192] activation: PER_GROUP (group 128 along the rows) or
    PER_TOKEN, f16 scales, to int8 / fp8 / fp4 E2M1 / E1M2 (round_mode: rint unless given)"""
    fp4 = dst_type in (ascq.FP4_E2M1, ascq.FP4_E1M2)
    mode = ascq.ROUND_RINT if round_mode is None else round_mode
    M = N = 8192
    out_b = M * N // 2 if fp4 else M * N
    ss = (M,) if policy == ascq.PER_TOKEN else ((M, N // g) if k_dim == 1 else (M // g, N))
    nbytes = 2 * M * N + out_b + 2 * int(np.prod(ss))
    R = rotation(nbytes)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    xs = [torch.randn((M, N), generator=gen, device="cuda").half() for _ in range(R)]
    # scales that keep |x * s| of N(0,1) data mostly inside the output format (E2M1 to +-6, E1M2 to +-1.75), so the
    # fp4 encoders see in-range values rather than saturating ones
    lo, hi = {ascq.FP4_E2M1: (0.5, 1.5), ascq.FP4_E1M2: (0.2, 0.45)}.get(dst_type, (0.5, 8.0))
    sc = torch.empty(ss, device="cuda").uniform_(lo, hi, generator=gen).half()
    shape = (M, N // 2) if fp4 else (M, N)
    qs = [torch.empty(shape, dtype=torch.uint8, device="cuda") for _ in range(R)]

    def fn(i):
        ascq.ascend_quant_policy(xs[i % R], sc, policy, dst_type, g if policy == ascq.PER_GROUP else 0, k_dim=k_dim,
                                 round_mode=mode, out=qs[i % R])

    ms = _time_loop(torch, fn, iters)
    gbs = nbytes / (ms * 1e-3) / 1e9
    name = {ascq.INT8: "int8", ascq.FP8_E4M3: "fp8_e4m3", ascq.FP4_E2M1: "E2M1", ascq.FP4_E1M2: "E1M2"}[dst_type]
    if round_mode is not None:
        name += {ascq.ROUND_RINT: " rint", ascq.ROUND_FLOOR: " floor", ascq.ROUND_CEIL: " ceil",
                 ascq.ROUND_ROUND: " round", ascq.ROUND_TRUNC: " trunc"}[round_mode]
    pol = "PER_TOKEN" if policy == ascq.PER_TOKEN else f"PER_GROUP g={g} kDim={k_dim}"
    sr = f"f16 scales in [{lo}, {hi}]"
    return dict(workload=f"AscendQuant {pol} f16 [{M},{N}] -> {name} ({sr})", ms=ms, value=gbs, unit="GB/s",
                frac_of_peak=gbs / HBM_PEAK_GBS)


def bench_antiquant_policy(torch, ascq, src_type, iters):
    """AscendAntiQuant policy form to an f16 / bf16 [8192, 8192] output: int8 with f16 scales and offsets in groups of
    128 rows (kDim 0), or fp4 E2M1 with E8M0 scales in groups of 32 along the rows"""
    M = N = 8192
    gen = torch.Generator(device="cuda")
    gen.manual_seed(6)
    if src_type in (ascq.FP4_E2M1, ascq.FP4_E1M2):
        g, sb, ss = 32, M * N // 2, (M, N // 32)
        sc = torch.randint(110, 140, ss, generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8)
        fname = "E2M1" if src_type == ascq.FP4_E2M1 else "E1M2"
        of, st, kd, dt, name = None, ascq.E8M0, 1, torch.bfloat16, f"fp4 {fname} (E8M0 scales, g=32 kDim=1) -> bf16"
        nbytes = sb + M * N // 32 + 2 * M * N
    else:
        g, sb, ss = 128, M * N, (M // 128, N)
        sc = torch.empty(ss, device="cuda").uniform_(0.01, 1.0, generator=gen).half()
        of = torch.empty(ss, device="cuda").uniform_(-4.0, 4.0, generator=gen).half()
        st, kd, dt, name = ascq.F16, 0, torch.float16, "int8 (f16 scale + offset, g=128 kDim=0) -> f16"
        nbytes = sb + 4 * (M // 128) * N + 2 * M * N
    R = rotation(nbytes)
    srcs = [torch.randint(0, 256, (sb,), generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8)
            for _ in range(R)]
    ys = [torch.empty((M, N), dtype=dt, device="cuda") for _ in range(R)]

    def fn(i):
        ascq.ascend_antiquant_policy(srcs[i % R], src_type, sc, st, ascq.PER_GROUP, M, N, g, of, kd, False, dt,
                                     out=ys[i % R])

    ms = _time_loop(torch, fn, iters)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(workload=f"AscendAntiQuant PER_GROUP [{M},{N}] {name}", ms=ms, value=gbs, unit="GB/s",
                frac_of_peak=gbs / HBM_PEAK_GBS)


def bench_quant_legacy(torch, ascq, iters):
    """legacy AscendQuant (half arithmetic) of an f16 [8192, 8192] tensor with per-channel f16 scale and offset
    vectors of 8192 entries"""
    M = N = 8192
    nbytes = 2 * M * N + M * N + 4 * N
    R = rotation(nbytes)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    xs = [torch.randn((M, N), generator=gen, device="cuda").half() for _ in range(R)]
    qs = [torch.empty((M, N), dtype=torch.int8, device="cuda") for _ in range(R)]
    sc = torch.empty(N, device="cuda").uniform_(0.5, 40.0, generator=gen).half()
    of = torch.empty(N, device="cuda").uniform_(-1.0, 1.0, generator=gen).half()

    def fn(i):
        ascq.ascend_quant(xs[i % R], scale=sc, offset=of, out=qs[i % R])

    ms = _time_loop(torch, fn, iters)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(workload=f"AscendQuant legacy per-channel (half arithmetic) f16 [{M},{N}] -> int8", ms=ms, value=gbs,
                unit="GB/s", frac_of_peak=gbs / HBM_PEAK_GBS)


def bench_antiquant_legacy(torch, ascq, iters):
    """legacy AscendAntiQuant of the antiquant matmul workload's weight: int4 [4096, 11008] with f16 scale and offset
    per 128 rows, to f16 in half arithmetic"""
    K, N, g = 4096, 11008, 128
    nbytes = K * N // 2 + 2 * 2 * (K // g) * N + 2 * K * N
    R = rotation(nbytes)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(8)
    ws = [torch.randint(0, 256, (K * N // 2,), generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8)
          for _ in range(R)]
    ys = [torch.empty((K, N), dtype=torch.float16, device="cuda") for _ in range(R)]
    sc = torch.empty((K // g, N), device="cuda").uniform_(0.001, 0.1, generator=gen).half()
    of = torch.empty((K // g, N), device="cuda").uniform_(-8.0, 8.0, generator=gen).half()

    def fn(i):
        ascq.ascend_antiquant(ws[i % R], ascq.INT4, sc, of, K, N, g, False, torch.float16, ascq.ARITH_F16, out=ys[i % R])

    ms = _time_loop(torch, fn, iters)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(workload=f"AscendAntiQuant legacy int4 [{K},{N}] g={g} -> f16 (half arithmetic)", ms=ms, value=gbs,
                unit="GB/s", frac_of_peak=gbs / HBM_PEAK_GBS)


def bench_dequant_channel(torch, ascq, iters):
    """AscendDequant (legacy form) of an int32 [8192, 8192] accumulator with a per-channel uint64 deqScale (fp32
    in the low word) to f16 -- the legacy form's f16-output combination"""
    M = N = 8192
    nbytes = 4 * M * N + 2 * M * N + 8 * N
    R = rotation(nbytes)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(9)
    xs = [torch.randint(-(1 << 20), 1 << 20, (M, N), generator=gen, device="cuda", dtype=torch.int32) for _ in range(R)]
    ys = [torch.empty((M, N), dtype=torch.float16, device="cuda") for _ in range(R)]
    sc = torch.empty(N, device="cuda").uniform_(1e-4, 1e-2, generator=gen).view(torch.int32).to(torch.int64)

    def fn(i):
        ascq.ascend_dequant(xs[i % R], sc, torch.float16, out=ys[i % R])

    ms = _time_loop(torch, fn, iters)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(workload=f"AscendDequant per-channel int32 [{M},{N}] -> f16 (uint64 deqScale)", ms=ms, value=gbs,
                unit="GB/s", frac_of_peak=gbs / HBM_PEAK_GBS)


OTHER = {
    "quant": [lambda t, a: bench_dequant_channel(t, a, 50),lambda t, a: bench_antiquant_legacy(t, a, 100),lambda t, a: bench_quant_legacy(t, a, 50),lambda t, a: bench_antiquant_policy(t, a, a.INT8, 50),
              lambda t, a: bench_antiquant_policy(t, a, a.FP4_E2M1, 50),lambda t, a: bench_quant_policy(t, a, a.INT8, a.PER_GROUP, 50),
              lambda t, a: bench_quant_policy(t, a, a.INT8, a.PER_GROUP, 50, k_dim=0),
              lambda t, a: bench_quant_policy(t, a, a.FP8_E4M3, a.PER_TOKEN, 50),
              lambda t, a: bench_quant_policy(t, a, a.FP4_E2M1, a.PER_GROUP, 50),
              lambda t, a: bench_quant_policy(t, a, a.FP4_E2M1, a.PER_GROUP, 50, round_mode=a.ROUND_FLOOR),
              lambda t, a: bench_quant_policy(t, a, a.FP4_E1M2, a.PER_GROUP, 50),
              lambda t, a: bench_antiquant_policy(t, a, a.FP4_E1M2, 50)],
    "w8a8": [lambda t, a: bench_w8a8(t, a, 128, 256, 512, 200), lambda t, a: bench_w8a8(t, a, 8192, 8192, 8192, 10)],
    "gemv": [lambda t, a, w=w, m=m: bench_gemv(t, a, getattr(a, w), m, 200)
             for w in ("INT4", "INT8") for m in (1, 16, 64)]
            + [lambda t, a, w=w: bench_prefill(t, a, getattr(a, w), 512, 20) for w in ("INT4", "INT8")],
    "group": [lambda t, a: bench_group(t, a, 20, True), lambda t, a: bench_group(t, a, 20, False),
              lambda t, a: bench_group_sample(t, a, 20)],
    "vendor": [lambda t, a: bench_vendor(t, "int8", 10), lambda t, a: bench_vendor(t, "fp8", 10)],
    "mx": [lambda t, a: bench_mx(t, a, 10, True), lambda t, a: bench_mx(t, a, 5, False),
           lambda t, a: bench_mx_e1m2_sample(t, a, 10)],
    "fp8": [lambda t, a: bench_fp8(t, a, 10, True), lambda t, a: bench_fp8(t, a, 5, False),
            lambda t, a: bench_mxfp8(t, a, 10)],
    "shapes": [lambda t, a, k=k, n=n, m=m: bench_wo_shape(t, a, k, n, m, 50 if m < 512 else 10)
               for k, n in WO_SHAPES for m in (1, 16, 64, 512)],
    "decode": [lambda t, a, kd=kd, k=k, n=n, m=m: bench_decode_matmul(t, a, kd, k, n, m)
               for kd in ("int8", "fp8", "mxfp4") for k, n in DECODE_SHAPES for m in (1, 16, 64)]
              + [lambda t, a, kd=kd, k=k, n=n, m=m: bench_decode_matmul(t, a, kd, k, n, m, trans_b=False)
                 for kd in ("int8", "fp8") for k, n in DECODE_SHAPES for m in (1, 64)]
              + [lambda t, a, tk=tk: bench_group_decode(t, a, tk) for tk in (16, 64, 256)],
}


def _with_roofline(r):
    """the roofline object of a GPU record: MFMA-bound GEMMs against their dense peak, HBM-bound ops against
    8 TB/s; the group matmul against its attainable min(peak, AI x HBM)"""
    if "value" not in r or "unit" not in r:
        return r
    if "frac_of_attainable" in r:
        peak = r["value"] / r["frac_of_attainable"]
        r["roofline"] = _roof("hbm" if peak < INT8_PEAK_TOPS - 1e-6 else "mfma", r["value"], round(peak, 2), r["unit"])
    elif "frac_of_peak" in r:
        r["roofline"] = _roof("hbm" if r["unit"] == "GB/s" else "mfma", r["value"], round(r["value"] / r["frac_of_peak"], 2),
                              r["unit"])
    return r


# CPU baselines of the benchmark workload families: (family, index in OTHER[family]) -> oracle timing
CPU_FOR = {
    ("w8a8", 0): lambda: cpu_baseline_w8a8(128, 256, 512),
    ("w8a8", 1): lambda: cpu_baseline_w8a8(8192, 8192, 8192),
    ("gemv", 0): lambda: cpu_baseline_gemv(4, 1), ("gemv", 1): lambda: cpu_baseline_gemv(4, 16),
    ("gemv", 2): lambda: cpu_baseline_gemv(4, 64), ("gemv", 3): lambda: cpu_baseline_gemv(8, 1),
    ("gemv", 4): lambda: cpu_baseline_gemv(8, 16), ("gemv", 5): lambda: cpu_baseline_gemv(8, 64),
    ("group", 0): cpu_baseline_group, ("group", 1): cpu_baseline_group,
    ("mx", 0): cpu_baseline_mx, ("mx", 1): cpu_baseline_mx,
}


def run_others(torch, ascq, which, with_cpu=False):
    out, cpu_cache = [], {}
    for key in (["quant", "w8a8", "gemv", "group", "mx", "fp8", "vendor"] if which == "all" else [which]):
        for idx, fn in enumerate(OTHER[key]):
            try:
                r = _with_roofline(fn(torch, ascq))
                rec = {k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()}
            except Exception as e:  # report, do not hide
                rec = {"error": repr(e)}
            torch.cuda.empty_cache()
            cf = CPU_FOR.get((key, idx)) if with_cpu else None
            if cf is not None:
                try:
                    if cf not in cpu_cache:
                        cpu_cache[cf] = cf()
                    rec["cpu_baseline"] = cpu_cache[cf]
                except Exception as e:
                    rec["cpu_baseline"] = {"error": repr(e)}
            out.append(rec)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-graph", action="store_true",
                    help="time the launch-bound lines (decode GEMV, the W8A8 sample) eagerly, without a HIP graph")
    ap.add_argument("--only", default="all",
                    choices=["all", "headline", "quant", "w8a8", "gemv", "group", "mx", "fp8", "vendor", "traffic",
                             "shapes", "decode"],
                    help="run one workload family (the JSON contract line is printed for all / headline)")
    args = ap.parse_args()
    global USE_GRAPH
    USE_GRAPH = not args.no_graph
    if args.gpus != 1:
        print(json.dumps({"error": "this library targets one MI355X; run with --gpus 1 (no multi-GPU path exists)"}))
        return 2

    import torch

    import ascq

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.init()
    if args.only == "traffic":
        print(json.dumps(traffic_probe(torch, ascq)))
        return 0
    if args.only in ("quant", "w8a8", "gemv", "group", "mx", "fp8", "vendor", "shapes", "decode"):
        print(json.dumps({"other_configs": run_others(torch, ascq, args.only, with_cpu=not args.no_cpu)}))
        return 0
    h = bench_headline(torch, ascq, args.steps, args.warmup)
    step_ms = h["total_ms"] / args.steps
    step_bytes = h["bytes_quant"] + h["bytes_dequant"]
    value = step_bytes / (step_ms * 1e-3) / 1e9
    traffic = parse_traffic().get("quant_dyn_row_f16_8192x8192")
    q_gbs = h["bytes_quant"] / (h["q_ms"] * 1e-3) / 1e9
    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16->int8 (fp32 scale arithmetic)",
        "data": "synthetic: N(0,1) f16 with 0.1% outliers x50, seeded; "
                f"{h['R']} rotating input/output sets (> 256 MB Infinity Cache)",
        "config": {"workload": "AscendQuant per-token dynamic quant f16 [8192,8192] -> int8 + fp32 scale[8192], "
                               "then AscendDequant -> f16", "rows": h["M"], "cols": h["N"],
                   "round_mode": "rint", "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(q_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(q_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "quant_dyn_row_kernel (AscendQuant per-token dynamic)",
                     "algorithmic_bytes_per_launch": h["bytes_quant"], "avg_launch_ms": round(h["q_ms"], 5),
                     "timed_launches": h["q_samples"],
                     "timing": "HIP events on the launch stream around back-to-back launches of this kernel alone"},
        "dequant_kernel": {"achieved": round(h["bytes_dequant"] / (h["d_ms"] * 1e-3) / 1e9, 2), "unit": "GB/s",
                           "avg_launch_ms": round(h["d_ms"], 5)},
    }
    if args.only == "all":
        rec["other_configs"] = run_others(torch, ascq, "all", with_cpu=not args.no_cpu)
    if not args.no_cpu:
        rec["cpu_baseline"] = cpu_baseline_headline()
    print(json.dumps(rec))
    return 0


if __name__ == "__main__":
    sys.exit(main())
