"""Weight-only antiquant matmul captured in a HIP graph: every replay, with eager work and synchronisations between
the replays, equals the eager call bit for bit (the decode-loop use of the entry point; it records no memset, no
allocation and no host synchronisation, so the calls capture as plain kernel nodes)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("w_type", ["int4", "int8"])
@pytest.mark.parametrize("M", [1, 16, 32, 64])
def test_antiquant_matmul_graph_replays(ascq_gpu, w_type, M):
    rng = seeded(4000 + M)
    K, N, g = 1024, 1008, 128
    at = ascq_gpu.INT8 if w_type == "int8" else ascq_gpu.INT4
    wb = K * N // (1 if w_type == "int8" else 2)
    w = torch.from_numpy(rng.integers(0, 256, wb, dtype=np.uint8)).cuda()
    wp = ascq_gpu.weight_pack(w, at, K, N)
    scale = torch.from_numpy(np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), (K // g, N))).astype(np.float16)).cuda()
    offset = torch.from_numpy(rng.uniform(-8, 8, (K // g, N)).astype(np.float16)).cuda()
    xs = [torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).cuda() for _ in range(2)]
    ys = [torch.empty((M, N), dtype=torch.float16, device="cuda") for _ in range(2)]
    eager = [ascq_gpu.antiquant_matmul(xs[i], wp, at, scale, offset, g, N) for i in range(2)]
    torch.cuda.synchronize()

    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(graph, stream=st):
            for i in range(2):
                ascq_gpu.antiquant_matmul(xs[i], wp, at, scale, offset, g, N, out=ys[i])
    torch.cuda.current_stream().wait_stream(st)
    for rep in range(4):
        for y in ys:
            y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(ys[i], eager[i]), f"replay {rep}, call {i} differs from the eager result"
        # eager work between replays, on the same buffers the graph reads
        ascq_gpu.antiquant_matmul(xs[1], wp, at, scale, offset, g, N, out=ys[0])
        torch.cuda.synchronize()
    del graph
