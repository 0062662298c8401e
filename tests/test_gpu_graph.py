"""The forward path under HIP graph capture.

A decode loop that cannot afford a host launch per Linear captures its
forwards in a graph and replays it.  Every forward kernel route here
(GEMV at M = 1, 4 and 16, row-blocked decode, chunked-staging decode,
prefill tiles, a multi-matrix launch, and the compressed Linear module)
allocates nothing of its own and records no memset, so it captures as it
is.  Each graph is replayed several times with the program's own eager
work and synchronizations between the replays, and every replay must
reproduce the eager output bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REPLAYS = 4


@pytest.fixture(scope="module")
def native():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mlbricks_amd.elasticbit._native as native   # fails loudly when the library is missing
    return native


def _matrix(native, rows, cols, b, seed):
    rng = np.random.default_rng(seed)
    qm = (1 << (b - 1)) - 1
    q = rng.integers(-qm, qm + 1, size=(rows, cols)).astype(np.int16)
    s = rng.uniform(0.002, 0.05, size=rows).astype(np.float32)
    return native.RuntimeMatrix._compressSelectedCodes(q, s, b, 0.01, 0.0), rng


def _replay_matches(graph, out, expected):
    for i in range(REPLAYS):
        out.fill_(float("nan"))                         # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected), i


@pytest.mark.parametrize("rows,cols,b,M", [
    (4096, 4096, 10, 1),       # GEMV, M = 1
    (4096, 4096, 10, 4),       # GEMV, M = 2..4
    (4096, 4096, 10, 16),      # GEMV, M = 5..16
    (11008, 4096, 10, 16),     # row-blocked decode
    (4096, 11008, 10, 16),     # decode kernel, chunked activation staging
    (4096, 4096, 16, 1),       # raw fp16 GEMV
    (4096, 4096, 13, 8),       # decoded-fp16 decode kernel
    (2048, 1024, 10, 300),     # prefill, 128-row tiles
    (4096, 4096, 10, 2048),    # prefill, 256 x 256 tiles
])
def test_forward_replays_from_a_graph(native, rows, cols, b, M):
    if b == 16:
        rng = np.random.default_rng(rows + M)
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        m = native.RuntimeMatrix._compressSelected(w, 16, 0.01, 0.0)
    else:
        m, rng = _matrix(native, rows, cols, b, rows + M)
    x = torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float16)).cuda()
    bias = torch.from_numpy(rng.standard_normal(rows).astype(np.float16)).cuda()
    expected = m.forwardTorch(x, bias=bias)
    out = torch.empty_like(expected)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        m.forwardTorch(x, bias=bias, out=out)          # warm on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        m.forwardTorch(x, bias=bias, out=out)
    _replay_matches(graph, out, expected)


def test_multi_matrix_forward_replays_from_a_graph(native):
    mats = [_matrix(native, rows, 4096, 10, rows)[0] for rows in (4096, 1024, 1000)]
    x = torch.randn(3, 4096, generator=torch.Generator().manual_seed(5)).half().cuda()
    expected = [mm.forwardTorch(x) for mm in mats]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = native.forward_torch_multi(mats, x, None)
    for i in range(REPLAYS):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for j, (o, e) in enumerate(zip(outs, expected)):
            assert torch.equal(o, e), (i, j)


def test_compressed_linear_module_replays_from_a_graph():
    """The module forward once its route is frozen (as a decode loop runs
    it): the output lives in the graph's memory pool."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mlbricks_amd import ElasticBit

    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(1024, 2048), torch.nn.Linear(2048, 1024)).cuda().half().eval()
    ElasticBit.compress(model, torch.randn(32, 1024).half(), 0.01)
    x = torch.randn(1, 1024, device="cuda").half()
    with torch.inference_mode():
        for _ in range(3):
            expected = model(x)                       # qualifies and freezes the routes
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = model(x)
        _replay_matches(graph, out, expected)
