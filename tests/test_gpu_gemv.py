"""GPU parity of the GEMV kernel at M = 2..16 (linear_gemv_kernel<B, MODE, 4 or 16>).

The launcher sends M = 2..16 to the GEMV kernel when K is a whole number of
128-column tiles from 2176 to 4096 (above eight rows only at K = 4096), x is
16-byte aligned, the arithmetic is the integer-code dot product at b != 11
(b <= 7 up to 256 row tiles), and the row-blocked decode does not take the
matrix.  Each wave stages M rows of its two tiles' activations; lanes 0-15
(M <= 4) or all lanes (M <= 16) return the output rows.  Checked against the
fp64 oracle, with a ragged last row tile, a bias, several matrices in one
launch, and row independence.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as ora

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module")
def native():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mlbricks_amd.elasticbit._native as native   # fails loudly when the library is missing
    return native


def _rel_max(y: np.ndarray, ref: np.ndarray) -> float:
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _case(native, rows, cols, b, seed):
    rng = np.random.default_rng(seed)
    qm = (1 << (b - 1)) - 1
    q = rng.integers(-qm, qm + 1, size=(rows, cols)).astype(np.int16)
    s = rng.uniform(0.002, 0.05, size=rows).astype(np.float32)
    return native.RuntimeMatrix._compressSelectedCodes(q, s, b, 0.01, 0.0), ora.pack_codes(q, b), s, rng


@pytest.mark.parametrize("rows,cols", [(1000, 4096), (4096, 2304), (33, 3072)])
@pytest.mark.parametrize("b", [4, 8, 10, 12])
@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 13, 16])
def test_gemv_small_batch_matches_oracle(native, rows, cols, b, M):
    m, payload, s, rng = _case(native, rows, cols, b, rows + cols + 10 * b + M)
    x = torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float16)).cuda()
    y = m.forwardTorch(x)
    assert y.shape == (M, rows)
    ref = ora.linear_intdot(payload, s, rows, cols, b, x.cpu().numpy().view(np.uint16))
    assert _rel_max(y.float().cpu().numpy(), ref) <= TOL
    bias = torch.from_numpy(rng.standard_normal(rows).astype(np.float16)).cuda()
    assert torch.equal(m.forwardTorch(x, bias=bias), y + bias)      # fp16_rn(fp16(y) + b), bit for bit


@pytest.mark.parametrize("M", [4, 16])
def test_gemv_small_batch_rows_are_independent(native, M):
    m, _, _, rng = _case(native, 1000, 4096, 10, 3)
    x = torch.from_numpy(rng.standard_normal((M, 4096)).astype(np.float16)).cuda()
    y = m.forwardTorch(x)
    assert torch.equal(m.forwardTorch(x[:2].contiguous()), y[:2])
    assert torch.equal(m.forwardTorch(x[3:].contiguous()), y[3:])
    assert torch.equal(y, m.forwardTorch(x))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 16])
def test_gemv_multi_matrix_equals_single_forwards(native, M):
    """A QKV-style group (4096 + 1024 + 1000 rows x 4096, b = 10) in one
    launch returns each matrix's own forward bit for bit."""
    rng = np.random.default_rng(40 + M)
    mats = []
    for rows in (4096, 1024, 1000):
        q = rng.integers(-511, 512, size=(rows, 4096)).astype(np.int16)
        s = rng.uniform(0.002, 0.05, size=rows).astype(np.float32)
        mats.append(native.RuntimeMatrix._compressSelectedCodes(q, s, 10, 0.01, 0.0))
    x = torch.from_numpy(rng.standard_normal((M, 4096)).astype(np.float16)).cuda()
    biases = [torch.from_numpy(rng.standard_normal(mm.rows).astype(np.float16)).cuda() for mm in mats]
    ys = native.forward_torch_multi(mats, x, biases)
    for j, (mm, yj) in enumerate(zip(mats, ys)):
        assert torch.equal(yj, mm.forwardTorch(x, bias=biases[j])), j


@pytest.mark.parametrize("M", [1, 3])
def test_multi_matrix_mixed_routes_equal_single_forwards(native, M):
    """At b = 7 the GEMV kernel takes at most 256 row tiles: in a group of a
    1024-row and a 4200-row matrix (263 row tiles) the two forwards take
    different kernels, so the group runs per matrix and each output still
    equals its own forward bit for bit."""
    rng = np.random.default_rng(70 + M)
    mats = []
    for rows in (1024, 4200):
        q = rng.integers(-63, 64, size=(rows, 4096)).astype(np.int16)
        s = rng.uniform(0.002, 0.05, size=rows).astype(np.float32)
        mats.append(native.RuntimeMatrix._compressSelectedCodes(q, s, 7, 0.01, 0.0))
    x = torch.from_numpy(rng.standard_normal((M, 4096)).astype(np.float16)).cuda()
    ys = native.forward_torch_multi(mats, x, None)
    for j, (mm, yj) in enumerate(zip(mats, ys)):
        assert torch.equal(yj, mm.forwardTorch(x)), j
