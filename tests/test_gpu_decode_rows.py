"""GPU parity of the row-blocked batched decode (eb_decode_rows.hip).

The launcher sends 8 <= M <= 16 to linear_decode_rows_kernel when the matrix
has more 16-row tiles than the device has CUs (from M = 12 when that is at
most two per CU), cols <= 4096 and b <= 12.  On MI355X (256 CUs) the shapes
below take 2 (4200 rows: 263 row tiles), 3 (8260 rows: 517 = 3 x 172 + 1, so
the last workgroup holds one row tile of four rows) and 4 (12500 rows: 782
row tiles) row tiles per workgroup.  Four row tiles are taken for the
integer-code arithmetic only (b != 11); the decoded-fp16 arithmetic and b =
11 keep linear_decode_kernel there, which the same checks cover.

Every output is compared with the fp64 oracle in the arithmetic that runs
(integer-code dot product for hardwareNative b <= 12, decoded fp16 for
fullPrecision), at the north star's tolerance.
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


def _case(native, rows, cols, b, policy, seed):
    rng = np.random.default_rng(seed)
    qm = (1 << (b - 1)) - 1
    q = rng.integers(-qm, qm + 1, size=(rows, cols)).astype(np.int16)
    s = rng.uniform(0.002, 0.05, size=rows).astype(np.float32)
    m = native.RuntimeMatrix._compressSelectedCodes(q, s, b, 0.01, 0.0, decodePolicy=policy)
    return m, ora.pack_codes(q, b), s, rng


def _oracle(payload, s, rows, cols, b, x, policy):
    xs = x.cpu().numpy().view(np.uint16)
    if policy == "hardwareNative":
        return ora.linear_intdot(payload, s, rows, cols, b, xs)
    return ora.linear_w16(payload, s, rows, cols, b, xs)


def test_mi355x_has_the_cu_count_the_routing_above_assumes(native):
    assert torch.cuda.get_device_properties(0).multi_processor_count == 256


@pytest.mark.parametrize("rows,M", [(4200, 12), (8260, 16), (8260, 8), (12500, 13)])
@pytest.mark.parametrize("cols", [256, 1000])
@pytest.mark.parametrize("b", [3, 7, 10, 11, 12])
@pytest.mark.parametrize("policy", ["hardwareNative", "fullPrecision"])
def test_decode_rows_matches_oracle(native, rows, M, cols, b, policy):
    m, payload, s, rng = _case(native, rows, cols, b, policy, rows + 7 * M + cols + b)
    x = torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float16)).cuda()
    y = m.forwardTorch(x).float().cpu().numpy()
    assert y.shape == (M, rows)
    assert _rel_max(y, _oracle(payload, s, rows, cols, b, x, policy)) <= TOL


@pytest.mark.parametrize("b", [9, 10, 11])
def test_decode_rows_full_k(native, b):
    """cols = 4096 (32 steps: two per wave), three row tiles per workgroup."""
    rows, cols, M = 8260, 4096, 16
    m, payload, s, rng = _case(native, rows, cols, b, "hardwareNative", b)
    x = torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float16)).cuda()
    y = m.forwardTorch(x).float().cpu().numpy()
    assert _rel_max(y, _oracle(payload, s, rows, cols, b, x, "hardwareNative")) <= TOL
    assert _rel_max(y, _oracle(payload, s, rows, cols, b, x, "fullPrecision")) <= TOL   # the reference's W16A16


def test_decode_rows_unaligned_activations_and_bias(native):
    """x at a 2-byte offset (scalar activation loads) and a bias added as
    torch adds it to the fp16 output, bit for bit."""
    rows, cols, b, M = 8260, 1000, 10, 16
    m, payload, s, rng = _case(native, rows, cols, b, "hardwareNative", 5)
    buf = torch.empty(M * cols + 1, dtype=torch.float16, device="cuda")
    x = buf[1:].view(M, cols)
    x.copy_(torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float16)))
    assert x.data_ptr() % 16 != 0
    y = m.forwardTorch(x)
    assert _rel_max(y.float().cpu().numpy(), _oracle(payload, s, rows, cols, b, x, "hardwareNative")) <= TOL
    bias = torch.from_numpy(rng.standard_normal(rows).astype(np.float16)).cuda()
    assert torch.equal(m.forwardTorch(x, bias=bias), y + bias)


def test_decode_rows_deterministic_and_independent_of_other_rows(native):
    """Repeated calls are bit-identical, and each activation row's output
    does not depend on the other rows of the batch."""
    rows, cols, b = 8260, 1000, 10
    m, _, _, rng = _case(native, rows, cols, b, "hardwareNative", 11)
    x = torch.from_numpy(rng.standard_normal((16, cols)).astype(np.float16)).cuda()
    y = m.forwardTorch(x)
    assert torch.equal(y, m.forwardTorch(x))
    y8 = m.forwardTorch(x[:8].contiguous())
    assert torch.equal(y8, y[:8])
