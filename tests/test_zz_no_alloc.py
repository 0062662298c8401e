"""The width search that allocates nothing (eb_analyze_widths_device_totals)
against the existing entry point (eb_analyze_widths_device), through the C ABI.

Its per-tile partials live in the library's static device array; the totals
must equal the existing entry point's partials summed over the tiles (the
same float32 partials, added in float64: within 1e-12 relative).  Two calls
in a row, the second with fewer rows and other data, show that nothing the
first left in the array leaks into the second.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def native():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mlbricks_amd.elasticbit._native as native   # fails loudly when the library is missing
    return native


def _inputs(seed: int, rows: int, cols: int, samples: int):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float16)
    w[:, : max(1, cols // 100)] *= 8
    x = rng.standard_normal((samples, cols)).astype(np.float16)
    w_t = torch.from_numpy(w).cuda()
    x_t = torch.from_numpy(x).cuda()
    max_abs = w_t.abs().amax(dim=1).float().contiguous()
    return w_t, x_t, max_abs


def _existing(native, w, x, max_abs) -> np.ndarray:
    rows, cols = w.shape
    tiles = -(-rows // native.ANALYZE_TILE_ROWS)
    partials = torch.empty((tiles, native.ANALYZE_SUMS), dtype=torch.float32, device="cuda")
    native.check(native.lib().eb_analyze_widths_device(w.data_ptr(), rows, cols, x.data_ptr(), x.shape[0],
                                                       max_abs.data_ptr(), partials.data_ptr(),
                                                       native.stream_handle(w.device)))
    return partials.double().sum(dim=0).cpu().numpy()


def _no_alloc(native, w, x, max_abs) -> np.ndarray:
    rows, cols = w.shape
    totals = torch.full((native.ANALYZE_SUMS,), float("nan"), dtype=torch.float64, device="cuda")
    native.check(native.lib().eb_analyze_widths_device_totals(w.data_ptr(), rows, cols, x.data_ptr(), x.shape[0],
                                                              max_abs.data_ptr(), totals.data_ptr(),
                                                              native.stream_handle(w.device)))
    return totals.cpu().numpy()


def test_totals_match_the_existing_entry_point_on_two_calls(native):
    for seed, rows, cols, samples in ((1, 3000, 1024, 32), (2, 100, 1000, 7)):
        w, x, max_abs = _inputs(seed, rows, cols, samples)
        got = _no_alloc(native, w, x, max_abs)
        want = _existing(native, w, x, max_abs)
        assert np.all(np.isfinite(got))
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=0)
        assert got[0] > 0 and np.all(got[1:] >= 0)


def test_rows_beyond_the_static_scratch_are_rejected_before_a_launch(native):
    w, x, max_abs = _inputs(3, 16, 64, 4)
    totals = torch.zeros(native.ANALYZE_SUMS, dtype=torch.float64, device="cuda")
    lib = native.lib()
    rc = lib.eb_analyze_widths_device_totals(w.data_ptr(), native.ANALYZE_STATIC_MAX_ROWS + 1, 64, x.data_ptr(), 4,
                                             max_abs.data_ptr(), totals.data_ptr(), native.stream_handle(w.device))
    assert rc != 0
    assert "static scratch" in lib.eb_last_error().decode()
    assert lib.eb_analyze_widths_device_totals(None, 16, 64, x.data_ptr(), 4, max_abs.data_ptr(),
                                               totals.data_ptr(), None) != 0
    assert torch.count_nonzero(totals) == 0
