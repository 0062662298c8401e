"""GPU tests of the fused width search (eb_analyze_widths_device), the
measurement behind ElasticBit.compress's width selection (_selectBitsTorch,
mlbricks/elasticbit/core.py:112-195).

The reference measures each width with torch operations and the vendor GEMM
(core.py:140-172); `_torch_width_errors` below runs those operations on the
same device as the floating-point reference.  The fused kernel sums in
another order, so its errors match within a tolerance, and the selected
width matches wherever no width's error lies within that tolerance of the
threshold (the reference's own selection at such margins depends on its
GEMM's rounding and is not pinned by any reference test).  Weights built
from a power-of-two scale pin exact zeros at the widths that represent them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlbricks_amd.elasticbit import _native
    return _native


@pytest.fixture(scope="module")
def native():
    return _need_gpu()


def _rel_l2(ref: torch.Tensor, cand: torch.Tensor) -> float:
    r = ref.float()
    den = torch.linalg.vector_norm(r).clamp_min(1.0e-30)
    return float((torch.linalg.vector_norm(cand.float() - r) / den).item())


def _torch_width_errors(weight: torch.Tensor, x16: torch.Tensor):
    """The reference's per-width measurement, core.py:140-172, all widths,
    with the integer-code output measured up to b = 12 (where this runtime's
    hardwareNative runs it; the reference stops at b = 8)."""
    reference = F.linear(x16, weight)
    w32 = weight.float()
    max_abs = w32.abs().amax(dim=1)
    full, hw = [], []
    for bits in range(3, 16):
        qmax = float((1 << (bits - 1)) - 1)
        scale = torch.where(max_abs > 0.0, max_abs / qmax, torch.ones_like(max_abs))
        q = torch.round(w32 / scale[:, None]).clamp(min=-qmax, max=qmax)
        deq16 = (q * scale[:, None]).to(torch.float16)
        f = _rel_l2(reference, F.linear(x16, deq16))
        if bits <= 12:
            idot = torch.matmul(x16.float(), q.transpose(0, 1).contiguous())
            h = _rel_l2(reference, (idot * scale[None, :]).to(torch.float16))
        else:
            h = f
        full.append(f)
        hw.append(h)
    return np.array(full), np.array(hw)


def _tol(err: np.ndarray, outputs: int) -> np.ndarray:
    """Two summation orders round an occasional output to the neighbouring
    fp16 value (one ulp, 2^-11 of the output), in ref and in the candidate.
    One such flip moves relL2 by about 2^-11 / sqrt(outputs); that bounds
    the difference where the error sits at the fp16 floor (b >= 12), and
    1e-3 of the error bounds it above."""
    return 1e-3 * err + 2.0 ** -11 * (3.0 / np.sqrt(outputs) + 0.01)


def _weights(rng, rows, cols, outliers=True):
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    if outliers:
        cols_out = rng.choice(cols, size=max(1, cols // 100), replace=False)
        w[:, cols_out] *= 8.0
    return torch.from_numpy(w.astype(np.float16)).cuda()


@pytest.mark.parametrize("rows,cols,samples", [
    (256, 512, 32), (100, 1000, 32), (37, 1003, 7), (300, 384, 40), (16, 4096, 1), (1024, 4096, 32),
])
def test_width_errors_match_torch_reference(native, rows, cols, samples):
    """Ragged rows (not whole 16-row tiles), columns that are not whole
    32-column chunks (1003 also takes the scalar loads), one and 40
    calibration rows (two launches)."""
    rng = np.random.default_rng(rows * 7 + cols + samples)
    w = _weights(rng, rows, cols)
    x16 = torch.from_numpy(rng.standard_normal((samples, cols)).astype(np.float16)).cuda()
    full, hw = native.width_errors_torch(w, x16)
    tf, th = _torch_width_errors(w, x16)
    n = rows * samples
    assert np.all(np.abs(full - tf) <= _tol(tf, n)), (full, tf)
    assert np.all(np.abs(hw - th) <= _tol(th, n)), (hw, th)
    # the errors fall with the width until the fp16 floor
    assert np.all(np.diff(full[:8]) < 0)


def test_power_of_two_weights_are_exact_where_representable(native):
    """w = k * 2^-7 with integer |k| <= 7 and every row reaching 7: widths
    whose qmax is a multiple of 7 (b = 4, 7, 10, 13) reproduce every weight,
    and at b >= 11 the fp16 rounding of q * s may restore it as well (numpy
    decides which).  With activations in {-1, 0, 1} over 256 columns every
    dot product is an integer of at most 1792 times 2^-7, exact in fp32 and
    in fp16, so the errors are exactly zero where the decoded weights equal
    w and positive where they do not."""
    rng = np.random.default_rng(11)
    rows, cols = 64, 256
    k = rng.integers(-7, 8, size=(rows, cols))
    k[:, 0] = 7
    w = torch.from_numpy((k * 2.0 ** -7).astype(np.float16)).cuda()
    x16 = torch.from_numpy(rng.integers(-1, 2, size=(32, cols)).astype(np.float16)).cuda()
    full, hw = native.width_errors_torch(w, x16)
    w32 = (k * 2.0 ** -7).astype(np.float32)
    for bits in range(3, 16):
        i = bits - 3
        qmax = np.float32((1 << (bits - 1)) - 1)
        scale = np.float32(7 * 2.0 ** -7) * (np.float32(1.0) / qmax)
        q = np.clip(np.rint(w32 / scale), -qmax, qmax).astype(np.float32)
        exact = np.array_equal((q * scale).astype(np.float16).astype(np.float32), w32)
        if bits in (4, 7, 10, 13):
            assert exact
        assert (full[i] == 0.0) == exact, bits
        if bits <= 12:
            # the integer-code output is exact only where q = (qmax / 7) k
            assert (hw[i] == 0.0) == (bits in (4, 7, 10)), bits
        else:
            assert hw[i] == full[i], bits
    from mlbricks_amd.elasticbit import core
    bits, err, codes, scales = core._selectBitsTorch(w, x16.float().cpu().numpy(), 0.0)
    assert (bits, err) == (4, 0.0)
    assert np.array_equal(codes, k.astype(np.int16))
    assert np.all(scales == np.float32(2.0 ** -7))


def test_all_zero_rows_and_matrix(native):
    rng = np.random.default_rng(3)
    w = _weights(rng, 48, 256)
    w[5] = 0
    w[40:] = 0
    x16 = torch.from_numpy(rng.standard_normal((32, 256)).astype(np.float16)).cuda()
    full, hw = native.width_errors_torch(w, x16)
    tf, th = _torch_width_errors(w, x16)
    assert np.all(np.abs(full - tf) <= _tol(tf, 48 * 32))
    assert np.all(np.abs(hw - th) <= _tol(th, 48 * 32))
    zero = torch.zeros(20, 64, dtype=torch.float16, device="cuda")
    full, hw = native.width_errors_torch(zero, x16[:, :64].contiguous())
    assert np.all(full == 0.0) and np.all(hw == 0.0)


@pytest.mark.parametrize("threshold", [0.02, 0.01, 0.005, 0.001, 1e-5])
def test_selection_matches_torch_reference_away_from_margins(native, threshold):
    from mlbricks_amd.elasticbit import core
    rng = np.random.default_rng(int(threshold * 1e6) + 1)
    w = _weights(rng, 512, 1024)
    calib = rng.standard_normal((32, 1024)).astype(np.float32)
    x16 = torch.from_numpy(calib).cuda().half()
    tf, th = _torch_width_errors(w, x16)
    terr = np.maximum(tf, th)
    tol = _tol(terr, 512 * 32)
    if np.any(np.abs(terr - threshold) <= 2 * tol):
        pytest.skip("a width's error lies at the threshold")
    passing = [b for b in range(3, 16) if terr[b - 3] <= threshold]
    expect = passing[0] if passing else 16
    bits, err, codes, scales = core._selectBitsTorch(w, calib, threshold)
    assert bits == expect
    if bits <= 15:
        assert abs(err - terr[bits - 3]) <= tol[bits - 3]
        qmax = (1 << (bits - 1)) - 1
        w32 = w.float().cpu().numpy()
        mx = np.abs(w32).max(axis=1)
        # torch divides by a Python scalar as a product with its fp32 reciprocal
        s = np.where(mx > 0, mx * (np.float32(1.0) / np.float32(qmax)), np.float32(1.0)).astype(np.float32)
        q = np.clip(np.rint(w32 / s[:, None]), -qmax, qmax).astype(np.int16)
        assert np.array_equal(scales, s)
        assert np.array_equal(codes, q)
    else:
        assert codes is None and scales is None


def test_width_errors_reject_bad_inputs(native):
    w = torch.zeros(16, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError, match="fp16 CUDA weights"):
        native.width_errors_torch(w.float(), torch.zeros(4, 64, dtype=torch.float16, device="cuda"))
    with pytest.raises(ValueError, match="calibration rows"):
        native.width_errors_torch(w, torch.zeros(4, 32, dtype=torch.float16, device="cuda"))
    with pytest.raises(ValueError, match="at least one row"):
        native.width_errors_torch(w, torch.zeros(0, 64, dtype=torch.float16, device="cuda"))
    lib = native.lib()
    x = torch.zeros(33, 64, dtype=torch.float16, device="cuda")
    mx = torch.zeros(16, dtype=torch.float32, device="cuda")
    out = torch.zeros(native.ANALYZE_SUMS, dtype=torch.float32, device="cuda")
    assert lib.eb_analyze_widths_device(w.data_ptr(), 16, 64, x.data_ptr(), 33, mx.data_ptr(), out.data_ptr(),
                                        None) != 0
    assert "samples must be in [1, 32]" in lib.eb_last_error().decode()
