"""Closed-form cases for the host width analyzer (elasticbit_runtime.cu:280-392).

Shared by ``test_oracle.py`` (the C oracle's ``ebo_analyze``) and
``test_capi_host.py`` (the library's ``eb_analyze``).  Each case fixes the
analyzer's errors by mathematics rather than by a second restatement of its
loops:

* **dyadic weights** ``k * 2^-7`` (|k| <= 7, every row reaching 7) against
  calibration rows in {-1, 0, 1}.  Every product and every partial sum is a
  multiple of 2^-7 well inside float32's range, so the analyzer's sequential
  float32 sums are exact and an error is exactly 0 wherever the outputs it
  compares are equal.  The full-precision outputs equal the reference
  outputs exactly when every decoded weight fp16_rn(q*s) equals w; that holds
  at b = 4, 7, 10, 13 (qmax = 2^(b-1) - 1 is a multiple of 7) and wherever the
  fp16 rounding snaps q*s back onto w, and fails elsewhere.
* **an all-zero matrix**: scale 1, every code 0, every output 0, so every
  error is 0 (the denominator is clamped to 1e-30, not divided by zero).
* **one nonzero weight per row**: every output is a single product, so the
  errors have the closed form sqrt(sum(d^2) / sum(ref^2)) over per-output
  differences d that numpy computes in float64 from the decoded weights.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as ora

WIDTHS = tuple(range(3, 17))


def dyadic_case(rows: int = 24, cols: int = 40, samples: int = 9, seed: int = 11):
    rng = np.random.default_rng(seed)
    k = rng.integers(-7, 8, size=(rows, cols))
    # every row reaches |k| = 7 so its scale is 7 * 2^-7 / qmax, and every k
    # value occurs so no width can be exact by accident of a missing value
    k[:, 0] = np.where(rng.random(rows) < 0.5, -7, 7)
    k[:, 1:16] = np.arange(-7, 8)[None, :]
    w = (k * 2.0 ** -7).astype(np.float32)
    x = rng.integers(-1, 2, size=(samples, cols)).astype(np.float32)
    x[:, 1:16] = 1.0            # the full range of k always meets a nonzero input
    return w, x


def decoded_equals_weights(w: np.ndarray, bits: int) -> bool:
    """True when the (golden-pinned) decode reproduces every weight exactly."""
    if bits == 16:
        return True
    s = ora.row_scales(w, bits)
    payload = ora.pack_weights(w, bits, s)
    deq, _ = ora.dequantize(payload, s, *w.shape, bits)
    return bool(np.array_equal(deq, w))


def one_hot_case(rows: int = 20, cols: int = 33, samples: int = 7, seed: int = 5):
    """One nonzero per row, at a column that differs between rows, with
    magnitudes that are not fp16-exact (so the fp16 rounding of the weights
    inside the reference outputs matters)."""
    rng = np.random.default_rng(seed)
    w = np.zeros((rows, cols), np.float32)
    cols_of = (np.arange(rows) * 7 + 3) % cols
    w[np.arange(rows), cols_of] = (rng.normal(0, 0.05, size=rows) + np.sign(rng.normal(size=rows)) * 0.01
                                   ).astype(np.float32)
    x = rng.normal(0, 1, size=(samples, cols)).astype(np.float32)
    return w, x, cols_of


def one_hot_expected(w: np.ndarray, x: np.ndarray, cols_of: np.ndarray, bits: int) -> tuple[float, float]:
    """(hardwareNative, fullPrecision) errors of the one-hot case in float64.

    Outputs: ref = fp16(w) * fp16(x) (a product of two binary16 values is
    exact in float32); full = fp16_rn(q*s) * fp16(x); hw = q*fp16(x) rounded to
    float32, times s rounded to float32 (b <= 8, the integer-dot form), or the
    full-precision output (b >= 9).  q = +-qmax because each row's only
    nonzero is its maximum."""
    rows = w.shape[0]
    wr = w[np.arange(rows), cols_of]
    wh = wr.astype(np.float16).astype(np.float64)
    xh = x[:, cols_of].astype(np.float16).astype(np.float64)          # [samples, rows]
    ref = xh * wh[None, :]
    if bits == 16:
        return 0.0, 0.0
    s = ora.row_scales(w, bits)
    payload = ora.pack_weights(w, bits, s)
    deq, _ = ora.dequantize(payload, s, *w.shape, bits)
    deq_r = deq[np.arange(rows), cols_of].astype(np.float64)
    full = xh * deq_r[None, :]
    if bits <= 8:
        q = ora.unpack_codes(payload, *w.shape, bits)[np.arange(rows), cols_of].astype(np.float64)
        idot = (xh * q[None, :]).astype(np.float32)                      # exact: |q| < 2^7, x fp16
        hw = (idot * s[None, :].astype(np.float32)).astype(np.float64)   # one float32 rounding
    else:
        hw = full
    den = max(float((ref ** 2).sum()), 1e-30)
    return (float(np.sqrt(((hw - ref) ** 2).sum() / den)),
            float(np.sqrt(((full - ref) ** 2).sum() / den)))
