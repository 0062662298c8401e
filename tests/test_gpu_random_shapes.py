"""Seeded random sweep over the forward's dispatch boundaries (needs an MI355X).

Each case draws a shape, width, policy, activation row count, alignment and
bias, so that together the cases cross every route the launcher picks: the
GEMV kernel, the decode kernel (activations staged whole, in K chunks or read
from L2; one, two or four 16-row blocks), the prefill kernel (64- and
128-row tiles, whole and half tiles), the wide tiles and the LDS-staged gemm
kernel for unaligned or ragged activations.  Every output is checked
against the fp32 product of the decoded weights (the W16A16 formula, within
the 2e-3 bound for every arithmetic), and a corner of it against the fp64
oracle of the reference formula.  A second sweep draws large prefill shapes
for the 256 x 256 kernels' launch plans.
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
        pytest.skip("no HIP device")
    from mlbricks_amd.elasticbit import _native
    return _native


def _case(seed: int):
    rng = np.random.default_rng(1000 + seed)
    rows = int(rng.choice([1, 7, 16, 40, 130, 257, 600, 1300]))
    cols = int(rng.choice([8, 13, 128, 200, 384, 1000, 1024, 2304, 4096, 5000]))
    M = int(rng.choice([1, 2, 5, 16, 17, 31, 33, 64, 65, 100, 128, 200, 300]))
    b = int(rng.integers(3, 17))
    policy = str(rng.choice(["hardwareNative", "fullPrecision"]))
    aligned = bool(rng.random() < 0.8)
    with_bias = bool(rng.random() < 0.4)
    return rng, rows, cols, M, b, policy, aligned, with_bias


@pytest.mark.parametrize("seed", range(48))
def test_random_shape_matches_decoded_product(native, seed):
    rng, rows, cols, M, b, policy, aligned, with_bias = _case(seed)
    if b == 16:
        w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        m = native.RuntimeMatrix._compressSelected(w, 16, 0.01, 0.0, decodePolicy=policy)
        s = None
    else:
        qm = (1 << (b - 1)) - 1
        q = rng.integers(-qm, qm + 1, size=(rows, cols)).astype(np.int16)
        # weights of comparable magnitude at every width
        s = (rng.uniform(0.002, 0.05, size=rows) * min(1.0, 127.0 / qm)).astype(np.float32)
        m = native.RuntimeMatrix._compressSelectedCodes(q, s, b, 0.01, 0.0, decodePolicy=policy)
    x0 = torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float16)).cuda()
    if aligned:
        x = x0
    else:
        buf = torch.empty(M * cols + 1, dtype=torch.float16, device="cuda")
        x = buf[1:].view(M, cols)
        x.copy_(x0)
    bias = torch.from_numpy((0.1 * rng.standard_normal(rows)).astype(np.float16)).cuda() if with_bias else None
    y = m.forwardTorch(x, bias=bias)
    torch.cuda.synchronize()
    assert y.shape == (M, rows)
    assert torch.isfinite(y).all(), (rows, cols, M, b, policy)
    wd = m._materializeTorch().float()
    full = torch.matmul(x.float(), wd.T.contiguous())
    yy = y.float() - (bias.float() if with_bias else 0.0)
    err = float((yy - full).abs().max() / full.abs().max().clamp_min(1e-30))
    assert err <= TOL, (rows, cols, M, b, policy, aligned, err)
    sub_r, sub_m = min(rows, 24), min(M, 24)
    xs = x[-sub_m:].cpu().numpy().view(np.uint16)
    if b == 16:
        ref = ora.linear_w16(ora.pack_weights(w[-sub_r:], 16), None, sub_r, cols, 16, xs)
    else:
        sub = ora.pack_codes(q[-sub_r:], b)
        if b <= 12 and policy == "hardwareNative":
            ref = ora.linear_intdot(sub, s[-sub_r:], sub_r, cols, b, xs)
        else:
            ref = ora.linear_w16(sub, s[-sub_r:], sub_r, cols, b, xs)
    got = y[-sub_m:, -sub_r:].float().cpu().numpy()
    if with_bias:
        got = got - bias[-sub_r:].float().cpu().numpy()
    ref_max = float(np.abs(ref).max())
    if ref_max > 0:
        assert float(np.abs(got - ref).max()) / ref_max <= TOL, (rows, cols, M, b, policy)


def _large_case(seed: int):
    rng = np.random.default_rng(5000 + seed)
    rows = int(rng.integers(2200, 16500))
    cols = int(rng.choice([256, 640, 1000, 1536]))
    M = int(rng.integers(256, 3300))
    b = int(rng.integers(3, 16))
    policy = str(rng.choice(["hardwareNative", "fullPrecision"]))
    waves = str(rng.choice(["wide", "wide8"]))
    return rng, rows, cols, M, b, policy, waves


@pytest.mark.parametrize("seed", range(12))
def test_random_large_prefill_plans_are_bit_identical(native, seed):
    """Seeded large prefill shapes through the 256 x 256 kernels: the launch
    plan (whole rounds of 256 x 256 tiles, the rest as 192 x 256 tiles where
    estimated faster), the plain 256 x 256 grid and 192 x 256 tiles
    throughout give the same bits, covering the output once whatever plan the
    shape draws; the result matches the decoded product."""
    rng, rows, cols, M, b, policy, waves = _large_case(seed)
    qm = (1 << (b - 1)) - 1
    q = rng.integers(-qm, qm + 1, size=(rows, cols)).astype(np.int16)
    s = (rng.uniform(0.002, 0.05, size=rows) * min(1.0, 127.0 / qm)).astype(np.float32)
    m = native.RuntimeMatrix._compressSelectedCodes(q, s, b, 0.01, 0.0, decodePolicy=policy)
    x = torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float16)).cuda()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ys = {}
    try:
        for suffix in ("", "plain", "short"):
            native.set_prefill_tiles(waves + suffix)
            ys[suffix] = m.forwardTorch(x)
        plan, _ = native.prefill_plan(M, rows, cus)
    finally:
        native.set_prefill_tiles("auto")
    case = (rows, cols, M, b, policy, waves, plan)
    assert torch.equal(ys[""], ys["plain"]), case
    assert torch.equal(ys["short"], ys["plain"]), case
    wd = m._materializeTorch().float()
    full = torch.matmul(x.float(), wd.T.contiguous())
    err = float((ys[""].float() - full).abs().max() / full.abs().max().clamp_min(1e-30))
    assert err <= TOL, (case, err)
