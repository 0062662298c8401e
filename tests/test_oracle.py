"""Pin the C oracle against closed forms, published constants and golden fixtures.

The reference ships no golden vectors for ElasticBit, so every oracle function
is checked against something it shares no code with: numpy's IEEE binary16
conversion, Python big-integer bitstreams, float64 matrix products, published
FNV-1a test vectors and the pure-Python analyzer in tests/golden/make_golden.py.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as ora


# -- binary16 -----------------------------------------------------------------

def test_f16_to_f32_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = ora.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_ties_and_neighbours():
    # every finite binary16 value, the midpoints between neighbours (ties), and
    # the float32 values one ulp either side of each midpoint
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    v = h.view(np.float16).astype(np.float64)
    mids = ((v[:-1] + v[1:]) / 2).astype(np.float32)
    cands = np.concatenate([
        v.astype(np.float32), mids,
        np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0)),
        np.float32([65504, 65519.996, 65520, 65536, 1e30, np.inf, 2.0**-25, 2.0**-24,
                    3 * 2.0**-26, 1e-45, 0.0]),
    ])
    cands = np.concatenate([cands, -cands])
    with np.errstate(over="ignore"):
        ref = cands.astype(np.float16).view(np.uint16)
    assert np.array_equal(ora.f32_to_f16_bits(cands), ref)


def test_f32_to_f16_random_and_nan():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x.astype(np.float16)
    ours = ora.f32_to_f16_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan].view(np.uint16))
    assert np.isnan(ours[nan].view(np.float16)).all()


# -- canonical storage ----------------------------------------------------------

@pytest.mark.parametrize("b", range(3, 16))
def test_scales_codes_payload_decoded_match_golden(golden, b):
    w = golden["w"]
    s = ora.row_scales(w, b)
    assert np.array_equal(s.view(np.uint32), golden[f"scales_b{b}"].view(np.uint32))
    assert s[0] == 1.0                                   # all-zero row
    q = ora.quantize(w, s, b)
    assert np.array_equal(q, golden[f"codes_b{b}"])
    assert np.abs(q).max() == ora.qmax(b)                # each nonzero row reaches +-qmax
    payload = ora.pack_codes(q, b)
    assert np.array_equal(payload, golden[f"payload_b{b}"])
    assert np.array_equal(ora.pack_weights(w, b, s), golden[f"payload_b{b}"])
    assert np.array_equal(ora.unpack_codes(payload, *w.shape, b), q)
    f32, f16 = ora.dequantize(payload, s, *w.shape, b)
    assert np.array_equal(f16, golden[f"dec16_b{b}"])
    assert np.array_equal(f32, golden[f"dec16_b{b}"].view(np.float16).astype(np.float32))


def test_fp16_fallback_payload(golden):
    w = golden["w"]
    payload = ora.pack_weights(w, 16)
    assert np.array_equal(payload, golden["payload_b16"])
    f32, f16 = ora.dequantize(payload, None, *w.shape, 16)
    assert np.array_equal(f32, w)                       # w is already fp16-representable


def _bigint_payload(codes: np.ndarray, b: int) -> bytes:
    total = 0
    for i, q in enumerate(codes.reshape(-1).tolist()):
        total |= (q + ((1 << (b - 1)) - 1)) << (i * b)
    return total.to_bytes((codes.size * b + 7) // 8, "little")


@pytest.mark.parametrize("b", [3, 4, 5, 7, 8, 9, 15])
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 13), (8, 31), (17, 32), (33, 65)])
def test_bitstream_invariant_bruteforce(b, rows, cols):
    qm = (1 << (b - 1)) - 1
    rng = np.random.default_rng(rows * 1000 + cols * 10 + b)
    codes = rng.integers(-qm, qm + 1, size=(rows, cols)).astype(np.int16)
    payload = ora.pack_codes(codes, b)
    assert payload.size == (rows * cols * b + 7) // 8
    assert payload.tobytes() == _bigint_payload(codes, b)
    assert np.array_equal(ora.unpack_codes(payload, rows, cols, b), codes)
    for i in (0, rows * cols - 1):
        u = ora.extract(payload, i, b)
        assert u <= (1 << b) - 2


def test_pack_codes_rejects_out_of_range():
    with pytest.raises(ValueError):
        ora.pack_codes(np.array([[4]], np.int16), 3)     # qmax(3) = 3
    with pytest.raises(ValueError):
        ora.pack_codes(np.array([[-4]], np.int16), 3)


def test_quantize_is_round_half_even():
    # w / s == k + 0.5 exactly: rint goes to the even neighbour
    s = np.float32(0.25)
    assert ora.lib().ebo_quantize(np.float32(0.625), s, 8) == 2     # 2.5 -> 2
    assert ora.lib().ebo_quantize(np.float32(0.875), s, 8) == 4     # 3.5 -> 4
    assert ora.lib().ebo_quantize(np.float32(-0.625), s, 8) == -2
    assert ora.lib().ebo_quantize(np.float32(1e6), s, 4) == 7       # clamp to qmax


def test_planted_offset_mistake_is_caught(golden):
    # decoding with the legacy op's offset 2^(b-1) instead of qmax must differ
    b = 10
    payload = golden["payload_b10"]
    u = np.array([ora.extract(payload, i, b) for i in range(payload.size * 8 // b)])
    wrong = (u - (1 << (b - 1))).astype(np.int16)[: golden["codes_b10"].size]
    assert not np.array_equal(wrong.reshape(golden["codes_b10"].shape), golden["codes_b10"])


# -- output semantics -----------------------------------------------------------

@pytest.mark.parametrize("b", list(range(3, 16)) + [16])
@pytest.mark.parametrize("M", [1, 4])
def test_linear_outputs_match_golden(golden, b, M):
    w = golden["w"]
    rows, cols = w.shape
    payload = golden[f"payload_b{b}"]
    s = golden.get(f"scales_b{b}")
    x16 = golden[f"x16_m{M}"]
    yw = ora.linear_w16(payload, s, rows, cols, b, x16)
    np.testing.assert_allclose(yw, golden[f"y_w16_m{M}_b{b}"], rtol=1e-12, atol=1e-15)
    if b < 16:
        yi = ora.linear_intdot(payload, s, rows, cols, b, x16)
        np.testing.assert_allclose(yi, golden[f"y_intdot_m{M}_b{b}"], rtol=1e-12, atol=1e-15)


def test_cpu_baseline_gemv_close_to_fp64(golden):
    rng = np.random.default_rng(3)
    rows, cols = 64, 256
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float16).astype(np.float32)
    x16 = rng.standard_normal(cols).astype(np.float16).view(np.uint16)
    for b in (4, 8, 10, 16):
        s = ora.row_scales(w, b) if b != 16 else None
        payload = ora.pack_weights(w, b, s)
        y16, used = ora.gemv_f32_baseline(payload, s, rows, cols, b, x16, threads=2)
        ref = (ora.linear_intdot if b <= 8 else ora.linear_w16)(payload, s, rows, cols, b, x16)[0]
        y = y16.view(np.float16).astype(np.float64)
        assert np.abs(y - ref).max() / np.abs(ref).max() < 2e-3
        assert used >= 1


# -- analyzer ---------------------------------------------------------------------

def test_analyzer_matches_pure_python_restatement(golden):
    out = ora.analyze(golden["analyze_w"], golden["analyze_calib"])
    ref = golden["analyze_errors"]
    assert [a["bits"] for a in out] == list(range(3, 17))
    for a, (b, hw, fp) in zip(out, ref):
        assert a["bits"] == int(b)
        np.testing.assert_allclose(a["hardwareNativeError"], hw, rtol=1e-12, atol=1e-300)
        np.testing.assert_allclose(a["fullPrecisionError"], fp, rtol=1e-12, atol=1e-300)
        assert a["error"] == max(a["hardwareNativeError"], a["fullPrecisionError"])
    assert out[-1]["error"] == 0.0                       # fp16 fallback is exact
    # selection: first compressed width within threshold, else the fp16 fallback
    idx = ora.select(out, 1.0)
    assert out[idx]["bits"] == 3
    idx = ora.select(out, 0.0)
    assert out[idx]["bits"] == 16
    thr = out[5]["error"]
    idx = ora.select(out, thr)
    assert out[idx]["error"] <= thr
    assert all(a["error"] > thr for a in out[:idx])
    with pytest.raises(ValueError):
        ora.select(out, float("nan"))


def test_analyzer_dyadic_weights_are_exact_where_the_decode_is():
    """Dyadic weights: an error is exactly 0 where the decoded weights equal w
    (b = 4, 7, 10, 13 among them, since their qmax is a multiple of 7) and
    positive elsewhere.  A dropped fp16 rounding, a wrong scale or a wrong
    reference output makes a zero positive or a positive zero."""
    from analyzer_cases import WIDTHS, decoded_equals_weights, dyadic_case

    w, x = dyadic_case()
    out = {a["bits"]: a for a in ora.analyze(w, x)}
    assert tuple(out) == WIDTHS
    exact = {b for b in WIDTHS if decoded_equals_weights(w, b)}
    assert {4, 7, 10, 13, 16} <= exact
    assert not {3, 5, 6, 8} & exact
    for b in WIDTHS:
        full = out[b]["fullPrecisionError"]
        assert (full == 0.0) == (b in exact), (b, full)
    # integer-dot outputs (b <= 8) are exact where q = (qmax/7)*k and s carries
    # the 1/(qmax/7): b = 4 (s = 2^-7) and b = 7 (9*fp32(2^-7/9) rounds to 2^-7)
    for b in (4, 7):
        assert out[b]["hardwareNativeError"] == 0.0
    for b in (3, 5, 6, 8):
        assert out[b]["hardwareNativeError"] > 0.0
    for b in range(9, 17):
        assert out[b]["hardwareNativeError"] == out[b]["fullPrecisionError"]
    assert ora.select(list(out.values()), 0.0) == 1       # b = 4 is the first exact width


def test_analyzer_all_zero_matrix():
    w = np.zeros((6, 10), np.float32)
    x = np.random.default_rng(1).normal(size=(4, 10)).astype(np.float32)
    out = ora.analyze(w, x)
    for a in out:
        assert a["hardwareNativeError"] == 0.0 and a["fullPrecisionError"] == 0.0
        b = a["bits"]
        assert a["storageBytes"] == (120 if b == 16 else (60 * b + 7) // 8 + 24)
    assert np.array_equal(ora.row_scales(w, 8), np.ones(6, np.float32))
    assert out[ora.select(out, 0.0)]["bits"] == 3


def test_analyzer_one_nonzero_per_row_closed_form():
    """Every output is one product, so each error is a float64 closed form of
    the decoded weights; a transposed output index, a missing square root or
    a reference built from unrounded weights all move it."""
    from analyzer_cases import WIDTHS, one_hot_case, one_hot_expected

    w, x, cols_of = one_hot_case()
    out = {a["bits"]: a for a in ora.analyze(w, x)}
    for b in WIDTHS:
        hw, full = one_hot_expected(w, x, cols_of, b)
        np.testing.assert_allclose(out[b]["hardwareNativeError"], hw, rtol=1e-12, atol=0)
        np.testing.assert_allclose(out[b]["fullPrecisionError"], full, rtol=1e-12, atol=0)
        assert out[b]["error"] == max(out[b]["hardwareNativeError"], out[b]["fullPrecisionError"])
    # the integer-dot output carries the unrounded weight (q*s = w to float32
    # precision) while the reference carries fp16(w): positive error at b <= 8
    assert all(out[b]["hardwareNativeError"] > 0 for b in range(3, 9))


# -- MLB4 / FNV ------------------------------------------------------------------------

def test_fnv1a64_published_vectors(golden):
    published = [0xCBF29CE484222325, 0xAF63DC4C8601EC8C, 0x85944171F73967E8]
    assert [int(v) for v in golden["fnv_vectors"]] == published
    assert [ora.fnv1a64(d) for d in (b"", b"a", b"foobar")] == published


@pytest.mark.parametrize("b", [3, 8, 10, 16])
def test_mlb4_bytes_match_golden(golden, golden_dir, b):
    w = golden["w"]
    s = golden.get(f"scales_b{b}")
    data = ora.mlb4_bytes(*w.shape, b, s, golden[f"payload_b{b}"], 0.01, 0.005 if b != 16 else 0.0)
    assert data == (golden_dir / f"mlb4_b{b}.mlb").read_bytes()


# -- legacy group-scale op ------------------------------------------------------------

@pytest.mark.parametrize("b", [2, 4, 8])
@pytest.mark.parametrize("g", [13, 32, 7])
def test_legacy_packed_linear_matches_golden(golden, b, g):
    y = ora.packed_linear(golden["legacy_x"], golden[f"legacy_packed_b{b}"],
                          golden[f"legacy_scales_b{b}_g{g}"], golden[f"legacy_bias_b{b}_g{g}"],
                          b, g, 5, 13)
    np.testing.assert_allclose(y, golden[f"legacy_y_b{b}_g{g}"], rtol=1e-6, atol=1e-6)
