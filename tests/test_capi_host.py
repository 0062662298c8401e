"""Host side of libelasticbit_hip.so against the oracle (CPU only).

Covers the C ABI's exported symbols, the canonical packer, the MLB4 reader and
writer, the host analyzer and host dequantize.  No call here touches a GPU:
without a device the library builds host-only matrices.
"""
from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

from conftest import ROOT
from oracle import oracle as ora

native = pytest.importorskip("mlbricks_amd.elasticbit._native")
RM = native.RuntimeMatrix


def header_symbols() -> set[str]:
    text = (ROOT / "include" / "elasticbit.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(eb_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    syms = header_symbols()
    assert len(syms) >= 20
    lib = native.lib()
    for name in sorted(syms):
        assert hasattr(lib, name), f"{name} declared in include/elasticbit.h but not exported"
    assert lib.eb_abi_version() == 1


def test_backend_info_without_device_is_safe():
    info = native.backendInfo()
    assert info["activateDType"] == "float16"
    assert info["weightWidths"] == tuple(range(3, 17))
    assert info["prefill"] == "native"
    if not info["available"]:
        assert info["deviceIndex"] == -1


@pytest.mark.parametrize("b", [3, 4, 5, 7, 8, 9, 10, 11, 15])
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 13), (8, 31), (17, 32), (33, 65), (5, 1000)])
def test_host_pack_matches_oracle(b, rows, cols):
    qm = (1 << (b - 1)) - 1
    rng = np.random.default_rng(rows * 31 + cols * 7 + b)
    codes = rng.integers(-qm, qm + 1, size=(rows, cols)).astype(np.int16)
    ours = native.host_pack_codes(codes, b)
    assert np.array_equal(ours, ora.pack_codes(codes, b))
    assert np.array_equal(native.host_unpack_codes(ours, codes.size, b), codes.reshape(-1))


def test_host_pack_rejects_out_of_range():
    with pytest.raises(ValueError, match="exceeds selected bit range"):
        native.host_pack_codes(np.array([8], np.int16), 4)


@pytest.mark.parametrize("b", range(3, 16))
def test_compress_selected_codes_canonical_and_dequantize(golden, b):
    w = golden["w"]
    q = golden[f"codes_b{b}"]
    s = golden[f"scales_b{b}"]
    m = RM._compressSelectedCodes(q, s, b, 0.01, 0.005)
    scales, payload = m._canonical()
    assert np.array_equal(scales, s)
    assert np.array_equal(payload, golden[f"payload_b{b}"])
    deq = m.dequantize()
    assert np.array_equal(deq, golden[f"dec16_b{b}"].view(np.float16).astype(np.float32))
    assert m.storageBits == b
    assert m.storageBytes == payload.size + 4 * w.shape[0]
    assert m.originalBytes == 2 * w.size


@pytest.mark.parametrize("b", [3, 8, 10, 15, 16])
def test_compress_selected_weights_matches_oracle(golden, b):
    w = golden["w"]
    m = RM._compressSelected(w, b, 0.01, 0.0)
    scales, payload = m._canonical()
    if b == 16:
        assert scales.size == 0
        assert np.array_equal(payload, golden["payload_b16"])
    else:
        assert np.array_equal(scales, golden[f"scales_b{b}"])
        assert np.array_equal(payload, golden[f"payload_b{b}"])


def test_pack_weights_matches_oracle_on_larger_random():
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((67, 301)) * 0.03).astype(np.float16).astype(np.float32)
    w[:, 7] *= 8
    for b in (5, 9, 12):
        m = RM._compressSelected(w, b, 0.01, 0.0)
        s, p = m._canonical()
        so = ora.row_scales(w, b)
        assert np.array_equal(s, so)
        assert np.array_equal(p, ora.pack_weights(w, b, so))
        _, d16 = ora.dequantize(p, s, *w.shape, b)
        assert np.array_equal(m.dequantize(), d16.view(np.float16).astype(np.float32))


@pytest.mark.parametrize("b", [3, 8, 10, 16])
def test_mlb4_load_save_roundtrip_matches_golden_bytes(golden_dir, tmp_path, b):
    src = golden_dir / f"mlb4_b{b}.mlb"
    m = RM.load(str(src))
    assert m.storageBits == b
    assert m.shape == (8, 32)
    assert m.threshold == 0.01
    out = tmp_path / "copy.mlb"
    m.save(str(out))
    assert out.read_bytes() == src.read_bytes()


@pytest.mark.parametrize("b", [3, 8, 10, 16])
def test_mlb4_corruption_and_truncation_are_rejected(golden_dir, tmp_path, b):
    with pytest.raises(RuntimeError, match="checksum mismatch"):
        RM.load(str(golden_dir / f"mlb4_b{b}_corrupt.mlb"))
    data = (golden_dir / f"mlb4_b{b}.mlb").read_bytes()
    short = tmp_path / "short.mlb"
    short.write_bytes(data[:-1])
    with pytest.raises(RuntimeError, match="invalid ElasticBit MLB4 metadata"):
        RM.load(str(short))
    bad = tmp_path / "magic.mlb"
    bad.write_bytes(b"MLB5" + data[4:])
    with pytest.raises(RuntimeError, match="invalid ElasticBit MLB4 file"):
        RM.load(str(bad))
    with pytest.raises(RuntimeError, match="failed to open"):
        RM.load(str(tmp_path / "missing.mlb"))


def test_analyzer_bit_exact_against_oracle():
    rng = np.random.default_rng(20260918)
    w = rng.normal(0, 0.04, size=(96, 128)).astype(np.float32)
    c = rng.normal(0, 1, size=(12, 128)).astype(np.float32)
    ours = native.analyze(w, c, 0.02)
    ref = ora.analyze(w, c)
    for a, r in zip(ours["candidates"], ref):
        assert a["bits"] == r["bits"]
        assert a["hardwareNativeError"] == r["hardwareNativeError"]
        assert a["fullPrecisionError"] == r["fullPrecisionError"]
        assert a["storageBytes"] == r["storageBytes"]
        assert a["passes"] == (r["error"] <= 0.02)
    assert ours["selectedBits"] == ref[ora.select(ref, 0.02)]["bits"]
    assert ours["selectedError"] <= 0.02


def test_analyzer_closed_forms():
    """eb_analyze on the cases whose errors mathematics fixes (dyadic weights:
    exact zeros where the decode reproduces w; one nonzero per row: float64
    closed form; all-zero matrix: all zeros, b = 3 selected)."""
    from analyzer_cases import WIDTHS, decoded_equals_weights, dyadic_case, one_hot_case, one_hot_expected

    w, x = dyadic_case()
    got = {a["bits"]: a for a in native.analyze(w, x, 0.0)["candidates"]}
    for b in WIDTHS:
        assert (got[b]["fullPrecisionError"] == 0.0) == decoded_equals_weights(w, b), b
    assert got[4]["hardwareNativeError"] == 0.0 and got[7]["hardwareNativeError"] == 0.0
    assert native.analyze(w, x, 0.0)["selectedBits"] == 4

    w, x, cols_of = one_hot_case()
    got = {a["bits"]: a for a in native.analyze(w, x, 0.01)["candidates"]}
    for b in WIDTHS:
        hw, full = one_hot_expected(w, x, cols_of, b)
        np.testing.assert_allclose(got[b]["hardwareNativeError"], hw, rtol=1e-12, atol=0)
        np.testing.assert_allclose(got[b]["fullPrecisionError"], full, rtol=1e-12, atol=0)

    zero = native.analyze(np.zeros((6, 10), np.float32), np.ones((3, 10), np.float32), 0.0)
    assert all(a["error"] == 0.0 for a in zero["candidates"])
    assert zero["selectedBits"] == 3 and zero["selectedError"] == 0.0


def test_analyzer_matches_pure_python_golden(golden):
    ours = native.analyze(golden["analyze_w"], golden["analyze_calib"], 0.01)
    for a, (b, hw, fp) in zip(ours["candidates"], golden["analyze_errors"]):
        assert a["bits"] == int(b)
        np.testing.assert_allclose(a["hardwareNativeError"], hw, rtol=1e-12, atol=1e-300)
        np.testing.assert_allclose(a["fullPrecisionError"], fp, rtol=1e-12, atol=1e-300)


def test_compress_uses_analyzer_selection():
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, size=(40, 64)).astype(np.float32)
    c = rng.normal(0, 1, size=(6, 64)).astype(np.float32)
    a = native.analyze(w, c, 0.01)
    m = RM.compress(w, c, 0.01)
    assert m.storageBits == a["selectedBits"]
    assert m.error == a["selectedError"]
    s, p = m._canonical()
    if m.storageBits < 16:
        assert np.array_equal(p, ora.pack_weights(w, m.storageBits, ora.row_scales(w, m.storageBits)))


def test_argument_validation_messages():
    q = np.zeros((2, 4), np.int16)
    with pytest.raises(ValueError, match="scales must contain one value per weight row"):
        RM._compressSelectedCodes(q, np.ones(3, np.float32), 8, 0.01, 0.0)
    with pytest.raises(ValueError, match="finite and positive"):
        RM._compressSelectedCodes(q, np.array([1.0, 0.0], np.float32), 8, 0.01, 0.0)
    with pytest.raises(ValueError, match="between 3 and 16"):
        RM._compressSelectedCodes(q, np.ones(2, np.float32), 2, 0.01, 0.0)
    with pytest.raises(ValueError, match="3..15-bit"):
        RM._compressSelectedCodes(q, np.ones(2, np.float32), 16, 0.01, 0.0)
    with pytest.raises(ValueError, match="does not satisfy threshold"):
        RM._compressSelectedCodes(q, np.ones(2, np.float32), 8, 0.01, 0.5)
    with pytest.raises(ValueError, match="finite non-negative"):
        native.analyze(np.ones((2, 2)), np.ones((1, 2)), float("nan"))
    with pytest.raises(ValueError, match="both be 2D"):
        native.analyze(np.ones(2), np.ones((1, 2)), 0.1)
    with pytest.raises(ValueError, match="decodePolicy"):
        RM._compressSelectedCodes(q, np.ones(2, np.float32), 8, 0.01, 0.0, decodePolicy="fast")


def test_policy_switch_changes_execution_semantics_metadata():
    m = RM._compressSelectedCodes(np.zeros((4, 32), np.int16), np.ones(4, np.float32), 10, 0.01, 0.0)
    assert m.decodePolicy == "hardwareNative"
    assert m.executionWidth == 10
    assert m.executionPlanner == "gfx950BitPlane"
    m.setDecodePolicy("fullPrecision")
    assert m.decodePolicy == "fullPrecision"
    assert m.executionWidth == 16
    assert m.executionPlanner == "fullPrecision"


def test_device_calls_fail_loudly_without_device():
    info = native.backendInfo()
    if info["available"]:
        pytest.skip("a HIP device is present")
    m = RM._compressSelectedCodes(np.zeros((4, 32), np.int16), np.ones(4, np.float32), 10, 0.01, 0.0)
    with pytest.raises(RuntimeError, match="CUDA runtime"):
        m.forward(np.zeros(32, np.float32))
    with pytest.raises(RuntimeError, match="CUDA runtime"):
        m._materializeTorch()


def test_device_code_factory_validates_arguments():
    lib = native.lib()
    out = ctypes.c_void_p()
    s = np.ones(4, np.float32)
    sp = s.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    assert lib.eb_compress_selected_codes_device(None, sp, 4, 32, 10, 0.01, 0.0, 0, ctypes.byref(out)) != 0
    assert "null pointer" in lib.eb_last_error().decode()
    p = ctypes.c_void_p(16)
    assert lib.eb_compress_selected_codes_device(p, sp, 4, 32, 16, 0.01, 0.0, 0, ctypes.byref(out)) != 0
    assert "3..15-bit" in lib.eb_last_error().decode()
    assert lib.eb_compress_selected_codes_device(p, sp, 4, 32, 10, 0.01, 0.5, 0, ctypes.byref(out)) != 0
    assert "does not satisfy threshold" in lib.eb_last_error().decode()


def test_analyze_widths_validates_arguments():
    lib = native.lib()
    p = ctypes.c_void_p(16)
    assert lib.eb_analyze_widths_device(None, 16, 64, p, 4, p, p, None) != 0
    assert "null pointer" in lib.eb_last_error().decode()
    assert lib.eb_analyze_widths_device(p, 0, 64, p, 4, p, p, None) != 0
    assert "rows and cols" in lib.eb_last_error().decode()
    assert lib.eb_analyze_widths_device(p, 16, 64, p, 0, p, p, None) != 0
    assert "samples must be in [1, 32]" in lib.eb_last_error().decode()


def test_forward_multi_validates_before_any_device_work():
    lib = native.lib()
    m = RM._compressSelectedCodes(np.zeros((4, 32), np.int16), np.ones(4, np.float32), 10, 0.01, 0.0)
    handles = (ctypes.c_void_p * 2)(m._h, m._h)
    ys = (ctypes.c_void_p * 2)(None, None)
    assert lib.eb_forward_multi(None, 1, None, 1, None, None, None) != 0
    assert "null pointer" in lib.eb_last_error().decode()
    assert lib.eb_forward_multi(handles, 0, ctypes.c_void_p(16), 1, ys, None, None) != 0
    assert "count must be positive" in lib.eb_last_error().decode()
    assert lib.eb_forward_multi(handles, 2, ctypes.c_void_p(16), 0, ys, None, None) != 0
    assert "M must be" in lib.eb_last_error().decode()


def test_prefill_tile_mode_is_validated():
    with pytest.raises(ValueError, match="prefill tile mode"):
        native.set_prefill_tiles("square")
    lib = native.lib()
    assert lib.eb_set_prefill_tiles(8) != 0
    assert lib.eb_set_prefill_tiles(-1) != 0
    for mode in ("narrow", "wide", "wide8", "wide8plain", "wide8short", "wideplain", "wideshort", "auto"):
        native.set_prefill_tiles(mode)


def _plan_coverage(M, rows, cus):
    """Every 64-row by 256-row block of the output below M is covered by
    exactly one tile of the plan, and no tile starts at or beyond M."""
    rects, cost = native.prefill_plan(M, rows, cus)
    nb = (rows + 255) // 256
    cells = np.zeros(((M + 63) // 64, nb), dtype=np.int32)
    for m0, mblocks, height, nb0, nblocks in rects:
        assert height in (256, 192) and m0 % 64 == 0
        assert 0 <= nb0 and nb0 + nblocks <= nb
        for i in range(mblocks):
            r0 = m0 + i * height
            assert r0 < M, (M, rows, cus, rects)
            c0, c1 = r0 // 64, min(r0 + height, M + 63) // 64
            cells[c0:min(c1, cells.shape[0]), nb0:nb0 + nblocks] += 1
    assert (cells == 1).all(), (M, rows, cus, rects)
    return rects, cost


def test_prefill_plan_covers_every_output_once():
    """The launch plan of the eight-wave prefill (host logic, no device):
    whatever mix of 256 x 256 and 192 x 256 tiles it picks covers the output
    exactly once, and its estimate never exceeds the plain grid's."""
    try:
        for cus in (256, 304, 80, 32):
            for rows in (256, 1000, 4096, 11008, 14336, 30000):
                for M in (256, 300, 1024, 1536, 1792, 2048, 2100, 3000, 4096, 8192):
                    for waves in ("wide8", "wide"):
                        native.set_prefill_tiles(waves)
                        rects, cost = _plan_coverage(M, rows, cus)
                        native.set_prefill_tiles(waves + "plain")
                        plain, plain_cost = _plan_coverage(M, rows, cus)
                        assert len(plain) == 1 and plain[0][2] == 256
                        assert cost <= plain_cost + 1e-12
                        native.set_prefill_tiles(waves + "short")
                        short, _ = _plan_coverage(M, rows, cus)
                        assert [r[2] for r in short] == [192]
    finally:
        native.set_prefill_tiles("auto")


def test_prefill_plan_at_the_measured_shapes():
    """The plan's choices at the shapes its cost model was measured on
    (256 CUs): configs[3] keeps the plain 448-tile grid, 14336 x 4096 at
    M = 1536 and 11008 x 4096 at M = 2048 balance their sparse last round."""
    native.set_prefill_tiles("auto")
    rects, _ = native.prefill_plan(2048, 14336, 256)
    assert rects == [(0, 8, 256, 0, 56)]
    for M, rows in ((1536, 14336), (2048, 11008)):
        rects, cost = native.prefill_plan(M, rows, 256)
        assert any(r[2] == 192 for r in rects), rects
        full = sum(r[1] * r[4] for r in rects if r[2] == 256)
        assert full <= 256
    assert lib_rejects_bad_plan_arguments()


def lib_rejects_bad_plan_arguments():
    lib = native.lib()
    rects = (ctypes.c_int32 * 15)()
    assert lib.eb_prefill_plan(0, 4096, 256, rects, None) != 0
    assert lib.eb_prefill_plan(256, 4096, 0, rects, None) != 0
    assert lib.eb_prefill_plan(256, 4096, 256, None, None) != 0
    return True
