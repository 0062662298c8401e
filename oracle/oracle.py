"""ElasticBit CPU oracle: ctypes wrapper over ``libeb_oracle.so``.

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the checker; the product
package ``mlbricks_amd`` never imports it.

The C source (``eb_oracle.c``) restates the MLBricks ElasticBit host algorithm
(``mlbricks/elasticbit/csrc/elasticbit_runtime.cu``); each wrapper below names
the reference lines its C function follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libeb_oracle.so"

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i16p = ctypes.POINTER(ctypes.c_int16)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)


class Analysis(ctypes.Structure):
    _fields_ = [
        ("bits", ctypes.c_int),
        ("hardware_native_error", ctypes.c_double),
        ("full_precision_error", ctypes.c_double),
        ("error", ctypes.c_double),
        ("storage_bytes", ctypes.c_uint64),
    ]


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s"] + (["-B"] if force else []) + ["-C", str(HERE)], check=True)
    return LIB_PATH


_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.ebo_f32_to_f16.restype = ctypes.c_uint16
        L.ebo_f32_to_f16.argtypes = [ctypes.c_float]
        L.ebo_f16_to_f32.restype = ctypes.c_float
        L.ebo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.ebo_f32_to_f16_array.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.ebo_f16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.ebo_qmax.restype = ctypes.c_uint32
        L.ebo_qmax.argtypes = [ctypes.c_int]
        L.ebo_packed_bytes.restype = ctypes.c_size_t
        L.ebo_packed_bytes.argtypes = [ctypes.c_size_t, ctypes.c_int]
        L.ebo_quantize.restype = ctypes.c_int32
        L.ebo_quantize.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_int]
        L.ebo_row_scales.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.ebo_pack_codes.restype = ctypes.c_int
        L.ebo_pack_codes.argtypes = [_i16p, ctypes.c_size_t, ctypes.c_int, _u8p]
        L.ebo_pack_weights.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _u8p]
        L.ebo_extract.restype = ctypes.c_uint32
        L.ebo_extract.argtypes = [_u8p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int]
        L.ebo_unpack_codes.argtypes = [_u8p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, _i16p]
        L.ebo_dequantize.argtypes = [_u8p, ctypes.c_size_t, _f32p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, _f32p, _u16p]
        for name in ("ebo_linear_intdot", "ebo_linear_w16"):
            fn = getattr(L, name)
            fn.argtypes = [_u8p, ctypes.c_size_t, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                           _u16p, ctypes.c_int, _f64p]
        L.ebo_gemv_f32_baseline.restype = ctypes.c_int
        L.ebo_gemv_f32_baseline.argtypes = [_u8p, ctypes.c_size_t, _f32p, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, _u16p, ctypes.c_int, ctypes.c_int, _u16p,
                                            ctypes.c_int]
        L.ebo_analyze.restype = ctypes.c_int
        L.ebo_analyze.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int,
                                  ctypes.POINTER(Analysis)]
        L.ebo_select.restype = ctypes.c_int
        L.ebo_select.argtypes = [ctypes.POINTER(Analysis), ctypes.c_int, ctypes.c_double]
        L.ebo_fnv1a64.restype = ctypes.c_uint64
        L.ebo_fnv1a64.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        L.ebo_mlb4_write.restype = ctypes.c_size_t
        L.ebo_mlb4_write.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _u8p,
                                     ctypes.c_size_t, ctypes.c_double, ctypes.c_double]
        L.ebo_packed_linear.argtypes = [_f64p, ctypes.c_int, _u8p, _f64p, _f64p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, _f64p]
        _LIB = L
    return _LIB


def _p(arr: np.ndarray, ctype):
    return arr.ctypes.data_as(ctypes.POINTER(ctype))


def _c(arr, dtype) -> np.ndarray:
    return np.ascontiguousarray(arr, dtype=dtype)


# -- binary16 ---------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = _c(x, np.float32).reshape(-1)
    out = np.empty(x.shape, np.uint16)
    lib().ebo_f32_to_f16_array(_p(x, ctypes.c_float), _p(out, ctypes.c_uint16), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16).reshape(-1)
    out = np.empty(h.shape, np.float32)
    lib().ebo_f16_to_f32_array(_p(h, ctypes.c_uint16), _p(out, ctypes.c_float), h.size)
    return out


# -- canonical storage (elasticbit_runtime.cu:54-238) -----------------------

def qmax(bits: int) -> int:
    return int(lib().ebo_qmax(bits))


def packed_bytes(count: int, bits: int) -> int:
    return int(lib().ebo_packed_bytes(count, bits))


def row_scales(w, bits: int) -> np.ndarray:
    """make_row_scales, elasticbit_runtime.cu:83-101."""
    w = _c(w, np.float32)
    rows, cols = w.shape
    out = np.ones(rows, np.float32)
    lib().ebo_row_scales(_p(w, ctypes.c_float), rows, cols, bits, _p(out, ctypes.c_float))
    return out


def quantize(w, scales, bits: int) -> np.ndarray:
    """quantize_scalar over a matrix, elasticbit_runtime.cu:77-81."""
    w = _c(w, np.float32)
    out = np.empty(w.shape, np.int16)
    for r in range(w.shape[0]):
        s = float(scales[r])
        for c in range(w.shape[1]):
            out[r, c] = lib().ebo_quantize(float(w[r, c]), s, bits)
    return out


def pack_codes(codes, bits: int) -> np.ndarray:
    """pack_exact_codes, elasticbit_runtime.cu:150-186."""
    q = _c(codes, np.int16).reshape(-1)
    out = np.zeros(packed_bytes(q.size, bits), np.uint8)
    rc = lib().ebo_pack_codes(_p(q, ctypes.c_int16), q.size, bits, _p(out, ctypes.c_uint8))
    if rc != 0:
        raise ValueError("prequantized ElasticBit code exceeds selected bit range")
    return out


def pack_weights(w, bits: int, scales=None) -> np.ndarray:
    """pack_exact_weights, elasticbit_runtime.cu:103-148."""
    w = _c(w, np.float32)
    rows, cols = w.shape
    nbytes = rows * cols * 2 if bits == 16 else packed_bytes(rows * cols, bits)
    out = np.zeros(nbytes, np.uint8)
    s = _c(scales if scales is not None else np.ones(rows), np.float32)
    lib().ebo_pack_weights(_p(w, ctypes.c_float), rows, cols, bits, _p(s, ctypes.c_float),
                           _p(out, ctypes.c_uint8))
    return out


def extract(payload, index: int, bits: int) -> int:
    payload = _c(payload, np.uint8)
    return int(lib().ebo_extract(_p(payload, ctypes.c_uint8), payload.size, index, bits))


def unpack_codes(payload, rows: int, cols: int, bits: int) -> np.ndarray:
    payload = _c(payload, np.uint8)
    out = np.empty((rows, cols), np.int16)
    lib().ebo_unpack_codes(_p(payload, ctypes.c_uint8), payload.size, rows * cols, bits,
                           _p(out, ctypes.c_int16))
    return out


def dequantize(payload, scales, rows: int, cols: int, bits: int):
    """dequantize_payload_host, elasticbit_runtime.cu:208-238 -> (f32, fp16 bits)."""
    payload = _c(payload, np.uint8)
    s = _c(scales if scales is not None and len(scales) else np.ones(rows), np.float32)
    out = np.empty((rows, cols), np.float32)
    out16 = np.empty((rows, cols), np.uint16)
    lib().ebo_dequantize(_p(payload, ctypes.c_uint8), payload.size, _p(s, ctypes.c_float), rows, cols,
                         bits, _p(out, ctypes.c_float), _p(out16, ctypes.c_uint16))
    return out, out16


def _linear(name, payload, scales, rows, cols, bits, x16) -> np.ndarray:
    payload = _c(payload, np.uint8)
    s = _c(scales if scales is not None and len(scales) else np.ones(rows), np.float32)
    x16 = _c(x16, np.uint16).reshape(-1, cols)
    M = x16.shape[0]
    y = np.empty((M, rows), np.float64)
    getattr(lib(), name)(_p(payload, ctypes.c_uint8), payload.size, _p(s, ctypes.c_float), rows, cols,
                         bits, _p(x16, ctypes.c_uint16), M, _p(y, ctypes.c_double))
    return y


def linear_intdot(payload, scales, rows, cols, bits, x16) -> np.ndarray:
    """hardwareNative integer-dot semantics, fp64 accumulation (runtime.cu:538-558)."""
    return _linear("ebo_linear_intdot", payload, scales, rows, cols, bits, x16)


def linear_w16(payload, scales, rows, cols, bits, x16) -> np.ndarray:
    """W16A16 semantics (decoded fp16 weights), fp64 accumulation (runtime.cu:635-647)."""
    return _linear("ebo_linear_w16", payload, scales, rows, cols, bits, x16)


def gemv_f32_baseline(payload, scales, rows, cols, bits, x16, row_begin=0, row_end=None,
                      threads=0):
    """CPU baseline GEMV (fp32 accumulate, fp16 output); returns (y16, threads_used)."""
    payload = _c(payload, np.uint8)
    s = _c(scales if scales is not None and len(scales) else np.ones(rows), np.float32)
    x16 = _c(x16, np.uint16).reshape(-1)
    row_end = rows if row_end is None else row_end
    y = np.empty(row_end - row_begin, np.uint16)
    used = lib().ebo_gemv_f32_baseline(_p(payload, ctypes.c_uint8), payload.size, _p(s, ctypes.c_float),
                                       rows, cols, bits, _p(x16, ctypes.c_uint16), row_begin, row_end,
                                       _p(y, ctypes.c_uint16), threads)
    if used < 0:
        raise ValueError("bad row range")
    return y, used


# -- analyzer (elasticbit_runtime.cu:280-436) --------------------------------

def analyze(w, calib) -> list[dict]:
    w = _c(w, np.float32)
    calib = _c(calib, np.float32)
    rows, cols = w.shape
    out = (Analysis * 14)()
    rc = lib().ebo_analyze(_p(w, ctypes.c_float), rows, cols, _p(calib, ctypes.c_float),
                           calib.shape[0], out)
    if rc != 0:
        raise ValueError("weights and calibration must be non-empty")
    return [
        {
            "bits": a.bits,
            "hardwareNativeError": a.hardware_native_error,
            "fullPrecisionError": a.full_precision_error,
            "error": a.error,
            "storageBytes": int(a.storage_bytes),
        }
        for a in out
    ]


def select(analyses: list[dict], threshold: float) -> int:
    arr = (Analysis * len(analyses))()
    for i, a in enumerate(analyses):
        arr[i].bits = a["bits"]
        arr[i].hardware_native_error = a["hardwareNativeError"]
        arr[i].full_precision_error = a["fullPrecisionError"]
        arr[i].error = a["error"]
        arr[i].storage_bytes = a["storageBytes"]
    idx = lib().ebo_select(arr, len(analyses), float(threshold))
    if idx < 0:
        raise ValueError("threshold must be a finite non-negative value")
    return idx


# -- MLB4 / FNV (elasticbit_runtime.cu:682-712, 1024-1049) -------------------

def fnv1a64(data: bytes) -> int:
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    return int(lib().ebo_fnv1a64(buf, len(data)))


def mlb4_bytes(rows, cols, bits, scales, payload, threshold, selected_error) -> bytes:
    payload = _c(payload, np.uint8)
    s = _c(scales if (scales is not None and bits != 16) else np.zeros(1), np.float32)
    n = 80 + (0 if bits == 16 else 4 * rows) + payload.size
    buf = np.zeros(n, np.uint8)
    wrote = lib().ebo_mlb4_write(_p(buf, ctypes.c_uint8), rows, cols, bits, _p(s, ctypes.c_float),
                                 _p(payload, ctypes.c_uint8), payload.size, float(threshold),
                                 float(selected_error))
    assert wrote == n
    return buf.tobytes()


# -- legacy op (bolt/ops_cuda.cu:2708-2750) ----------------------------------

def packed_linear(x, packed, scales, bias, bits, group_size, out_features, in_features):
    x = _c(x, np.float64).reshape(-1, in_features)
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.float64)
    b = None if bias is None or np.size(bias) == 0 else _c(bias, np.float64)
    y = np.empty((x.shape[0], out_features), np.float64)
    lib().ebo_packed_linear(_p(x, ctypes.c_double), x.shape[0], _p(packed, ctypes.c_uint8),
                            _p(scales, ctypes.c_double),
                            _p(b, ctypes.c_double) if b is not None else None,
                            bits, group_size, out_features, in_features, _p(y, ctypes.c_double))
    return y


__all__ = [name for name in dir() if not name.startswith("_")]
