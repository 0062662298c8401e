"""ctypes binding of libelasticbit_hip.so with the surface of MLBricks'
``mlbricks.elasticbit._C`` pybind11 module (elasticbit_runtime.cu:1411-1469):
``analyze``, ``backendInfo`` and the ``RuntimeMatrix`` class.

Importing this module loads the HIP library; it raises ImportError when the
library has not been built (``python -m mlbricks_amd.csrc.build``).  torch is
imported first so the library binds to the HIP runtime torch already loaded.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Any, Sequence

import numpy as np
import torch

LIB_PATH = Path(os.environ.get(
    "MLBRICKS_AMD_ELASTICBIT_LIB",
    Path(__file__).resolve().parents[1] / "lib" / "libelasticbit_hip.so",
))

if not LIB_PATH.exists():
    raise ImportError(f"ElasticBit HIP library not built: {LIB_PATH}")
try:
    _lib = ctypes.CDLL(str(LIB_PATH))
except OSError as exc:  # pragma: no cover - environment dependent
    raise ImportError(f"cannot load {LIB_PATH}: {exc}") from exc

EB_OK = 0
EB_INVALID_ARGUMENT = 1
POLICIES = {"hardwareNative": 1, "fullPrecision": 2}
POLICY_NAMES = {v: k for k, v in POLICIES.items()}
DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_d = ctypes.c_double
_f32p = ctypes.POINTER(ctypes.c_float)
_i16p = ctypes.POINTER(ctypes.c_int16)
_u8p = ctypes.POINTER(ctypes.c_uint8)


class _Props(ctypes.Structure):
    _fields_ = [
        ("rows", _i), ("cols", _i), ("storage_bits", _i), ("execution_width", _i),
        ("decode_policy", _i), ("device_index", _i),
        ("storage_bytes", _u64), ("execution_bytes", _u64), ("original_bytes", _u64),
        ("threshold", _d), ("selected_error", _d), ("memory_reduction", _d),
        ("execution_planner", ctypes.c_char * 32),
    ]


class _BitAnalysis(ctypes.Structure):
    _fields_ = [
        ("bits", _i), ("hardware_native_error", _d), ("full_precision_error", _d),
        ("error", _d), ("storage_bytes", _u64), ("memory_reduction", _d), ("passes", _i),
    ]


class _Backend(ctypes.Structure):
    _fields_ = [
        ("available", _i), ("device_index", _i), ("compute_units", _i),
        ("weight_widths", _i * 16), ("n_weight_widths", _i), ("validated", _i),
        ("device", ctypes.c_char * 128), ("architecture", ctypes.c_char * 64),
        ("activate_dtype", ctypes.c_char * 16), ("prefill", ctypes.c_char * 16),
        ("decode_planner", ctypes.c_char * 32), ("decode_engine", ctypes.c_char * 32),
        ("decode_status", ctypes.c_char * 32), ("decode_validation", ctypes.c_char * 64),
    ]


def _sig(name: str, argtypes: list, restype=_i) -> None:
    fn = getattr(_lib, name)
    fn.argtypes = argtypes
    fn.restype = restype


_sig("eb_last_error", [], ctypes.c_char_p)
_sig("eb_abi_version", [])
_sig("eb_analyze", [_f32p, _i, _i, _f32p, _i, _d, ctypes.POINTER(_BitAnalysis), ctypes.POINTER(_i)])
_sig("eb_backend_info", [ctypes.POINTER(_Backend)])
_sig("eb_compress", [_f32p, _i, _i, _f32p, _i, _d, _i, ctypes.POINTER(_vp)])
_sig("eb_compress_selected", [_f32p, _i, _i, _i, _d, _d, _i, ctypes.POINTER(_vp)])
_sig("eb_compress_selected_codes", [_i16p, _f32p, _i, _i, _i, _d, _d, _i, ctypes.POINTER(_vp)])
_sig("eb_compress_selected_codes_device", [_vp, _f32p, _i, _i, _i, _d, _d, _i, ctypes.POINTER(_vp)])
_sig("eb_load", [ctypes.c_char_p, _i, ctypes.POINTER(_vp)])
_sig("eb_save", [_vp, ctypes.c_char_p])
_sig("eb_destroy", [_vp], None)
_sig("eb_get_props", [_vp, ctypes.POINTER(_Props)])
_sig("eb_set_decode_policy", [_vp, _i])
_sig("eb_get_canonical", [_vp, _f32p, _u8p])
_sig("eb_dequantize_host", [_vp, _f32p])
_sig("eb_forward_host", [_vp, _f32p, _f32p])
_sig("eb_benchmark", [_vp, _f32p, _i, ctypes.POINTER(_d)])
_sig("eb_forward", [_vp, _vp, _i64, _vp, _vp, _vp])
_sig("eb_forward_multi", [_vp, _i, _vp, _i64, _vp, _vp, _vp])
_sig("eb_analyze_widths_device", [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp])
_sig("eb_analyze_widths_device_totals", [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp])
_sig("eb_materialize_fp16", [_vp, _vp, _vp])
_sig("eb_unpack_codes", [_vp, _vp, _vp])
_sig("eb_packed_linear", [_vp, _i, _i64, _vp, _vp, _i, _vp, _i, _i64, _i64, _i64, _vp, _vp])
_sig("eb_set_prefill_tiles", [_i])
_sig("eb_prefill_plan", [ctypes.c_int64, _i, _i, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_double)])
_sig("eb_host_pack_codes", [_i16p, _u64, _i, _u8p, _u64])
_sig("eb_host_unpack_codes", [_u8p, _u64, _u64, _i, _i16p])


def lib() -> ctypes.CDLL:
    return _lib


def check(status: int) -> None:
    """Map a C-ABI status to the reference's exception types."""
    if status == EB_OK:
        return
    message = (_lib.eb_last_error() or b"").decode("utf-8", "replace")
    if status == EB_INVALID_ARGUMENT:
        raise ValueError(message)
    raise RuntimeError(message)


def _ptr(arr: np.ndarray, ctype):
    return arr.ctypes.data_as(ctypes.POINTER(ctype))


def _f32_2d(value: Any, message: str) -> np.ndarray:
    arr = np.ascontiguousarray(value, dtype=np.float32)
    if arr.ndim != 2:
        raise ValueError(message)
    return arr


def _policy(value: str) -> int:
    try:
        return POLICIES[str(value)]
    except KeyError:
        raise ValueError("decodePolicy must be 'hardwareNative' or 'fullPrecision'") from None


# torch's raw current-stream query costs ~0.1 us; building a Stream object
# for the same answer costs ~2 us, which a decode loop pays per launch.
_raw_current_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _device_index(device: torch.device | int | None) -> int:
    if device is None:
        return torch.cuda.current_device()
    if isinstance(device, int):
        return device
    index = torch.device(device).index
    return torch.cuda.current_device() if index is None else index


def stream_handle(device: torch.device | int | None = None) -> int:
    """hipStream_t of torch's current stream on ``device`` (0 = legacy default)."""
    if _raw_current_stream is not None:
        return int(_raw_current_stream(_device_index(device)))
    return int(torch.cuda.current_stream(device).cuda_stream)


# ---------------------------------------------------------------------------
# module-level functions
# ---------------------------------------------------------------------------

def analyze(weights: Any, calibrationData: Any, threshold: float) -> dict:
    """``_C.analyze`` (elasticbit_runtime.cu:438-483)."""
    w = np.ascontiguousarray(weights, dtype=np.float32)
    c = np.ascontiguousarray(calibrationData, dtype=np.float32)
    if w.ndim != 2 or c.ndim != 2:
        raise ValueError("weights and calibrationData must both be 2D")
    if c.shape[1] != w.shape[1]:
        raise ValueError("calibrationData width must equal weight cols")
    out = (_BitAnalysis * 14)()
    sel = _i(0)
    check(_lib.eb_analyze(_ptr(w, ctypes.c_float), w.shape[0], w.shape[1], _ptr(c, ctypes.c_float),
                          c.shape[0], float(threshold), out, ctypes.byref(sel)))
    candidates = [
        {
            "bits": a.bits,
            "hardwareNativeError": a.hardware_native_error,
            "fullPrecisionError": a.full_precision_error,
            "error": a.error,
            "storageBytes": int(a.storage_bytes),
            "memoryReduction": a.memory_reduction,
            "passes": bool(a.passes),
        }
        for a in out
    ]
    chosen = candidates[sel.value]
    return {
        "threshold": float(threshold),
        "selectedBits": chosen["bits"],
        "selectedError": chosen["error"],
        "candidates": candidates,
    }


def backendInfo() -> dict:
    """``_C.backendInfo`` (elasticbit_runtime.cu:1386-1409)."""
    b = _Backend()
    check(_lib.eb_backend_info(ctypes.byref(b)))
    return {
        "available": bool(b.available),
        "device": b.device.decode(),
        "deviceIndex": int(b.device_index),
        "architecture": b.architecture.decode(),
        "computeUnits": int(b.compute_units),
        "weightWidths": tuple(b.weight_widths[i] for i in range(b.n_weight_widths)),
        "activateDType": b.activate_dtype.decode(),
        "prefill": b.prefill.decode(),
        "decodePlanner": b.decode_planner.decode(),
        "decodeEngine": b.decode_engine.decode(),
        "decodeStatus": b.decode_status.decode(),
        "decodeValidation": b.decode_validation.decode(),
        "validated": bool(b.validated),
    }


PREFILL_TILES = {"auto": 0, "narrow": 1, "wide": 2, "wide8": 3, "wide8plain": 4, "wide8short": 5,
                 "wideplain": 6, "wideshort": 7}


def forward_torch_multi(matrices: Sequence["RuntimeMatrix"], input: torch.Tensor,
                        biases: Sequence[torch.Tensor | None] | None = None) -> list[torch.Tensor]:
    """``[m.forwardTorch(input, bias=b) for m, b in zip(matrices, biases)]``
    in as few launches as the widths allow: matrices that read the same
    activations (a QKV or Gate/Up group) share one decode launch for up to
    16 rows of ``input`` (64 where the decode kernel is the faster route for
    each matrix).  Every matrix must have ``cols`` equal to the last
    dimension of ``input`` and live on its device.  No single-call
    counterpart in the reference, whose Stage-2F concatenates the
    materialized weights instead (stage2f.py:382-420)."""
    mats = list(matrices)
    if not mats:
        raise ValueError("forwardTorchMulti needs at least one matrix")
    props = [m._p() for m in mats]
    for m, p in zip(mats, props):
        m._check_input(input, p)
    if biases is not None and len(biases) != len(mats):
        raise ValueError("biases must hold one entry (or None) per matrix")
    x = input.contiguous()
    rows_in = x.numel() // props[0].cols
    outs = [torch.empty((*x.shape[:-1], p.rows), dtype=torch.float16, device=x.device) for p in props]
    bs: list[torch.Tensor | None] = []
    for j, p in enumerate(props):
        b = None if biases is None else biases[j]
        if b is not None:
            if b.dtype != torch.float16 or b.numel() != p.rows or b.device != x.device:
                raise ValueError("bias must be fp16 [rows] on the input device")
            b = b.contiguous()
        bs.append(b)
    if rows_in == 0:
        return outs
    n = len(mats)
    handles = (ctypes.c_void_p * n)(*[m._h for m in mats])
    ys = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    bptr = (ctypes.c_void_p * n)(*[b.data_ptr() if b is not None else None for b in bs])
    # eb_forward_multi makes the matrices' device current for the launch
    check(_lib.eb_forward_multi(handles, n, x.data_ptr(), rows_in, ys, bptr, stream_handle(props[0].device_index)))
    return outs


ANALYZE_TILE_ROWS = 16
ANALYZE_MAX_SAMPLES = 32
ANALYZE_SUMS = 24
ANALYZE_STATIC_MAX_ROWS = 262144      # eb_analyze_widths_device_totals
ANALYZE_WIDTHS = tuple(range(3, 16))


def width_errors_torch(weight: torch.Tensor, calibration16: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """relL2 errors of every storage width b = 3..15 against ``F.linear(x, W)``
    for fp16 CUDA weights ``[rows, cols]`` and fp16 calibration rows
    ``[samples, cols]`` on the same device, from one fused pass over the
    weights (eb_analyze_widths_device; the measurement of _selectBitsTorch,
    core.py:112-195).  Returns ``(full, hw)``, float64 arrays indexed by
    b - 3.  ``hw`` is the integer-code output's error for b <= 12 (the
    arithmetic hardwareNative runs there) and equals ``full`` for b >= 13,
    where hardwareNative runs W16A16."""
    if not weight.is_cuda or weight.dtype != torch.float16 or weight.dim() != 2:
        raise ValueError("width search needs fp16 CUDA weights [rows, cols]")
    if calibration16.device != weight.device or calibration16.dtype != torch.float16 or \
            calibration16.dim() != 2 or calibration16.shape[1] != weight.shape[1]:
        raise ValueError("calibration rows must be fp16 [samples, cols] on the weight device")
    rows, cols = weight.shape
    samples = calibration16.shape[0]
    if samples == 0:
        raise ValueError("calibrationData must contain at least one row")
    w = weight.contiguous()
    x = calibration16.contiguous()
    tiles = -(-rows // ANALYZE_TILE_ROWS)
    max_abs = w.abs().amax(dim=1).float().contiguous()
    chunks = -(-samples // ANALYZE_MAX_SAMPLES)
    partials = torch.empty((chunks, tiles, ANALYZE_SUMS), dtype=torch.float32, device=w.device)
    with torch.cuda.device(w.device):
        stream = stream_handle(w.device)
        for c in range(chunks):
            xs = x[c * ANALYZE_MAX_SAMPLES:(c + 1) * ANALYZE_MAX_SAMPLES]
            check(_lib.eb_analyze_widths_device(w.data_ptr(), rows, cols, xs.data_ptr(), xs.shape[0],
                                                max_abs.data_ptr(), partials[c].data_ptr(), stream))
    sums = partials.double().sum(dim=(0, 1)).cpu().numpy()
    den = max(float(np.sqrt(sums[0])), 1.0e-30)
    full = np.sqrt(sums[1:14]) / den
    hw = full.copy()
    hw[:10] = np.sqrt(sums[14:24]) / den
    return full, hw


def set_prefill_tiles(mode: str) -> None:
    """Tile shape of the prefill route (M > 16, b <= 15): 'auto' (default,
    picked by estimated rounds over the compute units), 'narrow' (128 x 256),
    'wide' (256 x 256, four waves) or 'wide8' (eight waves), each with a
    partial last round balanced by 192 x 256 tiles where estimated faster,
    'wideplain' / 'wide8plain' (without the balancing) or 'wideshort' /
    'wide8short' (192 x 256 tiles throughout).
    Process-wide; a tuning and test control with no counterpart in the
    reference."""
    if mode not in PREFILL_TILES:
        raise ValueError(f"prefill tile mode must be one of {sorted(PREFILL_TILES)}")
    check(_lib.eb_set_prefill_tiles(PREFILL_TILES[mode]))


def prefill_plan(M: int, rows: int, cus: int) -> tuple[list[tuple[int, int, int, int, int]], float]:
    """The 256 x 256 prefill launch plan for an M x rows output on `cus`
    compute units under the current tile mode: rectangles of tiles (first
    activation row, activation blocks, block height, first 256-row weight
    block, weight blocks), 256-row ones first, and the estimated time in full
    rounds of 256 x 256 tiles.  An inspection aid with no counterpart in the
    reference."""
    rects = (ctypes.c_int32 * 15)()
    cost = ctypes.c_double()
    check(_lib.eb_prefill_plan(M, rows, cus, rects, ctypes.byref(cost)))
    out = [tuple(rects[5 * i:5 * i + 5]) for i in range(3)]
    return [r for r in out if r[1] > 0 and r[4] > 0], cost.value


def host_pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    q = np.ascontiguousarray(codes, dtype=np.int16).reshape(-1)
    out = np.zeros((q.size * int(bits) + 7) // 8, np.uint8)
    check(_lib.eb_host_pack_codes(_ptr(q, ctypes.c_int16), q.size, int(bits), _ptr(out, ctypes.c_uint8), out.size))
    return out


def host_unpack_codes(payload: np.ndarray, count: int, bits: int) -> np.ndarray:
    p = np.ascontiguousarray(payload, dtype=np.uint8)
    out = np.empty(int(count), np.int16)
    check(_lib.eb_host_unpack_codes(_ptr(p, ctypes.c_uint8), p.size, int(count), int(bits),
                                    _ptr(out, ctypes.c_int16)))
    return out


def packed_linear(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None,
                  bits: int, group_size: int, out_features: int, in_features: int) -> torch.Tensor:
    """``elastic_linear_packed`` device launch (bolt/ops_cuda.cu:2752-2795)."""
    if x.dtype not in DTYPES or scales.dtype not in DTYPES:
        raise RuntimeError("x/scales must be floating point")
    rows = x.numel() // int(in_features) if int(in_features) > 0 else 0
    out = torch.empty((*x.shape[:-1], int(out_features)), dtype=x.dtype, device=x.device)
    has_bias = bias is not None and bias.numel() != 0
    with torch.cuda.device(x.device):
        check(_lib.eb_packed_linear(
            x.data_ptr(), DTYPES[x.dtype], rows, packed.data_ptr(), scales.data_ptr(), DTYPES[scales.dtype],
            bias.data_ptr() if has_bias else None, int(bits), int(group_size), int(out_features),
            int(in_features), out.data_ptr(), stream_handle(x.device)))
    return out


# ---------------------------------------------------------------------------
# RuntimeMatrix
# ---------------------------------------------------------------------------

class RuntimeMatrix:
    """Native matrix handle with the ``_C.RuntimeMatrix`` surface."""

    __slots__ = ("_h", "_props")

    def __init__(self, handle: ctypes.c_void_p) -> None:
        self._h = handle
        self._props = self._fetch()

    def __del__(self, _destroy=_lib.eb_destroy) -> None:
        # _destroy is bound at definition time: module globals may be gone at exit
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _destroy(h)
            self._h = None

    # -- factories (elasticbit_runtime.cu:720-871) ---------------------------

    @staticmethod
    def compress(weights: Any, calibrationData: Any, threshold: float,
                 decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        w = np.ascontiguousarray(weights, dtype=np.float32)
        c = np.ascontiguousarray(calibrationData, dtype=np.float32)
        if w.ndim != 2 or c.ndim != 2:
            raise ValueError("weights and calibrationData must both be 2D")
        if c.shape[1] != w.shape[1]:
            raise ValueError("calibrationData width must equal weight cols")
        h = _vp()
        check(_lib.eb_compress(_ptr(w, ctypes.c_float), w.shape[0], w.shape[1], _ptr(c, ctypes.c_float),
                               c.shape[0], float(threshold), _policy(decodePolicy), ctypes.byref(h)))
        return RuntimeMatrix(h)

    @staticmethod
    def _compressSelected(weights: Any, selectedBits: int, threshold: float, selectedError: float,
                          decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        w = _f32_2d(weights, "weights must be 2D")
        h = _vp()
        check(_lib.eb_compress_selected(_ptr(w, ctypes.c_float), w.shape[0], w.shape[1], int(selectedBits),
                                        float(threshold), float(selectedError), _policy(decodePolicy),
                                        ctypes.byref(h)))
        return RuntimeMatrix(h)

    @staticmethod
    def _compressSelectedCodes(codes: Any, scales: Any, selectedBits: int, threshold: float,
                               selectedError: float, decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        q = np.ascontiguousarray(codes, dtype=np.int16)
        s = np.ascontiguousarray(scales, dtype=np.float32)
        if q.ndim != 2:
            raise ValueError("codes must be 2D")
        if s.ndim != 1 or s.shape[0] != q.shape[0]:
            raise ValueError("scales must contain one value per weight row")
        h = _vp()
        check(_lib.eb_compress_selected_codes(_ptr(q, ctypes.c_int16), _ptr(s, ctypes.c_float), q.shape[0],
                                              q.shape[1], int(selectedBits), float(threshold),
                                              float(selectedError), _policy(decodePolicy), ctypes.byref(h)))
        return RuntimeMatrix(h)

    @staticmethod
    def _compressSelectedCodesTorch(codes: torch.Tensor, scales: Any, selectedBits: int, threshold: float,
                                    selectedError: float, decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        """_compressSelectedCodes for int16 codes already on the HIP device
        (the GPU width search's output): packed and repacked on the device,
        only the b-bit stream comes back to the host copy."""
        if not torch.is_tensor(codes) or not codes.is_cuda or codes.dtype != torch.int16 or codes.dim() != 2:
            raise ValueError("codes must be a 2D int16 CUDA tensor")
        q = codes.contiguous()
        s = np.ascontiguousarray(scales, dtype=np.float32)
        if s.ndim != 1 or s.shape[0] != q.shape[0]:
            raise ValueError("scales must contain one value per weight row")
        h = _vp()
        with torch.cuda.device(q.device):
            torch.cuda.current_stream(q.device).synchronize()   # the codes are complete before the legacy stream reads them
            check(_lib.eb_compress_selected_codes_device(
                ctypes.c_void_p(q.data_ptr()), _ptr(s, ctypes.c_float), q.shape[0], q.shape[1], int(selectedBits),
                float(threshold), float(selectedError), _policy(decodePolicy), ctypes.byref(h)))
        return RuntimeMatrix(h)

    @staticmethod
    def load(path: str, decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        h = _vp()
        check(_lib.eb_load(os.fsencode(str(path)), _policy(decodePolicy), ctypes.byref(h)))
        return RuntimeMatrix(h)

    # -- properties -----------------------------------------------------------

    def _fetch(self) -> _Props:
        p = _Props()
        check(_lib.eb_get_props(self._h, ctypes.byref(p)))
        return p

    def _p(self) -> _Props:
        # Only the decode policy changes after construction; setDecodePolicy refreshes.
        return self._props

    @property
    def rows(self) -> int:
        return self._p().rows

    @property
    def cols(self) -> int:
        return self._p().cols

    @property
    def shape(self) -> tuple[int, int]:
        p = self._p()
        return (p.rows, p.cols)

    @property
    def storageBits(self) -> int:
        return self._p().storage_bits

    @property
    def executionWidth(self) -> int:
        return self._p().execution_width

    @property
    def executionPlanner(self) -> str:
        return self._p().execution_planner.decode()

    @property
    def decodePolicy(self) -> str:
        return POLICY_NAMES[self._p().decode_policy]

    @property
    def activateDType(self) -> str:
        return "float16"

    @property
    def storageBytes(self) -> int:
        return int(self._p().storage_bytes)

    @property
    def executionBytes(self) -> int:
        return int(self._p().execution_bytes)

    @property
    def originalBytes(self) -> int:
        return int(self._p().original_bytes)

    @property
    def memoryReduction(self) -> float:
        return float(self._p().memory_reduction)

    @property
    def threshold(self) -> float:
        return float(self._p().threshold)

    @property
    def error(self) -> float:
        return float(self._p().selected_error)

    @property
    def deviceIndex(self) -> int:
        return int(self._p().device_index)

    # -- methods ----------------------------------------------------------------

    def setDecodePolicy(self, value: str) -> None:
        check(_lib.eb_set_decode_policy(self._h, _policy(value)))
        self._props = self._fetch()

    def save(self, path: str) -> None:
        check(_lib.eb_save(self._h, os.fsencode(str(path))))

    def dequantize(self) -> np.ndarray:
        p = self._p()
        out = np.empty((p.rows, p.cols), np.float32)
        check(_lib.eb_dequantize_host(self._h, _ptr(out, ctypes.c_float)))
        return out

    def _canonical(self) -> tuple[np.ndarray, np.ndarray]:
        """Canonical storage: (fp32 scales, payload bytes) -- the MLB4 body."""
        p = self._p()
        n_scales = 0 if p.storage_bits == 16 else p.rows
        scales = np.zeros(n_scales, np.float32)
        payload = np.zeros(int(p.storage_bytes) - 4 * n_scales, np.uint8)
        check(_lib.eb_get_canonical(self._h, _ptr(scales, ctypes.c_float) if n_scales else None,
                                    _ptr(payload, ctypes.c_uint8)))
        return scales, payload

    def forward(self, input: Any) -> np.ndarray:
        """Host round trip, fp32 [cols] -> fp32 [rows] (elasticbit_runtime.cu:873-900)."""
        p = self._p()
        x = np.ascontiguousarray(input, dtype=np.float32)
        if x.ndim != 1 or x.shape[0] != p.cols:
            raise ValueError("input must have shape [cols]")
        y = np.empty(p.rows, np.float32)
        check(_lib.eb_forward_host(self._h, _ptr(x, ctypes.c_float), _ptr(y, ctypes.c_float)))
        return y

    def benchmark(self, input: Any, iterations: int = 500) -> float:
        p = self._p()
        if int(iterations) <= 0:
            raise ValueError("iterations must be positive")
        x = np.ascontiguousarray(input, dtype=np.float32)
        if x.ndim != 1 or x.shape[0] != p.cols:
            raise ValueError("input must have shape [cols]")
        ms = _d(0.0)
        check(_lib.eb_benchmark(self._h, _ptr(x, ctypes.c_float), int(iterations), ctypes.byref(ms)))
        return float(ms.value)

    def _check_input(self, x: torch.Tensor, p: _Props) -> None:
        if not x.is_cuda:
            raise ValueError("forwardTorch requires a CUDA tensor")
        if x.dtype != torch.float16:
            raise ValueError("forwardTorch requires FP16 activations")
        if x.dim() < 1 or x.shape[-1] != p.cols:
            raise ValueError("forwardTorch expects activations whose last dimension equals cols")
        if x.get_device() != p.device_index:
            raise ValueError("input CUDA device does not match RuntimeMatrix device")

    def forwardTorch(self, input: torch.Tensor, bias: torch.Tensor | None = None,
                     out: torch.Tensor | None = None) -> torch.Tensor:
        """Fused unpack + dequant + linear on torch's current stream.

        ``input`` is fp16 ``[..., cols]`` (any number of rows, a superset of the
        reference's M=1 ``forwardTorch``); returns fp16 ``[..., rows]``.
        ``bias`` (fp16 [rows]) is added as torch adds it; ``out`` may supply a
        preallocated output."""
        p = self._p()
        self._check_input(input, p)
        x = input.contiguous()
        m = x.numel() // p.cols
        shape = (*x.shape[:-1], p.rows)
        if out is None:
            out = torch.empty(shape, dtype=torch.float16, device=x.device)
        elif not (out.is_cuda and out.device == x.device):
            raise ValueError("out must be on the input's device")
        elif out.dtype != torch.float16 or not out.is_contiguous() or tuple(out.shape) != shape:
            raise ValueError("out must be a contiguous fp16 tensor of the output shape")
        b = None
        if bias is not None:
            if bias.dtype != torch.float16 or bias.numel() != p.rows or bias.device != x.device:
                raise ValueError("bias must be fp16 [rows] on the input device")
            b = bias.contiguous()
        if m == 0:
            return out
        # eb_forward makes the matrix's device (checked equal to x's) current for the launch
        check(_lib.eb_forward(self._h, x.data_ptr(), m, out.data_ptr(),
                              b.data_ptr() if b is not None else None, stream_handle(p.device_index)))
        return out

    def _materializeTorch(self) -> torch.Tensor:
        """fp16 [rows, cols] decoded weights (elasticbit_runtime.cu:982-1022)."""
        p = self._p()
        if p.device_index < 0:
            raise RuntimeError("ElasticBit requires its CUDA runtime: no HIP device for this matrix")
        dev = torch.device("cuda", p.device_index)
        out = torch.empty((p.rows, p.cols), dtype=torch.float16, device=dev)
        with torch.cuda.device(dev):
            check(_lib.eb_materialize_fp16(self._h, out.data_ptr(), stream_handle(dev)))
        return out

    def _unpackCodesTorch(self) -> torch.Tensor:
        """int16 [rows, cols] codes q decoded on the device (parity probe)."""
        p = self._p()
        if p.device_index < 0:
            raise RuntimeError("ElasticBit requires its CUDA runtime: no HIP device for this matrix")
        dev = torch.device("cuda", p.device_index)
        out = torch.empty((p.rows, p.cols), dtype=torch.int16, device=dev)
        with torch.cuda.device(dev):
            check(_lib.eb_unpack_codes(self._h, out.data_ptr(), stream_handle(dev)))
        return out
