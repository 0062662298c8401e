"""Loader for the ElasticBit HIP runtime (libelasticbit_hip.so).

Mirrors ``mlbricks/elasticbit/native_api.py``: ``available()``,
``importError()`` and ``requireNative()``.  The native module is the ctypes
binding in ``_native``; there is no other implementation to fall back to.
"""
from __future__ import annotations

import importlib

try:
    _C = importlib.import_module(f"{__package__}._native")
except Exception as exc:  # pragma: no cover - depends on whether the library is built
    _C = None
    _IMPORT_ERROR = exc
else:
    _IMPORT_ERROR = None


def available() -> bool:
    return _C is not None


def importError() -> Exception | None:
    return _IMPORT_ERROR


def requireNative():
    if _C is None:
        raise RuntimeError(
            "ElasticBit requires its CUDA runtime: the HIP library libelasticbit_hip.so "
            "(gfx950) is not built. Run `python -m mlbricks_amd.csrc.build`."
        ) from _IMPORT_ERROR
    return _C


__all__ = ["available", "importError", "requireNative"]
