"""Execution-backend policy: ``auto`` / ``native`` / ``pytorch``.

Same contract as ``mlbricks/runtime.py:28-94``: ``auto`` lets the planner
qualify each backend-aware element once and freeze the winner, ``native``
requires the HIP route (RuntimeError when it cannot run), ``pytorch`` always
takes the PyTorch route.  Historical names are accepted as aliases.
"""
from __future__ import annotations

import warnings
from typing import Any

VALID_BACKENDS = frozenset({"auto", "native", "pytorch"})

_LEGACY = {
    "cuda": "native",
    "hip": "native",
    "cpp": "native",
    "cpp/cuda": "native",
    "torch": "pytorch",
    "python": "pytorch",
    "reference": "pytorch",
}


def normalize_backend(value: str | None = "auto", *, warn_legacy: bool = False) -> str:
    """Return the canonical backend name (runtime.py:45-64)."""
    if value is None:
        return "auto"
    name = str(value).strip().lower().replace("-", "_")
    if name in VALID_BACKENDS:
        return name
    if name in _LEGACY:
        mapped = _LEGACY[name]
        if warn_legacy:
            warnings.warn(
                f"backend={value!r} is a legacy backend name; use backend={mapped!r} instead.",
                DeprecationWarning,
                stacklevel=3,
            )
        return mapped
    raise ValueError(f"backend must be one of: auto, native, pytorch; got {value!r}.")


def set_module_backend(module: Any, backend: str, *, recursive: bool = True) -> Any:
    """Set ``backend`` on a module and its backend-aware children (runtime.py:67-94)."""
    value = normalize_backend(backend)
    setter = getattr(module, "set_backend", None)
    if callable(setter):
        try:
            return setter(value, recursive=recursive)
        except TypeError:
            setter(value)
    elif hasattr(module, "backend"):
        module.backend = value
    if recursive and hasattr(module, "modules"):
        for child in module.modules():
            if child is module:
                continue
            child_setter = getattr(child, "set_backend", None)
            if callable(child_setter):
                child_setter(value)
            elif hasattr(child, "backend"):
                child.backend = value
    return module


def backend_report(module: Any) -> list[dict[str, str]]:
    """Requested / resolved backend of every backend-aware child (runtime.py:97-125)."""
    rows: list[dict[str, str]] = []
    named = getattr(module, "named_modules", None)
    if not callable(named):
        return rows
    for name, child in named():
        if child is module and not name:
            continue
        requested = getattr(child, "backend", None)
        resolver = getattr(child, "resolved_backend", None)
        if requested is None and not callable(resolver):
            continue
        resolved = "dynamic"
        if callable(resolver):
            try:
                resolved = str(resolver())
            except TypeError:
                resolved = "dynamic-by-input"
            except Exception:
                resolved = "unavailable"
        rows.append({
            "name": name or child.__class__.__name__,
            "component": child.__class__.__name__,
            "requested": str(requested or "auto"),
            "resolved": resolved,
        })
    return rows


__all__ = ["VALID_BACKENDS", "normalize_backend", "set_module_backend", "backend_report"]
