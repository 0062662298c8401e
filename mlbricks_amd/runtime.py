"""Execution-backend policy shared by every backend-aware element.

Three names (the contract of ``mlbricks/runtime.py``):

* ``auto`` -- the planner qualifies each element on its first eligible call
  and freezes the winner on that element;
* ``native`` -- the HIP implementation is required (``RuntimeError`` when it
  cannot serve a call);
* ``pytorch`` -- the PyTorch implementation always.

Older spellings are accepted and mapped onto these, with a
``DeprecationWarning`` when the caller asks for one.
"""
from __future__ import annotations

import warnings
from typing import Any, Iterator

VALID_BACKENDS = frozenset({"auto", "native", "pytorch"})

# Historical names, grouped by the backend they stand for.
_ALIASES_BY_BACKEND = {
    "native": ("cuda", "hip", "rocm", "cpp", "cpp/cuda"),
    "pytorch": ("torch", "python", "reference"),
}
_ALIAS = {alias: backend for backend, aliases in _ALIASES_BY_BACKEND.items() for alias in aliases}


def normalize_backend(value: str | None = "auto", *, warn_legacy: bool = False) -> str:
    """The canonical backend for ``value`` (None means ``auto``); case,
    surrounding blanks and ``-`` versus ``_`` do not matter."""
    if value is None:
        return "auto"
    key = str(value).strip().lower().replace("-", "_")
    if key in VALID_BACKENDS:
        return key
    backend = _ALIAS.get(key)
    if backend is None:
        raise ValueError(f"backend must be one of: auto, native, pytorch; got {value!r}.")
    if warn_legacy:
        warnings.warn(f"backend={value!r} is a legacy backend name; use backend={backend!r} instead.",
                      DeprecationWarning, stacklevel=3)
    return backend


def _elements(module: Any, recursive: bool) -> Iterator[Any]:
    """The module itself, then (when recursive) every descendant once."""
    yield module
    walk = getattr(module, "modules", None)
    if recursive and callable(walk):
        for child in walk():
            if child is not module:
                yield child


def _assign(element: Any, backend: str) -> None:
    """Give one element the backend: through its ``set_backend`` when it has
    one (non-recursively, the walk covers its children), else its
    ``backend`` attribute when it has one."""
    setter = getattr(element, "set_backend", None)
    if callable(setter):
        try:
            setter(backend, recursive=False)
        except TypeError:
            setter(backend)
    elif hasattr(element, "backend"):
        element.backend = backend


def set_module_backend(module: Any, backend: str, *, recursive: bool = True) -> Any:
    """Set ``backend`` on a module and, by default, on all its backend-aware
    descendants (runtime.py:67-94).  Returns the module."""
    value = normalize_backend(backend)
    for element in _elements(module, recursive):
        _assign(element, value)
    return module


def _resolved(element: Any) -> str:
    resolver = getattr(element, "resolved_backend", None)
    if not callable(resolver):
        return "dynamic"
    try:
        return str(resolver())
    except TypeError:
        return "dynamic-by-input"
    except Exception:
        return "unavailable"


def backend_report(module: Any) -> list[dict[str, str]]:
    """One row per backend-aware descendant: its name, class, requested and
    resolved backend (runtime.py:97-125)."""
    walk = getattr(module, "named_modules", None)
    if not callable(walk):
        return []
    report = []
    for name, element in walk():
        if element is module and not name:
            continue
        requested = getattr(element, "backend", None)
        if requested is None and not callable(getattr(element, "resolved_backend", None)):
            continue
        report.append({"name": name or type(element).__name__, "component": type(element).__name__,
                       "requested": str(requested or "auto"), "resolved": _resolved(element)})
    return report


__all__ = ["VALID_BACKENDS", "normalize_backend", "set_module_backend", "backend_report"]
