"""torch.library registration of ``mlbricks_native::elastic_linear_packed``.

Same schema as bolt/ops.cpp:1132, with a fake (meta) kernel returning
``x.new_empty((*x.shape[:-1], out_features))`` as custom_ops.py:220-230 does,
so the op is visible to torch.compile / FakeTensor tracing.  Registration is
idempotent and skipped when another library already defined the namespace.
"""
from __future__ import annotations

import torch

from .native import elastic_linear_packed as _elastic_linear_packed

_SCHEMA = ("elastic_linear_packed(Tensor x, Tensor packed, Tensor scales, Tensor bias, int bits, "
           "int group_size, int out_features, int in_features) -> Tensor")
_LIB: torch.library.Library | None = None
_ERROR: Exception | None = None


def _register() -> None:
    global _LIB, _ERROR
    try:
        lib = torch.library.Library("mlbricks_native", "DEF")
        lib.define(_SCHEMA)

        def _impl(x, packed, scales, bias, bits, group_size, out_features, in_features):
            return _elastic_linear_packed(x, packed, scales, bias, bits, group_size, out_features, in_features)

        lib.impl("elastic_linear_packed", _impl, "CUDA")

        def _fake(x, packed, scales, bias, bits, group_size, out_features, in_features):
            return x.new_empty((*x.shape[:-1], out_features))

        torch.library.register_fake("mlbricks_native::elastic_linear_packed", _fake, lib=lib)
        _LIB = lib
    except Exception as exc:  # pragma: no cover - namespace already owned elsewhere
        _ERROR = exc


_register()


def custom_ops_registered() -> bool:
    return _LIB is not None


def custom_ops_error() -> Exception | None:
    return _ERROR


__all__ = ["custom_ops_registered", "custom_ops_error"]
