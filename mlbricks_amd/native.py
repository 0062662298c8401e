"""Direct packed linear op ``elastic_linear_packed`` (the legacy flat-group
ElasticBit op of ``mlbricks/esa/native.py:864-882``).

``y = x . W^T + bias`` with ``W[o][k] = (u - 2^(b-1)) * scales[(o*K + k) // group_size]``
read straight from the LSB-first packed stream, 2 <= b <= 8.  The op is also
registered as ``torch.ops.mlbricks_native.elastic_linear_packed`` (with a fake
kernel for meta tensors) by ``mlbricks_amd.custom_ops``.
"""
from __future__ import annotations

import torch

from .elasticbit.native_api import available as _available
from .elasticbit.native_api import importError as _importError
from .elasticbit.native_api import requireNative as _requireNative


def elastic_linear_packed(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor,
                          bits: int, group_size: int, out_features: int, in_features: int) -> torch.Tensor:
    """Packed ElasticBit linear without materializing the weight (bolt/ops.cpp:1012-1043)."""
    if not _available():
        raise RuntimeError(f"MLBricks native extension is unavailable: {_importError()}")
    if not x.is_cuda:
        raise RuntimeError("elastic_linear_packed requires CUDA")
    native = _requireNative()
    x = x.contiguous()
    packed = packed.contiguous()
    scales = scales.contiguous()
    bias = bias.contiguous() if bias is not None else None
    if not (x.is_floating_point() and scales.is_floating_point()):
        raise RuntimeError("x/scales must be floating point")
    if packed.dtype != torch.uint8:
        raise RuntimeError("packed weight must be uint8")
    if x.shape[-1] != int(in_features):
        raise RuntimeError("input feature mismatch")
    if not 2 <= int(bits) <= 8:
        raise RuntimeError("bits must be in [2,8]")
    if int(group_size) <= 0 or int(out_features) <= 0 or int(in_features) <= 0:
        raise RuntimeError("invalid ElasticBit dimensions")
    if packed.device != x.device or scales.device != x.device:
        raise RuntimeError("ElasticBit buffers must be on the same CUDA device as x")
    has_bias = bias is not None and bias.numel() != 0
    if has_bias and (bias.device != x.device or bias.dtype != x.dtype or bias.numel() != int(out_features)):
        raise RuntimeError("bias must be empty or match output features/device/dtype")
    needed_bits = int(out_features) * int(in_features) * int(bits)
    if packed.numel() * 8 < needed_bits:
        raise RuntimeError("packed weight is smaller than out_features * in_features * bits")
    needed_groups = (int(out_features) * int(in_features) + int(group_size) - 1) // int(group_size)
    if scales.numel() < needed_groups:
        raise RuntimeError("scales must hold one value per group")
    return native.packed_linear(x, packed, scales, bias if has_bias else None, int(bits), int(group_size),
                                int(out_features), int(in_features))


__all__ = ["elastic_linear_packed"]
