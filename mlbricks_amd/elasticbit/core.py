"""ElasticBit adaptive threshold-driven weight compression on MI355X.

Public contract (same as ``mlbricks/elasticbit/core.py``): the user supplies
calibration data and an error threshold; ElasticBit picks the smallest storage
width b in 3..15 whose hardware-native and full-precision outputs both stay
within the threshold, with fp16 (b = 16) as the fallback.  Storage is the
canonical MLB4 bitstream with one fp32 scale per row.

Execution on gfx950 reads the b-bit codes directly -- re-laid out at load time
as bit planes, still b bits per weight -- and decodes them in registers:

* ``hardwareNative``: b <= 12 multiplies the exact integer codes (every
  |q| <= 2047 is an fp16 integer) by fp16 activations and applies the row
  scale once; b >= 13 uses the decoded fp16 weights fp16_rn(q*s) (W16A16
  arithmetic, as the reference does for b >= 9);
* ``fullPrecision``: every width uses the decoded fp16 weights;
* one fused kernel family serves decode (M <= 16, and up to 64 where it is
  faster) and prefill on the matrix cores; activations stay fp16 everywhere.

``_ElasticLinear`` routes through the execution planner: ``backend='auto'``
qualifies the HIP route against the PyTorch route (materialize + F.linear)
once per phase and freezes the winner.
"""
from __future__ import annotations

import gc
import json
import os
import tempfile
import zipfile
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Mapping, Sequence

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

from ..planner import EXECUTION_PLANNER
from ..runtime import normalize_backend
from .native_api import available as _nativeAvailable
from .native_api import importError as _nativeImportError
from .native_api import requireNative as _requireNative

_VALID_POLICIES = {"hardwareNative", "fullPrecision"}
_MODEL_FORMAT = "ElasticBitModel"
_MODEL_FORMAT_VERSION = 1
# Linear calls with at most this many activation rows qualify as "decode":
# the native route runs its decode kernel up to 64 rows, where it reads the
# weights once and leads the materialize + F.linear route by 3-4x, so a
# batched decode is not tied to the route a long prompt chose.
_DECODE_MAX_ROWS = 64


def _checkPolicy(value: str) -> str:
    value = str(value)
    if value not in _VALID_POLICIES:
        raise ValueError("decodePolicy must be 'hardwareNative' or 'fullPrecision'")
    return value


def _toNumpy2D(value: Any, *, name: str) -> np.ndarray:
    if torch.is_tensor(value):
        value = value.detach().float().cpu().numpy()
    array = np.asarray(value, dtype=np.float32)
    if array.ndim != 2:
        raise ValueError(f"{name} must be a 2D matrix")
    return np.ascontiguousarray(array, dtype=np.float32)


def _toCalibrationBatches(calibrationData: Any) -> list[Any]:
    """core.py:71-82: one batch, a mapping, or an iterable of batches."""
    if torch.is_tensor(calibrationData) or isinstance(calibrationData, Mapping):
        return [calibrationData]
    if isinstance(calibrationData, (str, bytes)):
        raise TypeError("calibrationData must contain model inputs, not text")
    try:
        batches = list(calibrationData)
    except TypeError as exc:
        raise TypeError("calibrationData must be a model input or an iterable of model inputs") from exc
    if not batches:
        raise ValueError("calibrationData cannot be empty")
    return batches


def _callModel(model: nn.Module, batch: Any) -> Any:
    if isinstance(batch, Mapping):
        return model(**batch)
    if isinstance(batch, tuple):
        return model(*batch)
    return model(batch)


def _moveBatch(batch: Any, device: torch.device) -> Any:
    if torch.is_tensor(batch):
        return batch.to(device)
    if isinstance(batch, Mapping):
        return {k: _moveBatch(v, device) for k, v in batch.items()}
    if isinstance(batch, tuple):
        return tuple(_moveBatch(v, device) for v in batch)
    if isinstance(batch, list):
        return [_moveBatch(v, device) for v in batch]
    return batch


@torch.inference_mode()
def _selectBitsTorch(weight: torch.Tensor, calibration: np.ndarray, threshold: float,
                     codesOnDevice: bool = False
                     ) -> tuple[int, float, np.ndarray | torch.Tensor | None, np.ndarray | None]:
    """Width selection on the model's GPU (core.py:112-195).

    For b = 3..15: s = max|w_r| / qmax (1 for a zero row), q = clamp(round(w/s)),
    full = F.linear(x16, fp16(q*s)), and for b <= 8 also
    hw = fp16((x16.float() @ q^T) * s); the first b with
    max(relL2(ref, hw), relL2(ref, full)) <= threshold wins, ref = F.linear(x16, W16).
    The errors of all thirteen widths come from one fused HIP pass over the
    weights (``width_errors_torch``); only the selected width is quantized
    here, and its codes and scales are returned so packing never
    re-quantizes.  ``codesOnDevice`` keeps the codes as an int16 tensor on
    the weight's device (for ``_compressSelectedCodesTorch``) instead of a
    numpy copy.
    """
    if weight.device.type != "cuda":
        raise RuntimeError("ElasticBit GPU analyzer requires CUDA weights")
    if weight.dtype != torch.float16:
        raise RuntimeError("ElasticBit GPU analyzer requires FP16 weights")
    if not np.isfinite(threshold) or float(threshold) < 0.0:
        raise ValueError("threshold must be a finite non-negative value")
    native = _requireNative()
    x16 = torch.from_numpy(np.ascontiguousarray(calibration, dtype=np.float32)).to(
        device=weight.device, dtype=torch.float16)
    w = weight.detach()
    full, hw = native.width_errors_torch(w, x16)
    for bits in range(3, 16):
        err = max(float(hw[bits - 3]), float(full[bits - 3]))
        if err <= float(threshold):
            codes, scales = _quantizeRowsTorch(w, bits)
            if not codesOnDevice:
                codes = np.ascontiguousarray(codes.cpu().numpy(), dtype=np.int16)
            return bits, err, codes, scales
    return 16, 0.0, None, None


def _quantizeRowsTorch(weight: torch.Tensor, bits: int) -> tuple[torch.Tensor, np.ndarray]:
    """Codes (int16, on the weight's device) and row scales of one width, as
    core.py:142-155 forms them."""
    w32 = weight.float()
    max_abs = w32.abs().amax(dim=1)
    qmax = float((1 << (bits - 1)) - 1)
    scale = torch.where(max_abs > 0.0, max_abs / qmax, torch.ones_like(max_abs))
    q = torch.round(w32 / scale[:, None]).clamp(min=-qmax, max=qmax)
    codes = q.to(torch.int16).contiguous()
    scales = np.ascontiguousarray(scale.float().cpu().numpy(), dtype=np.float32)
    return codes, scales


def _moduleDevice(module: nn.Module) -> torch.device:
    for p in module.parameters():
        return p.device
    for b in module.buffers():
        return b.device
    return torch.device("cpu")


def _replaceNamedModule(root: nn.Module, name: str, replacement: nn.Module) -> None:
    parts = name.split(".") if name else []
    if not parts:
        raise ValueError("ElasticBit cannot replace the root module")
    parent = root
    for part in parts[:-1]:
        parent = parent._modules[part]
    parent._modules[parts[-1]] = replacement


@dataclass(frozen=True)
class BitCandidate:
    bits: int
    hardwareNativeError: float
    fullPrecisionError: float
    error: float
    storageBytes: int
    memoryReduction: float
    passes: bool


@dataclass(frozen=True)
class BitAnalysis:
    threshold: float
    selectedBits: int
    selectedError: float
    candidates: tuple[BitCandidate, ...]


@dataclass(frozen=True)
class BackendInfo:
    available: bool
    device: str | None
    deviceIndex: int | None
    architecture: str | None
    weightWidths: tuple[int, ...]
    activateDType: str | None
    prefill: str | None
    decodePlanner: str | None
    validated: bool
    error: str | None = None
    decodeEngine: str | None = None
    decodeStatus: str | None = None
    decodeValidation: str | None = None

    def __str__(self) -> str:
        if not self.available:
            return f"ElasticBitBackend(unavailable, error={self.error!r})"
        return ("ElasticBitBackend("
                f"device={self.device!r}, architecture={self.architecture!r}, "
                f"weightWidths={self.weightWidths}, activateDType={self.activateDType!r}, "
                f"prefill={self.prefill!r}, decodePlanner={self.decodePlanner!r}, "
                f"decodeEngine={self.decodeEngine!r}, decodeStatus={self.decodeStatus!r}, "
                f"decodeValidation={self.decodeValidation!r}, validated={self.validated})")


class RuntimeMatrix:
    """Single-matrix ElasticBit runtime (core.py:264-424).

    Built only by :meth:`compress` and :meth:`load`; there is no constructor
    that takes a user-chosen bit width."""

    def __init__(self, native: Any) -> None:
        self._native = native

    @classmethod
    def compress(cls, weights: Any, calibrationData: Any, threshold: float,
                 decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        native = _requireNative()
        policy = _checkPolicy(decodePolicy)
        w = _toNumpy2D(weights, name="weights")
        c = _toNumpy2D(calibrationData, name="calibrationData")
        return cls(native.RuntimeMatrix.compress(w, c, float(threshold), policy))

    @classmethod
    def _compressSelected(cls, weights: Any, selectedBits: int, threshold: float, selectedError: float,
                          decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        native = _requireNative()
        policy = _checkPolicy(decodePolicy)
        w = _toNumpy2D(weights, name="weights")
        return cls(native.RuntimeMatrix._compressSelected(w, int(selectedBits), float(threshold),
                                                          float(selectedError), policy))

    @classmethod
    def _compressSelectedCodes(cls, codes: np.ndarray, scales: np.ndarray, selectedBits: int,
                               threshold: float, selectedError: float,
                               decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        """Pack an analyzer result as selected, without re-quantizing."""
        native = _requireNative()
        policy = _checkPolicy(decodePolicy)
        q = np.ascontiguousarray(codes, dtype=np.int16)
        s = np.ascontiguousarray(scales, dtype=np.float32)
        if q.ndim != 2:
            raise ValueError("codes must be a 2D matrix")
        if s.ndim != 1 or s.shape[0] != q.shape[0]:
            raise ValueError("scales must contain one value per weight row")
        return cls(native.RuntimeMatrix._compressSelectedCodes(q, s, int(selectedBits), float(threshold),
                                                               float(selectedError), policy))

    @classmethod
    def _compressSelectedCodesTorch(cls, codes: torch.Tensor, scales: np.ndarray, selectedBits: int,
                                    threshold: float, selectedError: float,
                                    decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        """_compressSelectedCodes for codes that are an int16 tensor on the
        HIP device: packed on the device, without a host copy of the codes."""
        native = _requireNative()
        policy = _checkPolicy(decodePolicy)
        return cls(native.RuntimeMatrix._compressSelectedCodesTorch(codes, scales, int(selectedBits),
                                                                    float(threshold), float(selectedError), policy))

    @classmethod
    def load(cls, path: str | Path, decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        native = _requireNative()
        policy = _checkPolicy(decodePolicy)
        return cls(native.RuntimeMatrix.load(str(path), policy))

    def forward(self, x: Any) -> Any:
        """GPU fp16 activations stay on the device (any number of rows);
        anything else takes the host round trip of one row."""
        if torch.is_tensor(x):
            if x.is_cuda and x.dtype == torch.float16 and x.dim() >= 1 and x.shape[-1] == self.cols:
                return self._native.forwardTorch(x.contiguous())
            values = np.asarray(x.detach().float().cpu().numpy(), dtype=np.float32).reshape(-1)
            out = self._native.forward(np.ascontiguousarray(values))
            return torch.from_numpy(np.asarray(out)).to(device=x.device, dtype=x.dtype)
        values = np.asarray(x, dtype=np.float32).reshape(-1)
        return np.asarray(self._native.forward(np.ascontiguousarray(values)))

    @staticmethod
    def forwardTorchMulti(matrices: Sequence["RuntimeMatrix"], x: torch.Tensor,
                          biases: Sequence[torch.Tensor | None] | None = None) -> list[torch.Tensor]:
        """``[m.forward(x) (+ bias) for m in matrices]`` for matrices that read
        the same fp16 CUDA activations, in one decode launch per run of equal
        widths (up to four matrices; up to 16 activation rows, or 64 where the
        decode kernel is the faster route).  No
        single-call counterpart in the reference (its Stage-2F concatenates
        the materialized weights, stage2f.py:382-420)."""
        native = _requireNative()
        return native.forward_torch_multi([m._native for m in matrices], x, biases)

    def benchmark(self, x: Any, iterations: int = 500) -> float:
        if torch.is_tensor(x):
            x = x.detach().float().cpu().numpy()
        values = np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))
        return float(self._native.benchmark(values, int(iterations)))

    def dequantize(self) -> np.ndarray:
        return np.asarray(self._native.dequantize(), dtype=np.float32)

    def _materializeTorch(self) -> torch.Tensor:
        return self._native._materializeTorch()

    def save(self, path: str | Path) -> None:
        self._native.save(str(path))

    def setDecodePolicy(self, decodePolicy: str) -> "RuntimeMatrix":
        self._native.setDecodePolicy(_checkPolicy(decodePolicy))
        return self

    @property
    def rows(self) -> int:
        return int(self._native.rows)

    @property
    def cols(self) -> int:
        return int(self._native.cols)

    @property
    def shape(self) -> tuple[int, int]:
        return tuple(int(v) for v in self._native.shape)

    @property
    def storageBits(self) -> int:
        return int(self._native.storageBits)

    @property
    def executionWidth(self) -> int:
        return int(self._native.executionWidth)

    @property
    def executionPlanner(self) -> str:
        return str(self._native.executionPlanner)

    @property
    def decodePolicy(self) -> str:
        return str(self._native.decodePolicy)

    @property
    def activateDType(self) -> str:
        return str(self._native.activateDType)

    @property
    def storageBytes(self) -> int:
        return int(self._native.storageBytes)

    @property
    def executionBytes(self) -> int:
        return int(self._native.executionBytes)

    @property
    def originalBytes(self) -> int:
        return int(self._native.originalBytes)

    @property
    def memoryReduction(self) -> float:
        return float(self._native.memoryReduction)

    @property
    def threshold(self) -> float:
        return float(self._native.threshold)

    @property
    def error(self) -> float:
        return float(self._native.error)


class _RouteOwner:
    """Holds the planner's frozen route for one phase of one layer."""

    __slots__ = ("_mlbricks_frozen_auto_routes", "_mlbricks_frozen_auto_details", "_mlbricks_auto_route_cache")

    def __init__(self) -> None:
        self._mlbricks_frozen_auto_routes: dict = {}
        self._mlbricks_frozen_auto_details: dict = {}
        self._mlbricks_auto_route_cache = None


class _ElasticLinear(nn.Module):
    """Compressed Linear (core.py:427-471), routed through the execution planner."""

    def __init__(self, matrix: RuntimeMatrix, inFeatures: int, outFeatures: int,
                 bias: torch.Tensor | None, backend: str = "auto") -> None:
        super().__init__()
        self.matrix = matrix
        self.inFeatures = int(inFeatures)
        self.outFeatures = int(outFeatures)
        self.backend = normalize_backend(backend)
        if bias is None:
            self.register_parameter("bias", None)
        else:
            self.bias = nn.Parameter(bias.detach().clone(), requires_grad=False)
        self._routeOwners = {"decode": _RouteOwner(), "prefill": _RouteOwner()}

    def set_backend(self, backend: str, recursive: bool = True) -> "_ElasticLinear":
        self.backend = normalize_backend(backend)
        for owner in self._routeOwners.values():
            EXECUTION_PLANNER.clear_owner_routes(owner)
        return self

    def resolved_backend(self) -> str:
        routes = {phase: EXECUTION_PLANNER.owner_routes(owner) for phase, owner in self._routeOwners.items()}
        frozen = {phase: next(iter(r.values())) for phase, r in routes.items() if r}
        if self.backend != "auto":
            return self.backend
        if not frozen:
            return "auto"
        return ",".join(f"{phase}={route}" for phase, route in sorted(frozen.items()))

    def _forwardNative(self, x: torch.Tensor) -> torch.Tensor:
        bias = self.bias
        if bias is not None and (bias.dtype != torch.float16 or bias.device != x.device):
            bias = bias.to(device=x.device, dtype=torch.float16)
        return self.matrix._native.forwardTorch(x, bias=bias)

    def _forwardPytorch(self, x: torch.Tensor) -> torch.Tensor:
        weight = self.matrix._materializeTorch()
        if weight.device != x.device:
            raise RuntimeError("ElasticBit Linear expects activations on the device that holds its matrix")
        if weight.dtype != x.dtype:
            weight = weight.to(dtype=x.dtype)
        bias = self.bias
        if bias is not None and (bias.device != x.device or bias.dtype != x.dtype):
            bias = bias.to(device=x.device, dtype=x.dtype)
        return F.linear(x, weight, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.inFeatures:
            raise ValueError(f"ElasticBit Linear expected last dimension {self.inFeatures}, got {x.shape[-1]}")
        rows = x.numel() // self.inFeatures
        native_ok = (_nativeAvailable() and x.is_cuda and x.dtype == torch.float16
                     and self.matrix._native.deviceIndex == x.get_device())
        training = bool(torch.is_grad_enabled() and x.requires_grad)
        phase = "decode" if rows <= _DECODE_MAX_ROWS else "prefill"
        xc = x.contiguous() if native_ok else x
        route = EXECUTION_PLANNER.qualify_operator_once(
            self._routeOwners[phase], "elastic_linear", xc,
            {"native": lambda: self._forwardNative(xc), "pytorch": lambda: self._forwardPytorch(x)},
            requested_backend=self.backend, native_available=native_ok, training=training,
            extra=(self.outFeatures, self.inFeatures, self.matrix.storageBits, phase),
            default_auto="pytorch",
        )
        if route == "native":
            return self._forwardNative(xc)
        return self._forwardPytorch(x)


class _ModelElasticBit:
    """``model.elasticbit`` controller (core.py:474-547)."""

    def __init__(self, model: nn.Module, threshold: float, decodePolicy: str, compressedNames: Sequence[str],
                 skippedNames: Sequence[str], optimizationProfiles: Mapping[str, Any] | None = None) -> None:
        self._model = model
        self.threshold = float(threshold)
        self.decodePolicy = _checkPolicy(decodePolicy)
        self.compressedNames = tuple(compressedNames)
        self.skippedNames = tuple(skippedNames)
        self.optimizationProfiles = dict(optimizationProfiles or {})
        self.activeOptimization: dict[str, Any] | None = None

    def _layers(self) -> list[tuple[str, _ElasticLinear]]:
        modules = dict(self._model.named_modules())
        return [(n, modules[n]) for n in self.compressedNames if isinstance(modules.get(n), _ElasticLinear)]

    def setDecodePolicy(self, decodePolicy: str) -> "_ModelElasticBit":
        policy = _checkPolicy(decodePolicy)
        seen: set[int] = set()
        for _, layer in self._layers():
            if id(layer.matrix) in seen:
                continue
            layer.matrix.setDecodePolicy(policy)
            seen.add(id(layer.matrix))
        self.decodePolicy = policy
        return self

    def summary(self) -> str:
        backend = ElasticBit.backend()
        lines = [
            "ElasticBit Summary",
            "-" * 60,
            f"Threshold       : {self.threshold}",
            f"Decode Policy   : {self.decodePolicy}",
            f"Backend         : {backend.architecture or 'unavailable'}",
            f"Prefill         : {backend.prefill or 'unknown'}",
            f"Decode Engine   : {backend.decodeEngine or 'unknown'}",
            f"Decode Status   : {backend.decodeStatus or 'unknown'}",
            f"Decode Planner  : {backend.decodePlanner or 'unknown'}",
            f"Decode Validate : {backend.decodeValidation or 'unknown'}",
            f"Activate DType  : {backend.activateDType or 'unknown'}",
            "",
            f"{'Layer':36s} {'Stored':>8s} {'Execute':>10s} {'Planner':>14s} {'Error':>10s}",
        ]
        for name, layer in self._layers():
            m = layer.matrix
            lines.append(f"{name[:36]:36s} {str(m.storageBits) + '-bit':>8s} "
                         f"{'W' + str(m.executionWidth) + 'A16':>10s} {m.executionPlanner:>14s} {m.error:10.6f}")
        if self.skippedNames:
            lines.extend(["", "Uncompressed (no safe calibration path):"])
            lines.extend(f"  {n}" for n in self.skippedNames)
        text = "\n".join(lines)
        print(text)
        return text


def _semanticOutputWeightIds(model: nn.Module) -> set[int]:
    """Weights of the model's token-output head via ``get_output_embeddings()`` (core.py:550-568)."""
    getter = getattr(model, "get_output_embeddings", None)
    if not callable(getter):
        return set()
    try:
        output = getter()
    except Exception:
        return set()
    if isinstance(output, nn.Linear):
        return {id(output.weight)}
    return set()


class ElasticBit:
    """Public namespace (core.py:571-1017)."""

    RuntimeMatrix = RuntimeMatrix

    @staticmethod
    def analyze(weights: Any, calibrationData: Any, threshold: float) -> BitAnalysis:
        native = _requireNative()
        w = _toNumpy2D(weights, name="weights")
        c = _toNumpy2D(calibrationData, name="calibrationData")
        raw = native.analyze(w, c, float(threshold))
        candidates = tuple(
            BitCandidate(bits=int(i["bits"]), hardwareNativeError=float(i["hardwareNativeError"]),
                         fullPrecisionError=float(i["fullPrecisionError"]), error=float(i["error"]),
                         storageBytes=int(i["storageBytes"]), memoryReduction=float(i["memoryReduction"]),
                         passes=bool(i["passes"]))
            for i in raw["candidates"])
        return BitAnalysis(threshold=float(raw["threshold"]), selectedBits=int(raw["selectedBits"]),
                           selectedError=float(raw["selectedError"]), candidates=candidates)

    @staticmethod
    def compressMatrix(weights: Any, calibrationData: Any, threshold: float,
                       decodePolicy: str = "hardwareNative") -> RuntimeMatrix:
        return RuntimeMatrix.compress(weights, calibrationData, threshold, decodePolicy=decodePolicy)

    @staticmethod
    def loadMatrix(path: str | Path, decodePolicy: str = "hardwareNative") -> RuntimeMatrix:
        return RuntimeMatrix.load(path, decodePolicy=decodePolicy)

    @staticmethod
    def backend() -> BackendInfo:
        if not _nativeAvailable():
            err = _nativeImportError()
            return BackendInfo(available=False, device=None, deviceIndex=None, architecture=None,
                               weightWidths=(), activateDType=None, prefill=None, decodePlanner=None,
                               decodeEngine=None, decodeStatus=None, decodeValidation=None, validated=False,
                               error=None if err is None else str(err))
        raw = _requireNative().backendInfo()
        if not raw["available"]:
            return BackendInfo(available=False, device=None, deviceIndex=None, architecture=None,
                               weightWidths=tuple(raw["weightWidths"]), activateDType=raw["activateDType"],
                               prefill=None, decodePlanner=None, decodeEngine=None, decodeStatus=None,
                               decodeValidation=None, validated=False,
                               error="no HIP device is visible to the ElasticBit runtime")
        return BackendInfo(available=True, device=str(raw["device"]), deviceIndex=int(raw["deviceIndex"]),
                           architecture=str(raw["architecture"]),
                           weightWidths=tuple(int(v) for v in raw["weightWidths"]),
                           activateDType=str(raw["activateDType"]), prefill=str(raw["prefill"]),
                           decodePlanner=str(raw["decodePlanner"]), decodeEngine=str(raw["decodeEngine"]),
                           decodeStatus=str(raw["decodeStatus"]), decodeValidation=str(raw["decodeValidation"]),
                           validated=bool(raw["validated"]))

    @staticmethod
    def optimize(model: nn.Module, force: bool = False) -> nn.Module:
        """Stage-2F profile tuning (reference stage2f.py) is Tesla-T4/Granite-specific
        and not part of the MI355X build."""
        raise NotImplementedError("ElasticBit.optimize (Stage-2F) is not available in the MI355X build")

    @staticmethod
    def reduce(model: nn.Module, sample: Any = None) -> nn.Module:
        """Stage-2G FX reduction (reference stage2g.py) is not part of the MI355X build."""
        raise NotImplementedError("ElasticBit.reduce (Stage-2G) is not available in the MI355X build")

    @staticmethod
    def compress(model: nn.Module, calibrationData: Any, threshold: float, decodePolicy: str = "hardwareNative",
                 preserveOutputHead: bool = True) -> nn.Module:
        """Compress every unprotected fp16 nn.Linear of ``model`` (core.py:695-898)."""
        if not isinstance(model, nn.Module):
            raise TypeError("ElasticBit.compress() expects a torch.nn.Module")
        _requireNative()
        policy = _checkPolicy(decodePolicy)
        batches = _toCalibrationBatches(calibrationData)
        device = _moduleDevice(model)
        if device.type != "cuda":
            raise RuntimeError("ElasticBit model compression currently requires a CUDA model")
        for module in model.modules():
            if isinstance(module, nn.Linear) and module.weight.dtype != torch.float16:
                raise RuntimeError("ElasticBit.compress() currently requires FP16 Linear weights. "
                                   "Convert the model to float16 before compression.")

        embedding_ids = {id(m.weight) for m in model.modules() if isinstance(m, nn.Embedding)}
        output_ids = _semanticOutputWeightIds(model) if bool(preserveOutputHead) else set()
        protected = embedding_ids | output_ids

        collected: dict[str, list[np.ndarray]] = {}
        max_rows = 32          # calibration rows kept per Linear (core.py:734)

        def make_hook(name: str):
            def hook(_module: nn.Module, inputs: tuple[Any, ...]) -> None:
                if not inputs or not torch.is_tensor(inputs[0]):
                    return
                rows = inputs[0].detach().float().reshape(-1, inputs[0].shape[-1])
                remaining = max_rows - sum(a.shape[0] for a in collected.get(name, []))
                if remaining <= 0:
                    return
                collected.setdefault(name, []).append(rows[:remaining].cpu().numpy().astype(np.float32, copy=True))
            return hook

        handles = []
        linears: list[tuple[str, nn.Linear]] = []
        for name, module in model.named_modules():
            if isinstance(module, nn.Linear):
                linears.append((name, module))
                if id(module.weight) not in protected:
                    handles.append(module.register_forward_pre_hook(make_hook(name)))
        model.eval()
        try:
            with torch.inference_mode():
                for batch in batches:
                    _callModel(model, _moveBatch(batch, device))
        finally:
            for h in handles:
                h.remove()

        names_by_weight: dict[int, list[str]] = {}
        for name, module in linears:
            names_by_weight.setdefault(id(module.weight), []).append(name)
        del linears
        compressed: list[str] = []
        skipped: list[str] = [n for wid, names in names_by_weight.items() if wid in output_ids for n in names]
        progress = os.environ.get("MLBRICKS_ELASTICBIT_PROGRESS", "").strip().lower() in {"1", "true", "yes", "on"}
        work = [(wid, names) for wid, names in names_by_weight.items() if wid not in protected]

        for index, (_, names) in enumerate(work, start=1):
            module = model.get_submodule(names[0])
            if not isinstance(module, nn.Linear):
                raise RuntimeError(f"ElasticBit expected Linear module at {names[0]}")
            samples = [a for n in names for a in collected.get(n, [])]
            if not samples:
                skipped.extend(names)
                continue
            calibration = np.ascontiguousarray(np.concatenate(samples, axis=0), dtype=np.float32)
            if progress:
                print(f"[ElasticBit] {index}/{len(work)} analyzing {names[0]} "
                      f"shape={tuple(module.weight.shape)} rows={calibration.shape[0]}", flush=True)
            bits, err, codes, scales = _selectBitsTorch(module.weight, calibration, float(threshold),
                                                        codesOnDevice=True)
            if progress:
                print(f"[ElasticBit] {index}/{len(work)} selected {bits}-bit error={err:.6g}", flush=True)
            with torch.cuda.device(device):
                if bits <= 15:
                    matrix = RuntimeMatrix._compressSelectedCodesTorch(codes, scales, bits, float(threshold), err,
                                                                       decodePolicy=policy)
                else:
                    weights = np.ascontiguousarray(module.weight.detach().cpu().float().numpy(), dtype=np.float32)
                    matrix = RuntimeMatrix._compressSelected(weights, bits, float(threshold), err,
                                                             decodePolicy=policy)
            for name in names:
                current = model.get_submodule(name)
                if not isinstance(current, nn.Linear):
                    raise RuntimeError(f"ElasticBit expected Linear module at {name}")
                replacement = _ElasticLinear(matrix=matrix, inFeatures=current.in_features,
                                             outFeatures=current.out_features, bias=current.bias).to(device=device)
                _replaceNamedModule(model, name, replacement)
                compressed.append(name)
                collected.pop(name, None)
            del module, codes, scales, calibration, samples, matrix
            gc.collect()
            torch.cuda.empty_cache()

        model.elasticbit = _ModelElasticBit(model, threshold=float(threshold), decodePolicy=policy,
                                            compressedNames=compressed, skippedNames=skipped)
        return model

    @staticmethod
    def save(model: nn.Module, path: str | Path) -> Path:
        """Zip artifact: manifest.json, matrices/matrix_%05d.mlb, state.pt (core.py:900-955)."""
        controller = getattr(model, "elasticbit", None)
        if not isinstance(controller, _ModelElasticBit):
            raise ValueError("ElasticBit.save() expects a model produced by ElasticBit.compress()")
        destination = Path(path)
        destination.parent.mkdir(parents=True, exist_ok=True)
        modules = dict(model.named_modules())
        with tempfile.TemporaryDirectory(prefix="elasticbit-save-") as tmp:
            root = Path(tmp)
            (root / "matrices").mkdir()
            layers = []
            saved: dict[int, str] = {}
            for name in controller.compressedNames:
                layer = modules.get(name)
                if not isinstance(layer, _ElasticLinear):
                    raise RuntimeError(f"ElasticBit layer disappeared before save: {name}")
                file = saved.get(id(layer.matrix))
                if file is None:
                    file = f"matrix_{len(saved):05d}.mlb"
                    layer.matrix.save(root / "matrices" / file)
                    saved[id(layer.matrix)] = file
                layers.append({"name": name, "matrix": file, "inFeatures": layer.inFeatures,
                               "outFeatures": layer.outFeatures, "hasBias": layer.bias is not None})
            manifest = {
                "format": _MODEL_FORMAT,
                "version": _MODEL_FORMAT_VERSION,
                "threshold": controller.threshold,
                "decodePolicy": controller.decodePolicy,
                "compressedNames": list(controller.compressedNames),
                "skippedNames": list(controller.skippedNames),
                "optimizationProfiles": controller.optimizationProfiles,
                "layers": layers,
            }
            (root / "manifest.json").write_text(json.dumps(manifest, indent=2), encoding="utf-8")
            torch.save(model.state_dict(), root / "state.pt")
            with zipfile.ZipFile(destination, "w", compression=zipfile.ZIP_DEFLATED) as archive:
                for file in sorted(root.rglob("*")):
                    if file.is_file():
                        archive.write(file, file.relative_to(root).as_posix())
        return destination

    @staticmethod
    def load(model: nn.Module, path: str | Path, decodePolicy: str = "hardwareNative") -> nn.Module:
        """Rebuild compressed layers into an architecture instance (core.py:957-1017)."""
        if not isinstance(model, nn.Module):
            raise TypeError("ElasticBit.load() requires the model architecture as its first argument")
        _requireNative()
        source = Path(path)
        if not source.exists():
            raise FileNotFoundError(source)
        with tempfile.TemporaryDirectory(prefix="elasticbit-load-") as tmp:
            root = Path(tmp)
            with zipfile.ZipFile(source, "r") as archive:
                archive.extractall(root)
            manifest = json.loads((root / "manifest.json").read_text(encoding="utf-8"))
            if manifest.get("format") != _MODEL_FORMAT or manifest.get("version") != _MODEL_FORMAT_VERSION:
                raise ValueError("Unsupported ElasticBit model artifact")
            policy = _checkPolicy(decodePolicy)
            modules = dict(model.named_modules())
            cache: dict[str, RuntimeMatrix] = {}
            compressed: list[str] = []
            for entry in manifest["layers"]:
                name = str(entry["name"])
                target = modules.get(name)
                if not isinstance(target, nn.Linear):
                    raise ValueError(f"Model architecture does not contain expected Linear layer: {name}")
                device = target.weight.device
                if device.type != "cuda":
                    raise RuntimeError("ElasticBit.load() requires the target model on CUDA")
                file = str(entry["matrix"])
                matrix = cache.get(file)
                if matrix is None:
                    with torch.cuda.device(device):
                        matrix = RuntimeMatrix.load(root / "matrices" / file, decodePolicy=policy)
                    cache[file] = matrix
                replacement = _ElasticLinear(matrix=matrix, inFeatures=int(entry["inFeatures"]),
                                             outFeatures=int(entry["outFeatures"]),
                                             bias=target.bias if bool(entry["hasBias"]) else None).to(device=device)
                _replaceNamedModule(model, name, replacement)
                compressed.append(name)
                modules[name] = replacement
            state = torch.load(root / "state.pt", map_location=_moduleDevice(model), weights_only=True)
            model.load_state_dict(state, strict=True)
            model.elasticbit = _ModelElasticBit(model, threshold=float(manifest["threshold"]), decodePolicy=policy,
                                                compressedNames=compressed,
                                                skippedNames=tuple(manifest.get("skippedNames", ())),
                                                optimizationProfiles=manifest.get("optimizationProfiles", {}))
            return model


__all__ = ["ElasticBit", "RuntimeMatrix", "BitAnalysis", "BitCandidate", "BackendInfo"]
