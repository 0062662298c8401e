"""ElasticBit: threshold-driven weight compression with a HIP execution path.

The public contract is that of ``mlbricks/elasticbit/core.py``.  Given
calibration inputs and an error threshold, each ``nn.Linear`` gets the smallest
storage width b in 3..15 whose outputs stay within the threshold, else fp16
(b = 16).  Storage is the canonical MLB4 bitstream with one fp32 scale per
output row.  Names, signatures, error messages and the ``.elasticbit`` zip
layout are kept so that the module drops in; the implementation is this
package's own.

Execution on gfx950 keeps the b-bit codes on the device (re-laid out as bit
planes, still b bits per weight) and decodes them in registers:

* ``hardwareNative``: for b <= 12 the exact integer codes (every |q| <= 2047
  is an fp16 integer) multiply the fp16 activations and the row scale is
  applied once; b >= 13 uses the decoded weights fp16_rn(q*s);
* ``fullPrecision``: the decoded weights at every width.

``_ElasticLinear`` routes each call through the execution planner.  Under
``backend='auto'`` it qualifies the HIP route against the PyTorch route, once
per phase, and freezes the winner.  The PyTorch route is what the reference
executes: ``F.linear`` on a resident fp16 copy of the weights for b >= 9,
and on a copy materialized per call for b <= 8.
"""
from __future__ import annotations

import gc
import io
import json
import os
import tempfile
import zipfile
from dataclasses import dataclass, fields
from pathlib import Path
from typing import Any, Callable, Iterable, Mapping, Sequence

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

from ..planner import EXECUTION_PLANNER
from ..runtime import normalize_backend
from .native_api import available as _nativeAvailable
from .native_api import importError as _nativeImportError
from .native_api import requireNative as _requireNative

DECODE_POLICIES = ("hardwareNative", "fullPrecision")
ARTIFACT_FORMAT = ("ElasticBitModel", 1)          # manifest "format", "version"
CALIBRATION_ROWS = 32                             # kept per Linear (core.py:734)
# Calls with at most this many activation rows are the "decode" phase: the
# native route runs its decode kernel up to 64 rows, so a batched decode is
# qualified apart from a long prompt.
DECODE_PHASE_ROWS = 64
_RESIDENT_MIN_BITS = 9                            # the reference keeps fp16 resident from here


# -- argument coercion ----------------------------------------------------------

def _checkPolicy(value: str) -> str:
    policy = str(value)
    if policy in DECODE_POLICIES:
        return policy
    raise ValueError("decodePolicy must be 'hardwareNative' or 'fullPrecision'")


def _matrix_f32(value: Any, name: str) -> np.ndarray:
    """A C-contiguous float32 2-D copy of a tensor or array-like."""
    host = value.detach().to("cpu", torch.float32).numpy() if torch.is_tensor(value) else value
    array = np.ascontiguousarray(host, dtype=np.float32)
    if array.ndim != 2:
        raise ValueError(f"{name} must be a 2D matrix")
    return array


def _batch_list(calibrationData: Any) -> list[Any]:
    """Calibration as a list of model inputs (core.py:71-82): one tensor or
    mapping is a single batch; any other iterable is a sequence of batches."""
    if torch.is_tensor(calibrationData) or isinstance(calibrationData, Mapping):
        return [calibrationData]
    if isinstance(calibrationData, (str, bytes)):
        raise TypeError("calibrationData must contain model inputs, not text")
    try:
        batches = [batch for batch in calibrationData]
    except TypeError as exc:
        raise TypeError("calibrationData must be a model input or an iterable of model inputs") from exc
    if not batches:
        raise ValueError("calibrationData cannot be empty")
    return batches


def _on_device(batch: Any, device: torch.device) -> Any:
    if torch.is_tensor(batch):
        return batch.to(device)
    if isinstance(batch, Mapping):
        return {key: _on_device(item, device) for key, item in batch.items()}
    if isinstance(batch, (tuple, list)):
        return type(batch)(_on_device(item, device) for item in batch)
    return batch


def _feed(model: nn.Module, batch: Any) -> None:
    """Run one calibration batch: keyword inputs, positional inputs, or one input."""
    if isinstance(batch, Mapping):
        model(**batch)
    elif isinstance(batch, tuple):
        model(*batch)
    else:
        model(batch)


def _device_of(module: nn.Module) -> torch.device:
    tensor = next(iter(module.parameters()), None)
    if tensor is None:
        tensor = next(iter(module.buffers()), None)
    return torch.device("cpu") if tensor is None else tensor.device


def _replaceNamedModule(root: nn.Module, name: str, replacement: nn.Module) -> None:
    """Swap the submodule at dotted path ``name``; the root itself cannot be
    replaced (core.py:206-213)."""
    if not name:
        raise ValueError("ElasticBit cannot replace the root module")
    parent_name, _, leaf = name.rpartition(".")
    parent = root.get_submodule(parent_name) if parent_name else root
    parent._modules[leaf] = replacement


# -- GPU width selection --------------------------------------------------------

@torch.inference_mode()
def _selectBitsTorch(weight: torch.Tensor, calibration: np.ndarray, threshold: float,
                     codesOnDevice: bool = False
                     ) -> tuple[int, float, np.ndarray | torch.Tensor | None, np.ndarray | None]:
    """Width selection on the model's GPU (core.py:112-195).

    The reference's rule: for b = 3..15, s = max|w_r| / qmax (1 for a zero
    row), q = clamp(round(w/s)), full = F.linear(x16, fp16(q*s)) and, for
    b <= 8, hw = fp16((x16.float() @ q^T) * s); the first b whose
    max(relL2(ref, hw), relL2(ref, full)) <= threshold wins, with
    ref = F.linear(x16, W16).  Here one fused HIP pass
    (``width_errors_torch``) yields the errors of all thirteen widths; the
    hw error is the integer-code output's at every b <= 12, because that is
    the arithmetic the HIP route runs there.  Only the chosen width is then
    quantized, and its codes and scales are returned so that packing never
    quantizes again.  ``codesOnDevice`` leaves the codes as an int16 tensor
    on the weight's device.
    """
    if weight.device.type != "cuda":
        raise RuntimeError("ElasticBit GPU analyzer requires CUDA weights")
    if weight.dtype != torch.float16:
        raise RuntimeError("ElasticBit GPU analyzer requires FP16 weights")
    if not np.isfinite(threshold) or float(threshold) < 0.0:
        raise ValueError("threshold must be a finite non-negative value")
    native = _requireNative()
    x16 = torch.as_tensor(np.ascontiguousarray(calibration, dtype=np.float32)).to(weight.device, torch.float16)
    w = weight.detach()
    full, hw = native.width_errors_torch(w, x16)
    errors = np.maximum(np.asarray(full, np.float64), np.asarray(hw, np.float64))
    passing = np.flatnonzero(errors <= float(threshold))
    if passing.size == 0:
        return 16, 0.0, None, None
    bits = int(passing[0]) + 3
    codes, scales = _quantizeRowsTorch(w, bits)
    if not codesOnDevice:
        codes = np.ascontiguousarray(codes.cpu().numpy(), dtype=np.int16)
    return bits, float(errors[bits - 3]), codes, scales


def _quantizeRowsTorch(weight: torch.Tensor, bits: int) -> tuple[torch.Tensor, np.ndarray]:
    """Codes (int16, on the weight's device) and row scales of one width, with
    the reference's torch expressions (core.py:142-155): the scale divides a
    tensor by a Python scalar, which torch's kernels compute as a product
    with fp32(1/qmax)."""
    w32 = weight.float()
    peak = w32.abs().amax(dim=1)
    qmax = float((1 << (bits - 1)) - 1)
    scale = torch.where(peak > 0.0, peak / qmax, torch.ones_like(peak))
    codes = torch.round(w32 / scale[:, None]).clamp(min=-qmax, max=qmax).to(torch.int16).contiguous()
    return codes, np.ascontiguousarray(scale.cpu().numpy(), dtype=np.float32)


# -- result records (field names are the public interface) -----------------------

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

    _SHOWN = ("device", "architecture", "weightWidths", "activateDType", "prefill", "decodePlanner",
              "decodeEngine", "decodeStatus", "decodeValidation")

    def __str__(self) -> str:
        if not self.available:
            return f"ElasticBitBackend(unavailable, error={self.error!r})"
        parts = [f"{name}={getattr(self, name)!r}" for name in self._SHOWN]
        parts[2] = f"weightWidths={self.weightWidths}"
        return "ElasticBitBackend(" + ", ".join(parts + [f"validated={self.validated}"]) + ")"


def _unavailable_backend(error: str | None, widths: Iterable[int] = (), dtype: str | None = None) -> BackendInfo:
    return BackendInfo(available=False, device=None, deviceIndex=None, architecture=None,
                       weightWidths=tuple(widths), activateDType=dtype, prefill=None, decodePlanner=None,
                       validated=False, error=error)


# -- the single-matrix handle ----------------------------------------------------

def _native_reader(name: str, cast: Callable[[Any], Any]) -> property:
    return property(lambda self: cast(getattr(self._native, name)), doc=f"The matrix's {name}.")


class RuntimeMatrix:
    """One ElasticBit matrix on the HIP runtime (core.py:264-424).

    Built only by :meth:`compress`, :meth:`load` and the analyzer-driven
    internal factories; no constructor takes a user-chosen bit width."""

    def __init__(self, native: Any) -> None:
        self._native = native
        self._resident: torch.Tensor | None = None

    # factories ------------------------------------------------------------

    @classmethod
    def _build(cls, factory: str, *args: Any) -> "RuntimeMatrix":
        native = _requireNative()
        return cls(getattr(native.RuntimeMatrix, factory)(*args))

    @classmethod
    def compress(cls, weights: Any, calibrationData: Any, threshold: float,
                 decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        _requireNative()
        policy = _checkPolicy(decodePolicy)
        return cls._build("compress", _matrix_f32(weights, "weights"), _matrix_f32(calibrationData, "calibrationData"),
                          float(threshold), policy)

    @classmethod
    def _compressSelected(cls, weights: Any, selectedBits: int, threshold: float, selectedError: float,
                          decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        _requireNative()
        policy = _checkPolicy(decodePolicy)
        return cls._build("_compressSelected", _matrix_f32(weights, "weights"), int(selectedBits), float(threshold),
                          float(selectedError), policy)

    @classmethod
    def _compressSelectedCodes(cls, codes: np.ndarray, scales: np.ndarray, selectedBits: int,
                               threshold: float, selectedError: float,
                               decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        """Pack an analyzer result as selected, without quantizing again."""
        _requireNative()
        policy = _checkPolicy(decodePolicy)
        q = np.ascontiguousarray(codes, dtype=np.int16)
        s = np.ascontiguousarray(scales, dtype=np.float32)
        if q.ndim != 2:
            raise ValueError("codes must be a 2D matrix")
        if s.shape != (q.shape[0],):
            raise ValueError("scales must contain one value per weight row")
        return cls._build("_compressSelectedCodes", q, s, int(selectedBits), float(threshold), float(selectedError),
                          policy)

    @classmethod
    def _compressSelectedCodesTorch(cls, codes: torch.Tensor, scales: np.ndarray, selectedBits: int,
                                    threshold: float, selectedError: float,
                                    decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        """``_compressSelectedCodes`` for int16 codes already on the HIP
        device: packed there, with no host copy of the codes."""
        _requireNative()
        policy = _checkPolicy(decodePolicy)
        return cls._build("_compressSelectedCodesTorch", codes, scales, int(selectedBits), float(threshold),
                          float(selectedError), policy)

    @classmethod
    def load(cls, path: str | Path, decodePolicy: str = "hardwareNative") -> "RuntimeMatrix":
        _requireNative()
        return cls._build("load", str(path), _checkPolicy(decodePolicy))

    # execution ------------------------------------------------------------

    def forward(self, x: Any) -> Any:
        """fp16 activations on the matrix's device stay there (any number of
        rows ``[..., cols]``); anything else makes the host round trip of one
        row, as the reference's numpy path does."""
        if torch.is_tensor(x) and x.is_cuda and x.dtype == torch.float16 and x.dim() >= 1 \
                and x.shape[-1] == self.cols:
            return self._native.forwardTorch(x.contiguous())
        host = x.detach().to("cpu", torch.float32).numpy() if torch.is_tensor(x) else x
        row = np.ascontiguousarray(np.asarray(host, dtype=np.float32).reshape(-1))
        out = np.asarray(self._native.forward(row))
        return torch.from_numpy(out).to(device=x.device, dtype=x.dtype) if torch.is_tensor(x) else out

    @staticmethod
    def forwardTorchMulti(matrices: Sequence["RuntimeMatrix"], x: torch.Tensor,
                          biases: Sequence[torch.Tensor | None] | None = None) -> list[torch.Tensor]:
        """``[m.forward(x) (+ bias) for m in matrices]`` for matrices that read
        the same fp16 activations, in one decode launch per run of equal
        widths (up to four matrices).  No single-call counterpart in the
        reference (its Stage-2F concatenates materialized weights,
        stage2f.py:382-420)."""
        return _requireNative().forward_torch_multi([m._native for m in matrices], x, biases)

    def benchmark(self, x: Any, iterations: int = 500) -> float:
        host = x.detach().to("cpu", torch.float32).numpy() if torch.is_tensor(x) else x
        row = np.ascontiguousarray(np.asarray(host, dtype=np.float32).reshape(-1))
        return float(self._native.benchmark(row, int(iterations)))

    def dequantize(self) -> np.ndarray:
        return np.asarray(self._native.dequantize(), dtype=np.float32)

    def _materializeTorch(self) -> torch.Tensor:
        return self._native._materializeTorch()

    def _residentFp16(self) -> torch.Tensor:
        """The decoded fp16 weights, materialized once and kept: what the
        reference's execution holds for b = 9..16 (runtime.cu:989-999)."""
        if self._resident is None:
            self._resident = self._materializeTorch()
        return self._resident

    def _releaseResident(self) -> None:
        self._resident = None

    def save(self, path: str | Path) -> None:
        self._native.save(str(path))

    def setDecodePolicy(self, decodePolicy: str) -> "RuntimeMatrix":
        self._native.setDecodePolicy(_checkPolicy(decodePolicy))
        return self

    @property
    def shape(self) -> tuple[int, int]:
        return tuple(int(v) for v in self._native.shape)


for _name, _cast in (("rows", int), ("cols", int), ("storageBits", int), ("executionWidth", int),
                     ("storageBytes", int), ("executionBytes", int), ("originalBytes", int),
                     ("executionPlanner", str), ("decodePolicy", str), ("activateDType", str),
                     ("memoryReduction", float), ("threshold", float), ("error", float)):
    setattr(RuntimeMatrix, _name, _native_reader(_name, _cast))
del _name, _cast


# -- the compressed Linear ---------------------------------------------------------

class _RouteOwner:
    """Carries the planner's frozen route for one phase of one layer."""

    __slots__ = ("_mlbricks_frozen_auto_routes", "_mlbricks_frozen_auto_details", "_mlbricks_auto_route_cache")

    def __init__(self) -> None:
        EXECUTION_PLANNER.clear_owner_routes(self)


class _ElasticLinear(nn.Module):
    """A Linear whose weight is an ElasticBit matrix (core.py:427-471); every
    call goes through the planner (``backend``: auto / native / pytorch)."""

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
        if self.backend != "auto":
            return self.backend
        frozen = []
        for phase in sorted(self._routeOwners):
            routes = EXECUTION_PLANNER.owner_routes(self._routeOwners[phase])
            if routes:
                frozen.append(f"{phase}={next(iter(routes.values()))}")
        return ",".join(frozen) or "auto"

    def _bias_as(self, x: torch.Tensor) -> torch.Tensor | None:
        bias = self.bias
        if bias is None or (bias.dtype == x.dtype and bias.device == x.device):
            return bias
        return bias.to(device=x.device, dtype=x.dtype)

    def _forwardNative(self, x: torch.Tensor) -> torch.Tensor:
        return self.matrix._native.forwardTorch(x, bias=self._bias_as(x))

    def _forwardPytorch(self, x: torch.Tensor) -> torch.Tensor:
        """The reference's prefill route (core.py:462-471): F.linear on the
        decoded fp16 weights, resident for b >= 9, materialized per call
        below."""
        weight = (self.matrix._residentFp16() if self.matrix.storageBits >= _RESIDENT_MIN_BITS
                  else self.matrix._materializeTorch())
        if weight.device != x.device:
            raise RuntimeError("ElasticBit Linear expects activations on the device that holds its matrix")
        return F.linear(x, weight.to(dtype=x.dtype), self._bias_as(x))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.inFeatures:
            raise ValueError(f"ElasticBit Linear expected last dimension {self.inFeatures}, got {x.shape[-1]}")
        hip_ok = (_nativeAvailable() and x.is_cuda and x.dtype == torch.float16
                  and self.matrix._native.deviceIndex == x.get_device())
        rows = x.numel() // self.inFeatures
        phase = "decode" if rows <= DECODE_PHASE_ROWS else "prefill"
        owner = self._routeOwners[phase]
        xc = x.contiguous() if hip_ok else x
        if hip_ok and self.backend == "auto" and not (torch.is_grad_enabled() and x.requires_grad):
            # A route the planner already froze for this owner is what
            # qualify_operator_once would return: skip its per-call set-up
            # (a decode loop pays it on every launch).
            if EXECUTION_PLANNER.frozen_route(owner, "elastic_linear") == "native":
                return self._forwardNative(xc)
        route = EXECUTION_PLANNER.qualify_operator_once(
            owner, "elastic_linear", xc,
            {"native": lambda: self._forwardNative(xc), "pytorch": lambda: self._forwardPytorch(x)},
            requested_backend=self.backend, native_available=hip_ok,
            training=bool(torch.is_grad_enabled() and x.requires_grad),
            extra=(self.outFeatures, self.inFeatures, self.matrix.storageBits, phase),
            default_auto="pytorch",
        )
        if route == "native":
            self._drop_unused_resident()
            return self._forwardNative(xc)
        return self._forwardPytorch(x)

    def _drop_unused_resident(self) -> None:
        """A resident fp16 copy made for the qualification race stays only
        while some phase of this layer runs the PyTorch route."""
        if self.matrix._resident is None:
            return
        for owner in self._routeOwners.values():
            if "pytorch" in EXECUTION_PLANNER.owner_routes(owner).values():
                return
        if self.backend != "pytorch":
            self.matrix._releaseResident()


# -- model-level controller ----------------------------------------------------------

class _ModelElasticBit:
    """``model.elasticbit`` (core.py:474-547): what was compressed, the decode
    policy, and a summary table."""

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
        found = []
        for name in self.compressedNames:
            try:
                layer = self._model.get_submodule(name)
            except AttributeError:
                continue
            if isinstance(layer, _ElasticLinear):
                found.append((name, layer))
        return found

    def _matrices(self) -> list[RuntimeMatrix]:
        """Each distinct matrix once (shared weights share one)."""
        unique: dict[int, RuntimeMatrix] = {}
        for _, layer in self._layers():
            unique.setdefault(id(layer.matrix), layer.matrix)
        return list(unique.values())

    def setDecodePolicy(self, decodePolicy: str) -> "_ModelElasticBit":
        policy = _checkPolicy(decodePolicy)
        for matrix in self._matrices():
            matrix.setDecodePolicy(policy)
        self.decodePolicy = policy
        return self

    def summary(self) -> str:
        info = ElasticBit.backend()
        header = [
            ("Threshold", self.threshold), ("Decode Policy", self.decodePolicy),
            ("Backend", info.architecture or "unavailable"), ("Prefill", info.prefill or "unknown"),
            ("Decode Engine", info.decodeEngine or "unknown"), ("Decode Status", info.decodeStatus or "unknown"),
            ("Decode Planner", info.decodePlanner or "unknown"),
            ("Decode Validate", info.decodeValidation or "unknown"),
            ("Activate DType", info.activateDType or "unknown"),
        ]
        lines = ["ElasticBit Summary", "-" * 60]
        lines += [f"{label:<16s}: {value}" for label, value in header]
        lines += ["", f"{'Layer':36s} {'Stored':>8s} {'Execute':>10s} {'Planner':>14s} {'Error':>10s}"]
        for name, layer in self._layers():
            m = layer.matrix
            lines.append(f"{name[:36]:36s} {f'{m.storageBits}-bit':>8s} {f'W{m.executionWidth}A16':>10s} "
                         f"{m.executionPlanner:>14s} {m.error:10.6f}")
        if self.skippedNames:
            lines += ["", "Uncompressed (no safe calibration path):"] + [f"  {n}" for n in self.skippedNames]
        text = "\n".join(lines)
        print(text)
        return text


def _semanticOutputWeightIds(model: nn.Module) -> set[int]:
    """The token-output head's weight, found through the model's own
    ``get_output_embeddings()`` rather than by module names (core.py:550-568)."""
    getter = getattr(model, "get_output_embeddings", None)
    try:
        head = getter() if callable(getter) else None
    except Exception:
        head = None
    return {id(head.weight)} if isinstance(head, nn.Linear) else set()


# -- compression pipeline ---------------------------------------------------------------

class _CalibrationTap:
    """Forward pre-hooks that keep the first CALIBRATION_ROWS input rows each
    hooked Linear sees, as float32 host arrays."""

    def __init__(self, linears: Mapping[str, nn.Linear]) -> None:
        self._linears = dict(linears)
        self._rows: dict[str, list[np.ndarray]] = {name: [] for name in self._linears}
        self._kept: dict[str, int] = {name: 0 for name in self._linears}
        self._handles: list[Any] = []

    def _hook(self, name: str):
        def capture(_module: nn.Module, inputs: tuple[Any, ...]) -> None:
            room = CALIBRATION_ROWS - self._kept[name]
            if room <= 0 or not inputs or not torch.is_tensor(inputs[0]):
                return
            flat = inputs[0].detach().reshape(-1, inputs[0].shape[-1])[:room]
            self._rows[name].append(flat.to("cpu", torch.float32).numpy().copy())
            self._kept[name] += flat.shape[0]
        return capture

    def __enter__(self) -> "_CalibrationTap":
        self._handles = [linear.register_forward_pre_hook(self._hook(name))
                         for name, linear in self._linears.items()]
        return self

    def __exit__(self, *exc: Any) -> None:
        for handle in self._handles:
            handle.remove()
        self._handles = []

    def rows_for(self, names: Sequence[str]) -> np.ndarray | None:
        """The captured rows of every use of one weight, in name order."""
        parts = [block for name in names for block in self._rows.get(name, [])]
        return np.ascontiguousarray(np.concatenate(parts), dtype=np.float32) if parts else None

    def forget(self, names: Iterable[str]) -> None:
        for name in names:
            self._rows.pop(name, None)


@dataclass
class _WeightGroup:
    """Every Linear name that uses one weight tensor (in module order)."""
    weight_id: int
    names: list[str]


def _weight_groups(model: nn.Module) -> list[_WeightGroup]:
    groups: dict[int, _WeightGroup] = {}
    for name, module in model.named_modules():
        if isinstance(module, nn.Linear):
            groups.setdefault(id(module.weight), _WeightGroup(id(module.weight), [])).names.append(name)
    return list(groups.values())


def _progress_enabled() -> bool:
    return os.environ.get("MLBRICKS_ELASTICBIT_PROGRESS", "").strip().lower() in {"1", "true", "yes", "on"}


def _free_vram(device: torch.device) -> str:
    free, total = torch.cuda.mem_get_info(device)
    return f"free={free / 2**30:.2f}/{total / 2**30:.2f} GiB"


def _matrix_for(linear: nn.Linear, calibration: np.ndarray, threshold: float, policy: str,
                report: Callable[[str], None]) -> RuntimeMatrix:
    """Select the width of one Linear's weight and build its matrix on the
    weight's device: packed from the analyzer's codes for b <= 15, the fp16
    values themselves for the fallback."""
    bits, err, codes, scales = _selectBitsTorch(linear.weight, calibration, threshold, codesOnDevice=True)
    torch.cuda.empty_cache()      # hand the analysis blocks back before the runtime allocates
    report(f"selected {bits}-bit error={err:.6g}")
    with torch.cuda.device(linear.weight.device):
        if bits <= 15:
            return RuntimeMatrix._compressSelectedCodesTorch(codes, scales, bits, threshold, err, decodePolicy=policy)
        fp16 = _matrix_f32(linear.weight, "weights")
        return RuntimeMatrix._compressSelected(fp16, bits, threshold, err, decodePolicy=policy)


def _install(model: nn.Module, names: Sequence[str], matrix: RuntimeMatrix, device: torch.device) -> None:
    """Replace every Linear of one weight group by an _ElasticLinear sharing
    ``matrix`` (so the group's fp16 weight can be freed at once)."""
    for name in names:
        current = model.get_submodule(name)
        if not isinstance(current, nn.Linear):
            raise RuntimeError(f"ElasticBit expected Linear module at {name}")
        layer = _ElasticLinear(matrix, current.in_features, current.out_features, current.bias)
        _replaceNamedModule(model, name, layer.to(device=device))


# -- the zip artifact ---------------------------------------------------------------------

class _Artifact:
    """``manifest.json``, ``matrices/matrix_%05d.mlb`` (MLB4) and ``state.pt``
    in one DEFLATE zip (core.py:900-1017)."""

    MANIFEST = "manifest.json"
    STATE = "state.pt"
    MATRICES = "matrices"

    @classmethod
    def write(cls, model: nn.Module, controller: _ModelElasticBit, path: Path) -> None:
        files: dict[int, str] = {}
        layers = []
        with zipfile.ZipFile(path, "w", compression=zipfile.ZIP_DEFLATED) as archive, \
                tempfile.TemporaryDirectory(prefix="elasticbit-save-") as scratch:
            for name in controller.compressedNames:
                try:
                    layer = model.get_submodule(name)
                except AttributeError:
                    layer = None
                if not isinstance(layer, _ElasticLinear):
                    raise RuntimeError(f"ElasticBit layer disappeared before save: {name}")
                member = files.get(id(layer.matrix))
                if member is None:
                    member = files[id(layer.matrix)] = f"matrix_{len(files):05d}.mlb"
                    staged = Path(scratch) / member
                    layer.matrix.save(staged)
                    archive.write(staged, f"{cls.MATRICES}/{member}")
                layers.append({"name": name, "matrix": member, "inFeatures": layer.inFeatures,
                               "outFeatures": layer.outFeatures, "hasBias": layer.bias is not None})
            manifest = {"format": ARTIFACT_FORMAT[0], "version": ARTIFACT_FORMAT[1],
                        "threshold": controller.threshold, "decodePolicy": controller.decodePolicy,
                        "compressedNames": list(controller.compressedNames),
                        "skippedNames": list(controller.skippedNames),
                        "optimizationProfiles": controller.optimizationProfiles, "layers": layers}
            archive.writestr(cls.MANIFEST, json.dumps(manifest, indent=2))
            state = io.BytesIO()
            torch.save(model.state_dict(), state)
            archive.writestr(cls.STATE, state.getvalue())

    @classmethod
    def read_manifest(cls, archive: zipfile.ZipFile) -> dict[str, Any]:
        manifest = json.loads(archive.read(cls.MANIFEST).decode("utf-8"))
        if (manifest.get("format"), manifest.get("version")) != ARTIFACT_FORMAT:
            raise ValueError("Unsupported ElasticBit model artifact")
        return manifest

    @classmethod
    def load_matrix(cls, archive: zipfile.ZipFile, member: str, policy: str, device: torch.device) -> RuntimeMatrix:
        with tempfile.TemporaryDirectory(prefix="elasticbit-load-") as scratch:
            staged = Path(scratch) / "matrix.mlb"
            staged.write_bytes(archive.read(f"{cls.MATRICES}/{member}"))
            with torch.cuda.device(device):
                return RuntimeMatrix.load(staged, decodePolicy=policy)

    @classmethod
    def load_state(cls, archive: zipfile.ZipFile, device: torch.device) -> dict[str, Any]:
        return torch.load(io.BytesIO(archive.read(cls.STATE)), map_location=device, weights_only=True)


# -- public namespace -------------------------------------------------------------------------

class ElasticBit:
    """The public ElasticBit namespace (core.py:571-1017)."""

    RuntimeMatrix = RuntimeMatrix

    @staticmethod
    def analyze(weights: Any, calibrationData: Any, threshold: float) -> BitAnalysis:
        """The host analyzer's errors for every width (runtime.cu:280-483)."""
        raw = _requireNative().analyze(_matrix_f32(weights, "weights"),
                                       _matrix_f32(calibrationData, "calibrationData"), float(threshold))
        types = {f.name: f.type for f in fields(BitCandidate)}
        casts = {"int": int, "float": float, "bool": bool}
        candidates = tuple(BitCandidate(**{key: casts[types[key]](item[key]) for key in types})
                           for item in raw["candidates"])
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
            return _unavailable_backend(None if err is None else str(err))
        raw = _requireNative().backendInfo()
        if not raw["available"]:
            return _unavailable_backend("no HIP device is visible to the ElasticBit runtime",
                                        raw["weightWidths"], raw["activateDType"])
        text = ("device", "architecture", "activateDType", "prefill", "decodePlanner", "decodeEngine",
                "decodeStatus", "decodeValidation")
        return BackendInfo(available=True, deviceIndex=int(raw["deviceIndex"]),
                           weightWidths=tuple(int(v) for v in raw["weightWidths"]),
                           validated=bool(raw["validated"]), **{key: str(raw[key]) for key in text})

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
        """Compress every fp16 ``nn.Linear`` of ``model`` except embeddings and
        the output head (core.py:695-898).

        The calibration batches run once through the model; each Linear keeps
        its first 32 input rows.  A weight shared by several Linears is
        analysed once on all their rows and becomes one shared matrix.  Each
        weight group is replaced as soon as its matrix exists, so peak device
        memory stays near the compressed model's."""
        if not isinstance(model, nn.Module):
            raise TypeError("ElasticBit.compress() expects a torch.nn.Module")
        _requireNative()
        policy = _checkPolicy(decodePolicy)
        batches = _batch_list(calibrationData)
        device = _device_of(model)
        if device.type != "cuda":
            raise RuntimeError("ElasticBit model compression currently requires a CUDA model")
        linears = {name: m for name, m in model.named_modules() if isinstance(m, nn.Linear)}
        if any(m.weight.dtype != torch.float16 for m in linears.values()):
            raise RuntimeError("ElasticBit.compress() currently requires FP16 Linear weights. "
                               "Convert the model to float16 before compression.")
        head_ids = _semanticOutputWeightIds(model) if preserveOutputHead else set()
        protected = head_ids | {id(m.weight) for m in model.modules() if isinstance(m, nn.Embedding)}

        tap = _CalibrationTap({name: m for name, m in linears.items() if id(m.weight) not in protected})
        del linears
        model.eval()
        with tap, torch.inference_mode():
            for batch in batches:
                _feed(model, _on_device(batch, device))

        groups = _weight_groups(model)
        skipped = [name for g in groups if g.weight_id in head_ids for name in g.names]
        work = [g for g in groups if g.weight_id not in protected]
        compressed: list[str] = []
        chatty = _progress_enabled()
        for index, group in enumerate(work, start=1):
            def report(message: str, index: int = index) -> None:
                if chatty:
                    print(f"[ElasticBit] {index}/{len(work)} {message}", flush=True)

            linear = model.get_submodule(group.names[0])
            if not isinstance(linear, nn.Linear):
                raise RuntimeError(f"ElasticBit expected Linear module at {group.names[0]}")
            calibration = tap.rows_for(group.names)
            if calibration is None:
                skipped.extend(group.names)
                continue
            report(f"analyzing {group.names[0]} shape={tuple(linear.weight.shape)} rows={calibration.shape[0]} "
                   f"{_free_vram(device)}" if chatty else "")
            matrix = _matrix_for(linear, calibration, float(threshold), policy, report)
            del linear, calibration
            _install(model, group.names, matrix, device)
            compressed.extend(group.names)
            tap.forget(group.names)
            del matrix
            gc.collect()
            torch.cuda.empty_cache()
            if chatty:
                report(f"packed/replaced {_free_vram(device)}")

        model.elasticbit = _ModelElasticBit(model, threshold=float(threshold), decodePolicy=policy,
                                            compressedNames=compressed, skippedNames=skipped)
        return model

    @staticmethod
    def save(model: nn.Module, path: str | Path) -> Path:
        """Write the compressed model as one zip artifact (core.py:900-955)."""
        controller = getattr(model, "elasticbit", None)
        if not isinstance(controller, _ModelElasticBit):
            raise ValueError("ElasticBit.save() expects a model produced by ElasticBit.compress()")
        destination = Path(path)
        destination.parent.mkdir(parents=True, exist_ok=True)
        _Artifact.write(model, controller, destination)
        return destination

    @staticmethod
    def load(model: nn.Module, path: str | Path, decodePolicy: str = "hardwareNative") -> nn.Module:
        """Rebuild the compressed layers of an artifact into an instance of the
        original architecture, then load its state (core.py:957-1017)."""
        if not isinstance(model, nn.Module):
            raise TypeError("ElasticBit.load() requires the model architecture as its first argument")
        _requireNative()
        source = Path(path)
        if not source.exists():
            raise FileNotFoundError(source)
        with zipfile.ZipFile(source, "r") as archive:
            manifest = _Artifact.read_manifest(archive)
            policy = _checkPolicy(decodePolicy)
            matrices: dict[str, RuntimeMatrix] = {}
            compressed: list[str] = []
            for entry in manifest["layers"]:
                name = str(entry["name"])
                try:
                    target = model.get_submodule(name)
                except AttributeError:
                    target = None
                if not isinstance(target, nn.Linear):
                    raise ValueError(f"Model architecture does not contain expected Linear layer: {name}")
                device = target.weight.device
                if device.type != "cuda":
                    raise RuntimeError("ElasticBit.load() requires the target model on CUDA")
                member = str(entry["matrix"])
                if member not in matrices:
                    matrices[member] = _Artifact.load_matrix(archive, member, policy, device)
                layer = _ElasticLinear(matrices[member], int(entry["inFeatures"]), int(entry["outFeatures"]),
                                       target.bias if bool(entry["hasBias"]) else None)
                _replaceNamedModule(model, name, layer.to(device=device))
                compressed.append(name)
            model.load_state_dict(_Artifact.load_state(archive, _device_of(model)), strict=True)
        model.elasticbit = _ModelElasticBit(model, threshold=float(manifest["threshold"]), decodePolicy=policy,
                                            compressedNames=compressed,
                                            skippedNames=tuple(manifest.get("skippedNames", ())),
                                            optimizationProfiles=manifest.get("optimizationProfiles", {}))
        return model


__all__ = ["ElasticBit", "RuntimeMatrix", "BitAnalysis", "BitCandidate", "BackendInfo"]
