"""Route planner for backend-aware operators: for each call, does the native
(HIP) implementation or the PyTorch one serve it?

Contract (the interface of ``mlbricks/planner.py`` that callers and the
reference's planner tests rely on):

* an explicit ``native`` / ``pytorch`` request is honoured as asked (``native``
  raises ``RuntimeError`` when it cannot run);
* ``auto`` resolves per *owner* (one layer, one phase) and then stays frozen
  on that owner until ``clear_owner_routes``.  ``qualify_operator_once``
  resolves it by measurement: PyTorch is the correctness reference, a native
  result that is not close to it never wins, and among correct routes the
  faster one wins unless it beats ``AUTO_OPERATOR_DEFAULTS`` by less than
  ``switch_margin``;
* the owner attributes ``_mlbricks_frozen_auto_routes`` and
  ``_mlbricks_frozen_auto_details`` and the reason strings
  (``correctness-gate:...``, ``correctness-pass;benchmark-once:...``,
  ``heuristic:...``) are what the reference's tests read.

Only the ``elastic_linear`` operator is registered here; the reference
planner's resource model for its other components is not on this path.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Any, Callable, Final, Iterator, Mapping

import torch

from .runtime import normalize_backend

ROUTES: Final = ("native", "pytorch")

# Initial auto route per operator; qualification may override it
# (planner.py:53 starts ElasticBit on PyTorch).
AUTO_OPERATOR_DEFAULTS: Final[dict[str, str]] = {
    "elastic_linear": "pytorch",
}

_OWNER_ROUTES = "_mlbricks_frozen_auto_routes"
_OWNER_DETAILS = "_mlbricks_frozen_auto_details"
_OWNER_HOT = "_mlbricks_auto_route_cache"


def ceil_power_of_two(value: int) -> int:
    """Smallest power of two >= value (>= 1)."""
    n = max(1, int(value))
    return 1 << (n - 1).bit_length()


def sequence_bucket(length: int) -> int:
    """Sequence lengths share a decision within a power-of-two bucket of at
    least 64 (planner.py:70-72)."""
    return max(64, ceil_power_of_two(length))


@dataclass(frozen=True)
class HardwareProfile:
    device_index: int
    compute_capability: tuple[int, int]
    multiprocessors: int
    warp_size: int
    max_threads_per_sm: int

    @property
    def resident_threads(self) -> int:
        return self.multiprocessors * self.max_threads_per_sm


@dataclass
class RouteDecision:
    """What the planner knows about one operator key."""
    route: str
    reason: str
    timings_ms: dict[str, float] | None = None


# -- output comparison (the correctness gate) ----------------------------------

def _leaves(obj: object, path: str) -> Iterator[tuple[str, str, object]]:
    """(path, kind, value) for every leaf of a nested output, in a canonical
    order: mappings by sorted key, sequences by index.  Containers yield a
    'shape' leaf of their own so that structures compare too."""
    if torch.is_tensor(obj):
        yield path, "tensor", obj
    elif isinstance(obj, Mapping):
        keys = sorted(obj.keys(), key=repr)
        yield path, "mapping", tuple(repr(k) for k in keys)
        for k in keys:
            yield from _leaves(obj[k], f"{path}[{k!r}]")
    elif isinstance(obj, (tuple, list)):
        yield path, type(obj).__name__, len(obj)
        for i, item in enumerate(obj):
            yield from _leaves(item, f"{path}[{i}]")
    else:
        yield path, "value", obj


@dataclass
class ParityReport:
    rtol: float
    atol: float
    checked: bool = True
    allclose: bool = True
    tensor_leaves: int = 0
    max_abs: float = 0.0
    max_relative_l2: float = 0.0
    mismatch: str | None = None

    def fail(self, where: str, why: str) -> None:
        self.allclose = False
        if self.mismatch is None:
            self.mismatch = f"{where}: {why}"

    def as_dict(self) -> dict[str, object]:
        return {"checked": self.checked, "allclose": self.allclose, "rtol": self.rtol, "atol": self.atol,
                "tensor_leaves": self.tensor_leaves, "max_abs": self.max_abs,
                "max_relative_l2": self.max_relative_l2, "mismatch": self.mismatch}


def _same_value(a: object, b: object) -> bool:
    try:
        return bool(a == b)
    except Exception:
        return repr(a) == repr(b)


def compare_outputs(reference: object, candidate: object, *, rtol: float, atol: float) -> ParityReport:
    """Leaf-by-leaf comparison of two outputs: same structure, tensors of the
    same shape that are ``allclose`` (floating point; statistics in float32
    or complex64) or equal (integer / bool), other leaves equal."""
    report = ParityReport(rtol=float(rtol), atol=float(atol))
    ref_leaves = list(_leaves(reference, "output"))
    cand_leaves = list(_leaves(candidate, "output"))
    cand_at = {path: (kind, value) for path, kind, value in cand_leaves}
    for path, kind, ref in ref_leaves:
        if path not in cand_at:
            report.fail(path, "missing from the native output")
            continue
        ckind, cand = cand_at[path]
        if kind != ckind:
            report.fail(path, f"{kind} in the PyTorch output, {ckind} in the native output")
            continue
        if kind != "tensor":
            if not _same_value(ref, cand):
                report.fail(path, f"{ref!r} != {cand!r}")
            continue
        if tuple(ref.shape) != tuple(cand.shape):
            report.fail(path, f"shape {tuple(ref.shape)} != {tuple(cand.shape)}")
            continue
        report.tensor_leaves += 1
        r = ref.detach()
        c = cand.detach().to(r.device)
        if r.is_floating_point() or r.is_complex():
            wide = torch.complex64 if r.is_complex() else torch.float32
            r, c = r.to(wide), c.to(wide)
            if r.numel():
                diff = c - r
                report.max_abs = max(report.max_abs, float(diff.abs().max()))
                rel = float(torch.linalg.vector_norm(diff.reshape(-1))
                            / (torch.linalg.vector_norm(r.reshape(-1)) + 1e-12))
                report.max_relative_l2 = max(report.max_relative_l2, rel)
            close = bool(torch.allclose(c, r, rtol=rtol, atol=atol))
        else:
            close = bool(torch.equal(c, r))
        if not close:
            report.fail(path, "tensor values differ from PyTorch reference")
    ref_paths = {path for path, _, _ in ref_leaves}
    extra = [path for path, _, _ in cand_leaves if path not in ref_paths]
    if extra:
        report.fail(extra[0], "not in the PyTorch output")
    return report


def _default_tolerances(tensor: torch.Tensor) -> tuple[float, float]:
    """2e-2 for 16-bit floating inputs, 1e-4 / 1e-5 otherwise (planner.py:453-465)."""
    if tensor.dtype in (torch.float16, torch.bfloat16):
        return 2.0e-2, 2.0e-2
    return 1.0e-4, 1.0e-5


# -- owner state ---------------------------------------------------------------

def _owner_dict(owner: object, name: str) -> dict:
    table = getattr(owner, name, None)
    if not isinstance(table, dict):
        table = {}
        try:
            setattr(owner, name, table)
        except Exception:
            pass
    return table


class MLBricksExecutionPlanner:
    """Route decisions for backend-aware operators (planner.py:88-1053)."""

    def __init__(self) -> None:
        self._decisions: dict[tuple[object, ...], RouteDecision] = {}
        self._revision = 0

    # -- the decision book ---------------------------------------------------

    def _record(self, key: tuple[object, ...], route: str, reason: str,
                timings: Mapping[str, float] | None = None) -> str:
        old = self._decisions.get(key)
        if old is None or old.route != route:
            self._revision += 1
        self._decisions[key] = RouteDecision(route, reason, None if timings is None else dict(timings))
        return route

    @property
    def operator_cache(self) -> dict[tuple[object, ...], str]:
        return {key: d.route for key, d in self._decisions.items()}

    @property
    def operator_reasons(self) -> dict[tuple[object, ...], str]:
        return {key: d.reason for key, d in self._decisions.items()}

    @property
    def operator_benchmarks(self) -> dict[tuple[object, ...], dict[str, float]]:
        return {key: d.timings_ms for key, d in self._decisions.items() if d.timings_ms is not None}

    @property
    def operator_revision(self) -> int:
        return self._revision

    def operator_decisions(self) -> list[dict[str, object]]:
        return [{"key": key, "route": d.route, "reason": d.reason, "benchmarks_ms": d.timings_ms}
                for key, d in self._decisions.items()]

    def clear(self) -> None:
        self._decisions.clear()
        self._revision += 1

    # -- keys ------------------------------------------------------------------

    def hardware_profile(self, device: torch.device | str) -> HardwareProfile:
        if not torch.cuda.is_available():
            raise RuntimeError("GPU hardware profile requested without a HIP device")
        dev = torch.device(device)
        index = torch.cuda.current_device() if dev.index is None else int(dev.index)
        props = torch.cuda.get_device_properties(index)
        return HardwareProfile(index, (int(props.major), int(props.minor)), int(props.multi_processor_count),
                               int(getattr(props, "warp_size", 64)),
                               int(getattr(props, "max_threads_per_multi_processor", 2048)))

    def operator_key(self, op: str, tensor: torch.Tensor, *, training: bool,
                     extra: tuple[object, ...] = ()) -> tuple[object, ...]:
        """("op", name, device..., dtype, shape, training, extra...): exact
        batch and feature sizes, the sequence size (second to last of a 3-D
        or larger input) bucketed (planner.py:230-256)."""
        shape = [int(v) for v in tensor.shape]
        if len(shape) >= 3:
            shape[-2] = sequence_bucket(shape[-2])
        if tensor.is_cuda and torch.cuda.is_available():
            hw = self.hardware_profile(tensor.device)
            device: tuple[object, ...] = ("cuda", hw.device_index, hw.compute_capability, hw.multiprocessors,
                                          hw.warp_size)
        else:
            device = (tensor.device.type, tensor.device.index)
        return ("op", str(op), *device, str(tensor.dtype), tuple(shape), bool(training), *tuple(extra))

    @staticmethod
    def _default_route(op: str, override: str | None) -> str:
        route = str(override or AUTO_OPERATOR_DEFAULTS.get(str(op), "pytorch")).lower()
        return route if route in ROUTES else "pytorch"

    # -- per-owner frozen routes ------------------------------------------------

    @staticmethod
    def owner_routes(owner: object) -> dict[tuple[object, ...], str]:
        table = getattr(owner, _OWNER_ROUTES, None)
        if not isinstance(table, dict):
            return {}
        return {key: route for key, route in table.items() if route in ROUTES}

    @staticmethod
    def frozen_route(owner: object, op: str, training: bool = False) -> str | None:
        """The route frozen for ``op`` on ``owner``, or None: the answer
        qualify_operator_once gives an auto owner once it has qualified,
        without building its arguments."""
        table = getattr(owner, _OWNER_ROUTES, None)
        route = table.get((str(op), bool(training))) if isinstance(table, dict) else None
        return route if route in ROUTES else None

    @staticmethod
    def clear_owner_routes(owner: object) -> None:
        """Forget an owner's frozen auto decisions (planner.py:420-433)."""
        for name, empty in ((_OWNER_ROUTES, {}), (_OWNER_DETAILS, {}), (_OWNER_HOT, None)):
            try:
                setattr(owner, name, empty)
            except Exception:
                pass

    # -- resolution ---------------------------------------------------------------

    def select_operator(self, op: str, tensor: torch.Tensor, *, requested_backend: str = "auto",
                        native_available: bool, native_supports_training: bool = False,
                        training: bool | None = None, extra: tuple[object, ...] = (),
                        default_auto: str | None = None) -> str:
        """One call's route (planner.py:778-835): explicit requests as asked;
        ``auto`` from the decision book, else PyTorch when the native route
        cannot serve the call, else the operator's default."""
        policy = normalize_backend(requested_backend, warn_legacy=True)
        is_training = torch.is_grad_enabled() if training is None else bool(training)
        inference_only = is_training and not native_supports_training
        if policy == "pytorch":
            return "pytorch"
        if policy == "native":
            if not native_available:
                raise RuntimeError(f"backend='native' requested but native route for {op!r} is unavailable")
            if inference_only:
                raise RuntimeError(f"backend='native' requested for {op!r}, but its native route is "
                                   "inference-only for this call")
            return "native"
        key = self.operator_key(op, tensor, training=is_training, extra=extra)
        if inference_only:
            return self._record(key, "pytorch", "training-safe:pytorch")
        if not native_available:
            return self._record(key, "pytorch", "native-unavailable:pytorch")
        known = self._decisions.get(key)
        if known is not None and known.route in ROUTES:
            return known.route
        route = self._default_route(op, default_auto)
        return self._record(key, route, f"heuristic:{route}")

    def select_operator_once(self, owner: object, op: str, tensor: torch.Tensor, *,
                             requested_backend: str = "auto", native_available: bool,
                             native_supports_training: bool = False, training: bool | None = None,
                             extra: tuple[object, ...] = (), default_auto: str | None = None) -> str:
        """``auto`` resolved once per owner and then frozen there
        (planner.py:361-417); explicit requests pass straight through."""
        policy = normalize_backend(requested_backend, warn_legacy=True)
        is_training = torch.is_grad_enabled() if training is None else bool(training)
        ask = dict(native_available=native_available, native_supports_training=native_supports_training,
                   training=is_training, extra=extra, default_auto=default_auto)
        if policy != "auto":
            return self.select_operator(op, tensor, requested_backend=policy, **ask)
        frozen = _owner_dict(owner, _OWNER_ROUTES)
        slot = (str(op), is_training)
        if frozen.get(slot) in ROUTES:
            return frozen[slot]
        frozen[slot] = self.select_operator(op, tensor, requested_backend="auto", **ask)
        return frozen[slot]

    def select_operator_cached(self, owner: object, op: str, tensor: torch.Tensor, *,
                               requested_backend: str = "auto", native_available: bool,
                               native_supports_training: bool = False, training: bool | None = None,
                               extra: tuple[object, ...] = (), default_auto: str | None = None) -> str:
        """``select_operator`` behind a one-entry cache on the owner, keyed by
        everything the answer depends on and invalidated whenever any
        decision changes (planner.py:293-358)."""
        is_training = torch.is_grad_enabled() if training is None else bool(training)
        policy = normalize_backend(requested_backend, warn_legacy=True)
        fingerprint = (str(op), policy, bool(native_available), bool(native_supports_training), is_training,
                       tuple(tensor.shape), str(tensor.dtype), str(tensor.device), tuple(extra), default_auto)
        hot = getattr(owner, _OWNER_HOT, None)
        if isinstance(hot, tuple) and len(hot) == 3 and hot[0] == fingerprint and hot[1] == self._revision:
            return hot[2]
        route = self.select_operator(op, tensor, requested_backend=policy, native_available=native_available,
                                     native_supports_training=native_supports_training, training=is_training,
                                     extra=extra, default_auto=default_auto)
        try:
            setattr(owner, _OWNER_HOT, (fingerprint, self._revision, route))
        except Exception:
            pass
        return route

    # -- qualification ------------------------------------------------------------

    @staticmethod
    def _time_ms(fn: Callable[[], object], tensor: torch.Tensor, warmup: int, trials: int) -> float:
        """Median milliseconds of ``trials`` calls after ``warmup`` calls:
        device events on a GPU tensor, the host clock otherwise."""
        for _ in range(warmup):
            fn()
        samples = []
        if tensor.is_cuda:
            torch.cuda.synchronize(tensor.device)
            for _ in range(trials):
                begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                begin.record()
                fn()
                end.record()
                end.synchronize()
                samples.append(float(begin.elapsed_time(end)))
        else:
            for _ in range(trials):
                t0 = time.perf_counter()
                fn()
                samples.append((time.perf_counter() - t0) * 1e3)
        return sorted(samples)[len(samples) // 2]

    def qualify_operator_once(self, owner: object, op: str, tensor: torch.Tensor,
                              candidates: Mapping[str, Callable[[], object]], *,
                              requested_backend: str = "auto", native_available: bool,
                              native_supports_training: bool = False, training: bool | None = None,
                              extra: tuple[object, ...] = (), default_auto: str | None = None,
                              warmup: int = 2, trials: int = 5, switch_margin: float = 0.05,
                              verify_parity: bool = True, parity_rtol: float | None = None,
                              parity_atol: float | None = None) -> str:
        """Qualify an owner's ``auto`` route once by correctness and speed,
        then freeze it on the owner (planner.py:570-776)."""
        policy = normalize_backend(requested_backend, warn_legacy=True)
        is_training = torch.is_grad_enabled() if training is None else bool(training)
        ask = dict(native_available=native_available, native_supports_training=native_supports_training,
                   training=is_training, extra=extra, default_auto=default_auto)
        if policy != "auto":
            return self.select_operator(op, tensor, requested_backend=policy, **ask)
        if is_training and not native_supports_training:
            return "pytorch"
        frozen = _owner_dict(owner, _OWNER_ROUTES)
        slot = (str(op), is_training)
        usable = {str(name): fn for name, fn in candidates.items() if str(name) in ROUTES and callable(fn)}
        if not native_available or not usable:
            return self.select_operator_once(owner, op, tensor, requested_backend="auto", **ask)
        if frozen.get(slot) in ROUTES:
            return frozen[slot]
        run = _Qualification(self, tensor, usable, parity_rtol, parity_atol)
        key = self.operator_key(op, tensor, training=is_training, extra=extra)
        if verify_parity and len(usable) == 2:
            rejected = run.parity_gate()
            if rejected is not None:
                return run.freeze(owner, key, slot, "pytorch", rejected)
        run.race(max(0, int(warmup)), max(1, int(trials)))
        if not run.timings:
            return self.select_operator_once(owner, op, tensor, requested_backend="auto", **ask)
        route = run.winner(self._default_route(op, default_auto), max(0.0, float(switch_margin)))
        return run.freeze(owner, key, slot, route, run.race_reason())

    # -- explicit calibration ------------------------------------------------------

    def set_operator_route(self, op: str, tensor: torch.Tensor, route: str, *, training: bool = False,
                           extra: tuple[object, ...] = (), reason: str = "manual") -> str:
        value = str(route).strip().lower()
        if value not in ROUTES:
            raise ValueError("route must be 'native' or 'pytorch'")
        return self._record(self.operator_key(op, tensor, training=training, extra=extra), value, str(reason))

    def record_operator_benchmark(self, op: str, tensor: torch.Tensor, timings_ms: Mapping[str, float], *,
                                  training: bool = False, extra: tuple[object, ...] = ()) -> str:
        """Store measured timings and make the fastest route the decision."""
        valid = {}
        for name, ms in timings_ms.items():
            if str(name) in ROUTES and float(ms) > 0.0:
                valid[str(name)] = float(ms)
        if not valid:
            raise ValueError("timings_ms must contain positive native/pytorch timings")
        winner = min(valid, key=valid.__getitem__)
        reason = "benchmark:" + ",".join(f"{name}={valid[name]:.6f}ms" for name in sorted(valid))
        return self._record(self.operator_key(op, tensor, training=training, extra=extra), winner, reason, valid)

    def benchmark_candidates(self, op: str, tensor: torch.Tensor,
                             candidates: Mapping[str, Callable[[], object]], *, warmup: int = 5,
                             trials: int = 20, training: bool = False,
                             extra: tuple[object, ...] = ()) -> tuple[str, dict[str, float]]:
        """Time the given routes and record the winner (planner.py:886-938)."""
        usable = {name: fn for name, fn in candidates.items() if name in ROUTES}
        if not usable:
            raise ValueError("candidates must include 'native' and/or 'pytorch'")
        timings = {name: self._time_ms(fn, tensor, max(0, int(warmup)), max(1, int(trials)))
                   for name, fn in usable.items()}
        return self.record_operator_benchmark(op, tensor, timings, training=training, extra=extra), timings


@dataclass
class _Qualification:
    """One qualification run: the correctness gate, the timing race and the
    freeze, with what each phase learned."""
    planner: MLBricksExecutionPlanner
    tensor: torch.Tensor
    usable: dict[str, Callable[[], object]]
    rtol: float | None
    atol: float | None
    timings: dict[str, float] = field(default_factory=dict)
    errors: dict[str, str] = field(default_factory=dict)
    parity: dict[str, object] = field(default_factory=lambda: {"checked": False, "allclose": None})

    def _settle(self) -> None:
        if self.tensor.is_cuda:
            torch.cuda.synchronize(self.tensor.device)

    def parity_gate(self) -> str | None:
        """Run PyTorch, then native, and compare.  Returns the rejection
        reason, or None when native matched (then it may race)."""
        rtol, atol = _default_tolerances(self.tensor)
        rtol = max(0.0, float(rtol if self.rtol is None else self.rtol))
        atol = max(0.0, float(atol if self.atol is None else self.atol))
        try:
            reference = self.usable["pytorch"]()
            self._settle()
        except Exception as exc:
            self.errors["pytorch_reference"] = f"{type(exc).__name__}: {exc}"
            self.parity = {"checked": False, "allclose": None, "rtol": rtol, "atol": atol,
                           "reference_error": self.errors["pytorch_reference"]}
            return "correctness-gate:reference-error;pytorch"
        try:
            candidate = self.usable["native"]()
            self._settle()
        except Exception as exc:
            self.errors["native_validation"] = f"{type(exc).__name__}: {exc}"
            self.parity = {"checked": True, "allclose": False, "rtol": rtol, "atol": atol,
                           "mismatch": "native candidate raised during correctness validation"}
            return "correctness-gate:native-error;pytorch"
        report = compare_outputs(reference, candidate, rtol=rtol, atol=atol)
        self.parity = report.as_dict()
        return None if report.allclose else "correctness-gate:parity-failed;pytorch"

    def race(self, warmup: int, trials: int) -> None:
        for name, fn in self.usable.items():
            try:
                self.timings[name] = self.planner._time_ms(fn, self.tensor, warmup, trials)
            except Exception as exc:
                self.errors[name] = f"{type(exc).__name__}: {exc}"

    def winner(self, default: str, margin: float) -> str:
        """The fastest route, unless the default is within `margin` of it."""
        fastest = min(self.timings, key=self.timings.__getitem__)
        if fastest == default or default not in self.timings:
            return fastest
        base = self.timings[default]
        gain = (base - self.timings[fastest]) / max(base, 1e-12)
        return fastest if gain >= margin else default

    def race_reason(self) -> str:
        head = "correctness-pass;benchmark-once:" if self.parity.get("checked") else "benchmark-once:"
        text = head + ",".join(f"{name}={self.timings[name]:.6f}ms" for name in sorted(self.timings))
        if self.errors:
            text += ";errors=" + ",".join(f"{name}:{msg}" for name, msg in sorted(self.errors.items()))
        return text

    def freeze(self, owner: object, key: tuple[object, ...], slot: tuple[str, bool], route: str,
               reason: str) -> str:
        self.planner._record(key, route, reason, self.timings)
        _owner_dict(owner, _OWNER_ROUTES)[slot] = route
        _owner_dict(owner, _OWNER_DETAILS)[slot] = {
            "route": route, "timings_ms": dict(self.timings), "errors": dict(self.errors),
            "parity": dict(self.parity), "reason": reason,
        }
        return route


EXECUTION_PLANNER = MLBricksExecutionPlanner()

__all__ = [
    "AUTO_OPERATOR_DEFAULTS",
    "ROUTES",
    "HardwareProfile",
    "MLBricksExecutionPlanner",
    "EXECUTION_PLANNER",
    "RouteDecision",
    "ParityReport",
    "compare_outputs",
    "ceil_power_of_two",
    "sequence_bucket",
]
