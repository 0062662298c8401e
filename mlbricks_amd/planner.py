"""Operator routing planner (the ``elastic_linear`` part of MLBricks' planner).

Behaviour follows ``mlbricks/planner.py``: explicit ``native`` / ``pytorch``
requests are never overridden; ``auto`` resolves once per owning element --
a one-time parity gate against the PyTorch route, a small timing race, a
hysteresis band around ``AUTO_OPERATOR_DEFAULTS`` -- and then stays frozen on
the owner until ``clear_owner_routes``.  The ESA resource model of the
reference planner (Compass / hierarchy sizing) is not on the ElasticBit path
and is not part of this package.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Callable, Final, Mapping

import torch

from .runtime import normalize_backend

# Conservative initial route; a qualification race overrides it
# (planner.py:53: ElasticBit starts on the PyTorch route).
AUTO_OPERATOR_DEFAULTS: Final[dict[str, str]] = {
    "elastic_linear": "pytorch",
}

_ROUTES = ("native", "pytorch")


def ceil_power_of_two(value: int) -> int:
    value = max(1, int(value))
    return 1 << ((value - 1).bit_length())


def sequence_bucket(length: int) -> int:
    """Power-of-two bucket (>= 64) for sequence lengths (planner.py:70-72)."""
    return max(64, ceil_power_of_two(int(length)))


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


class MLBricksExecutionPlanner:
    """Route cache for backend-aware operators (planner.py:88-1053)."""

    def __init__(self) -> None:
        self.operator_cache: dict[tuple[object, ...], str] = {}
        self.operator_benchmarks: dict[tuple[object, ...], dict[str, float]] = {}
        self.operator_reasons: dict[tuple[object, ...], str] = {}
        self._operator_revision = 0

    # -- keys ---------------------------------------------------------------

    @staticmethod
    def _device_index(device: torch.device | str) -> int:
        resolved = torch.device(device)
        return int(resolved.index) if resolved.index is not None else int(torch.cuda.current_device())

    def hardware_profile(self, device: torch.device | str) -> HardwareProfile:
        if not torch.cuda.is_available():
            raise RuntimeError("GPU hardware profile requested without a HIP device")
        index = self._device_index(device)
        props = torch.cuda.get_device_properties(index)
        return HardwareProfile(
            device_index=index,
            compute_capability=(int(props.major), int(props.minor)),
            multiprocessors=int(props.multi_processor_count),
            warp_size=int(getattr(props, "warp_size", 64)),
            max_threads_per_sm=int(getattr(props, "max_threads_per_multi_processor", 2048)),
        )

    def _device_signature(self, tensor: torch.Tensor) -> tuple[object, ...]:
        if tensor.is_cuda and torch.cuda.is_available():
            hw = self.hardware_profile(tensor.device)
            return ("cuda", hw.device_index, hw.compute_capability, hw.multiprocessors, hw.warp_size)
        return (tensor.device.type, tensor.device.index)

    def operator_key(self, op: str, tensor: torch.Tensor, *, training: bool,
                     extra: tuple[object, ...] = ()) -> tuple[object, ...]:
        """Exact batch / feature dims with a bucketed sequence dim (planner.py:230-256)."""
        shape = tuple(int(v) for v in tensor.shape)
        if len(shape) >= 3:
            bucketed = shape[:-2] + (sequence_bucket(shape[-2]), shape[-1])
        else:
            bucketed = shape
        return ("op", str(op), *self._device_signature(tensor), str(tensor.dtype), bucketed,
                bool(training), *tuple(extra))

    @property
    def operator_revision(self) -> int:
        return int(self._operator_revision)

    # -- per-owner frozen routes -----------------------------------------------

    @staticmethod
    def _owner_cache(owner: object) -> dict:
        cache = getattr(owner, "_mlbricks_frozen_auto_routes", None)
        if not isinstance(cache, dict):
            cache = {}
            try:
                setattr(owner, "_mlbricks_frozen_auto_routes", cache)
            except Exception:
                pass
        return cache

    @staticmethod
    def clear_owner_routes(owner: object) -> None:
        """Forget one element's frozen auto decisions (planner.py:420-433)."""
        for name, value in (("_mlbricks_frozen_auto_routes", {}), ("_mlbricks_auto_route_cache", None),
                            ("_mlbricks_frozen_auto_details", {})):
            try:
                setattr(owner, name, value)
            except Exception:
                pass

    @staticmethod
    def owner_routes(owner: object) -> dict[tuple[object, ...], str]:
        cache = getattr(owner, "_mlbricks_frozen_auto_routes", None)
        if not isinstance(cache, dict):
            return {}
        return {k: v for k, v in cache.items() if v in _ROUTES}

    def _auto_default(self, op: str, *, fallback: str | None = None) -> str:
        value = str(fallback or AUTO_OPERATOR_DEFAULTS.get(str(op), "pytorch")).lower()
        return value if value in _ROUTES else "pytorch"

    def select_operator_once(self, owner: object, op: str, tensor: torch.Tensor, *,
                             requested_backend: str = "auto", native_available: bool,
                             native_supports_training: bool = False, training: bool | None = None,
                             extra: tuple[object, ...] = (), default_auto: str | None = None) -> str:
        """Resolve ``auto`` once per owner and keep it (planner.py:361-417)."""
        policy = normalize_backend(requested_backend, warn_legacy=True)
        is_training = bool(torch.is_grad_enabled()) if training is None else bool(training)
        if policy != "auto":
            return self.select_operator(op, tensor, requested_backend=policy,
                                        native_available=native_available,
                                        native_supports_training=native_supports_training,
                                        training=is_training, extra=extra, default_auto=default_auto)
        cache = self._owner_cache(owner)
        key = (str(op), is_training)
        route = cache.get(key)
        if route in _ROUTES:
            return route
        route = self.select_operator(op, tensor, requested_backend="auto", native_available=native_available,
                                     native_supports_training=native_supports_training,
                                     training=is_training, extra=extra, default_auto=default_auto)
        cache[key] = route
        return route

    # -- parity gate -----------------------------------------------------------

    @staticmethod
    def _parity_tolerances(tensor: torch.Tensor, *, rtol: float | None, atol: float | None) -> tuple[float, float]:
        """2e-2 for half types, 1e-4 / 1e-5 otherwise (planner.py:453-465)."""
        low = tensor.dtype in (torch.float16, torch.bfloat16)
        if rtol is None:
            rtol = 2.0e-2 if low else 1.0e-4
        if atol is None:
            atol = 2.0e-2 if low else 1.0e-5
        return max(0.0, float(rtol)), max(0.0, float(atol))

    @classmethod
    def _compare_candidate_outputs(cls, reference: object, candidate: object, *, rtol: float, atol: float,
                                   path: str = "output") -> tuple[bool, dict[str, object]]:
        """Structural compare with ``allclose`` at tensor leaves (planner.py:467-568)."""
        stats: dict[str, object] = {"checked": True, "allclose": True, "rtol": float(rtol),
                                    "atol": float(atol), "tensor_leaves": 0, "max_abs": 0.0,
                                    "max_relative_l2": 0.0, "mismatch": None}

        def fail(where: str, reason: str) -> bool:
            stats["allclose"] = False
            if stats["mismatch"] is None:
                stats["mismatch"] = f"{where}: {reason}"
            return False

        def visit(ref: object, cand: object, where: str) -> bool:
            if torch.is_tensor(ref) or torch.is_tensor(cand):
                if not (torch.is_tensor(ref) and torch.is_tensor(cand)):
                    return fail(where, "tensor/non-tensor type mismatch")
                if tuple(ref.shape) != tuple(cand.shape):
                    return fail(where, f"shape {tuple(ref.shape)} != {tuple(cand.shape)}")
                r = ref.detach()
                c = cand.detach().to(r.device)
                if r.is_floating_point() or r.is_complex():
                    kind = torch.complex64 if r.is_complex() else torch.float32
                    rn, cn = r.to(kind), c.to(kind)
                    diff = (cn - rn).abs()
                    if diff.numel():
                        stats["max_abs"] = max(float(stats["max_abs"]), float(diff.max().item()))
                        rel = float((torch.linalg.vector_norm((cn - rn).reshape(-1)) /
                                     (torch.linalg.vector_norm(rn.reshape(-1)) + 1.0e-12)).item())
                        stats["max_relative_l2"] = max(float(stats["max_relative_l2"]), rel)
                    close = bool(torch.allclose(cn, rn, rtol=rtol, atol=atol, equal_nan=False))
                else:
                    close = bool(torch.equal(c, r))
                stats["tensor_leaves"] = int(stats["tensor_leaves"]) + 1
                return True if close else fail(where, "tensor values differ from PyTorch reference")
            if isinstance(ref, Mapping) or isinstance(cand, Mapping):
                if not (isinstance(ref, Mapping) and isinstance(cand, Mapping)):
                    return fail(where, "mapping/non-mapping type mismatch")
                if set(ref.keys()) != set(cand.keys()):
                    return fail(where, "mapping keys differ")
                ok = True
                for key in sorted(ref.keys(), key=repr):
                    ok = visit(ref[key], cand[key], f"{where}[{key!r}]") and ok
                return ok
            if isinstance(ref, (tuple, list)) or isinstance(cand, (tuple, list)):
                if type(ref) is not type(cand):
                    return fail(where, f"sequence types differ: {type(ref).__name__} != {type(cand).__name__}")
                if len(ref) != len(cand):
                    return fail(where, f"sequence lengths differ: {len(ref)} != {len(cand)}")
                ok = True
                for i, (a, b) in enumerate(zip(ref, cand)):
                    ok = visit(a, b, f"{where}[{i}]") and ok
                return ok
            if ref is None or cand is None:
                return True if ref is cand else fail(where, "None/non-None mismatch")
            try:
                equal = bool(ref == cand)
            except Exception:
                equal = repr(ref) == repr(cand)
            return True if equal else fail(where, f"value mismatch: {ref!r} != {cand!r}")

        ok = visit(reference, candidate, path)
        stats["allclose"] = bool(ok and stats["allclose"])
        return bool(stats["allclose"]), stats

    # -- qualification ----------------------------------------------------------

    def _time_ms(self, fn: Callable[[], object], tensor: torch.Tensor, warmup: int, trials: int) -> float:
        for _ in range(warmup):
            fn()
        samples: list[float] = []
        if tensor.is_cuda:
            torch.cuda.synchronize(tensor.device)
            for _ in range(trials):
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record()
                fn()
                end.record()
                end.synchronize()
                samples.append(float(start.elapsed_time(end)))
        else:
            for _ in range(trials):
                t0 = time.perf_counter()
                fn()
                samples.append((time.perf_counter() - t0) * 1000.0)
        samples.sort()
        return samples[len(samples) // 2]

    def qualify_operator_once(self, owner: object, op: str, tensor: torch.Tensor,
                              candidates: Mapping[str, Callable[[], object]], *,
                              requested_backend: str = "auto", native_available: bool,
                              native_supports_training: bool = False, training: bool | None = None,
                              extra: tuple[object, ...] = (), default_auto: str | None = None,
                              warmup: int = 2, trials: int = 5, switch_margin: float = 0.05,
                              verify_parity: bool = True, parity_rtol: float | None = None,
                              parity_atol: float | None = None) -> str:
        """Validate and time one element once, then freeze its route (planner.py:570-776)."""
        policy = normalize_backend(requested_backend, warn_legacy=True)
        is_training = bool(torch.is_grad_enabled()) if training is None else bool(training)
        common = dict(native_available=native_available, native_supports_training=native_supports_training,
                      training=is_training, extra=extra, default_auto=default_auto)
        if policy != "auto":
            return self.select_operator(op, tensor, requested_backend=policy, **common)
        if is_training and not native_supports_training:
            return "pytorch"
        if not native_available:
            return self.select_operator_once(owner, op, tensor, requested_backend="auto", **common)

        cache = self._owner_cache(owner)
        frozen_key = (str(op), is_training)
        if cache.get(frozen_key) in _ROUTES:
            return cache[frozen_key]

        usable = {str(k): fn for k, fn in candidates.items() if str(k) in _ROUTES and callable(fn)}
        if not usable:
            return self.select_operator_once(owner, op, tensor, requested_backend="auto", **common)

        key = self.operator_key(op, tensor, training=is_training, extra=extra)
        timings: dict[str, float] = {}
        errors: dict[str, str] = {}
        parity: dict[str, object] = {"checked": False, "allclose": None}

        def freeze(route: str, reason: str) -> str:
            self.operator_benchmarks[key] = dict(timings)
            if self.operator_cache.get(key) != route:
                self._operator_revision += 1
            self.operator_cache[key] = route
            self.operator_reasons[key] = reason
            cache[frozen_key] = route
            try:
                details = getattr(owner, "_mlbricks_frozen_auto_details", None)
                if not isinstance(details, dict):
                    details = {}
                    setattr(owner, "_mlbricks_frozen_auto_details", details)
                details[frozen_key] = {"route": route, "timings_ms": dict(timings), "errors": dict(errors),
                                       "parity": dict(parity), "reason": reason}
            except Exception:
                pass
            return route

        # Correctness gate: PyTorch is the reference; native may race only after matching it.
        if verify_parity and "pytorch" in usable and "native" in usable:
            rtol, atol = self._parity_tolerances(tensor, rtol=parity_rtol, atol=parity_atol)
            try:
                reference = usable["pytorch"]()
                if tensor.is_cuda:
                    torch.cuda.synchronize(tensor.device)
            except Exception as exc:
                errors["pytorch_reference"] = f"{type(exc).__name__}: {exc}"
                parity.update({"checked": False, "allclose": None, "rtol": rtol, "atol": atol,
                               "reference_error": errors["pytorch_reference"]})
                return freeze("pytorch", "correctness-gate:reference-error;pytorch")
            try:
                native_out = usable["native"]()
                if tensor.is_cuda:
                    torch.cuda.synchronize(tensor.device)
            except Exception as exc:
                errors["native_validation"] = f"{type(exc).__name__}: {exc}"
                parity.update({"checked": True, "allclose": False, "rtol": rtol, "atol": atol,
                               "mismatch": "native candidate raised during correctness validation"})
                return freeze("pytorch", "correctness-gate:native-error;pytorch")
            ok, details = self._compare_candidate_outputs(reference, native_out, rtol=rtol, atol=atol)
            parity.clear()
            parity.update(details)
            if not ok:
                return freeze("pytorch", "correctness-gate:parity-failed;pytorch")

        warmup = max(0, int(warmup))
        trials = max(1, int(trials))
        for name, fn in usable.items():
            try:
                timings[name] = self._time_ms(fn, tensor, warmup, trials)
            except Exception as exc:
                errors[name] = f"{type(exc).__name__}: {exc}"

        if not timings:
            return self.select_operator_once(owner, op, tensor, requested_backend="auto", **common)

        fastest = min(timings, key=timings.get)
        default = self._auto_default(op, fallback=default_auto)
        route = fastest
        if default in timings and fastest != default:
            base = float(timings[default])
            gain = (base - float(timings[fastest])) / max(base, 1.0e-12)
            if gain < max(0.0, float(switch_margin)):
                route = default
        reason = "correctness-pass;benchmark-once:" if parity.get("checked") else "benchmark-once:"
        reason += ",".join(f"{name}={ms:.6f}ms" for name, ms in sorted(timings.items()))
        if errors:
            reason += ";errors=" + ",".join(f"{k}:{v}" for k, v in sorted(errors.items()))
        return freeze(route, reason)

    def select_operator(self, op: str, tensor: torch.Tensor, *, requested_backend: str = "auto",
                        native_available: bool, native_supports_training: bool = False,
                        training: bool | None = None, extra: tuple[object, ...] = (),
                        default_auto: str | None = None) -> str:
        """Resolve one call to ``native`` or ``pytorch`` (planner.py:778-835)."""
        policy = normalize_backend(requested_backend, warn_legacy=True)
        is_training = bool(torch.is_grad_enabled()) if training is None else bool(training)
        if policy == "pytorch":
            return "pytorch"
        if policy == "native":
            if not native_available:
                raise RuntimeError(f"backend='native' requested but native route for {op!r} is unavailable")
            if is_training and not native_supports_training:
                raise RuntimeError(f"backend='native' requested for {op!r}, but its native route is "
                                   "inference-only for this call")
            return "native"
        key = self.operator_key(op, tensor, training=is_training, extra=extra)
        if is_training and not native_supports_training:
            self.operator_cache[key] = "pytorch"
            self.operator_reasons[key] = "training-safe:pytorch"
            return "pytorch"
        if not native_available:
            self.operator_cache[key] = "pytorch"
            self.operator_reasons[key] = "native-unavailable:pytorch"
            return "pytorch"
        cached = self.operator_cache.get(key)
        if cached in _ROUTES:
            return cached
        route = self._auto_default(op, fallback=default_auto)
        self.operator_cache[key] = route
        self.operator_reasons[key] = f"heuristic:{route}"
        return route

    def set_operator_route(self, op: str, tensor: torch.Tensor, route: str, *, training: bool = False,
                           extra: tuple[object, ...] = (), reason: str = "manual") -> str:
        value = str(route).strip().lower()
        if value not in _ROUTES:
            raise ValueError("route must be 'native' or 'pytorch'")
        key = self.operator_key(op, tensor, training=training, extra=extra)
        if self.operator_cache.get(key) != value:
            self._operator_revision += 1
        self.operator_cache[key] = value
        self.operator_reasons[key] = str(reason)
        return value

    def record_operator_benchmark(self, op: str, tensor: torch.Tensor, timings_ms: Mapping[str, float], *,
                                  training: bool = False, extra: tuple[object, ...] = ()) -> str:
        valid = {str(k): float(v) for k, v in timings_ms.items() if str(k) in _ROUTES and float(v) > 0.0}
        if not valid:
            raise ValueError("timings_ms must contain positive native/pytorch timings")
        winner = min(valid, key=valid.get)
        key = self.operator_key(op, tensor, training=training, extra=extra)
        if self.operator_cache.get(key) != winner:
            self._operator_revision += 1
        self.operator_benchmarks[key] = valid
        self.operator_cache[key] = winner
        self.operator_reasons[key] = "benchmark:" + ",".join(f"{k}={v:.6f}ms" for k, v in sorted(valid.items()))
        return winner

    def benchmark_candidates(self, op: str, tensor: torch.Tensor,
                             candidates: Mapping[str, Callable[[], object]], *, warmup: int = 5,
                             trials: int = 20, training: bool = False,
                             extra: tuple[object, ...] = ()) -> tuple[str, dict[str, float]]:
        """Explicit calibration: time candidates and cache the winner (planner.py:886-938)."""
        usable = {k: v for k, v in candidates.items() if k in _ROUTES}
        if not usable:
            raise ValueError("candidates must include 'native' and/or 'pytorch'")
        timings = {name: self._time_ms(fn, tensor, max(0, int(warmup)), max(1, int(trials)))
                   for name, fn in usable.items()}
        return self.record_operator_benchmark(op, tensor, timings, training=training, extra=extra), timings

    def operator_decisions(self) -> list[dict[str, object]]:
        return [{"key": key, "route": route, "reason": self.operator_reasons.get(key, "cached"),
                 "benchmarks_ms": self.operator_benchmarks.get(key)}
                for key, route in self.operator_cache.items()]

    def clear(self) -> None:
        self.operator_cache.clear()
        self.operator_benchmarks.clear()
        self.operator_reasons.clear()
        self._operator_revision += 1


EXECUTION_PLANNER = MLBricksExecutionPlanner()

__all__ = [
    "AUTO_OPERATOR_DEFAULTS",
    "HardwareProfile",
    "MLBricksExecutionPlanner",
    "EXECUTION_PLANNER",
    "ceil_power_of_two",
    "sequence_bucket",
]
