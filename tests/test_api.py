"""Public API contract, mirroring the reference's tests/test_elasticbit.py and
its planner tests (tests/test_unified_execution_planner.py,
tests/test_stable_auto_routes.py, tests/test_elementwise_auto_planner.py).
CPU only."""
from __future__ import annotations

import inspect
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn

import mlbricks_amd as mlb
import mlbricks_amd.planner as planner_module
from mlbricks_amd import EXECUTION_PLANNER, BackendInfo, ElasticBit, RuntimeMatrix
from mlbricks_amd.elasticbit.core import _ElasticLinear, _semanticOutputWeightIds
from mlbricks_amd.planner import AUTO_OPERATOR_DEFAULTS, MLBricksExecutionPlanner
from mlbricks_amd.runtime import normalize_backend, set_module_backend


def test_clean_public_surface_has_no_fixed_bit_api():
    for name in ("bits", "quantize", "dequantize", "quantize_module", "apply"):
        assert not hasattr(ElasticBit, name)
    assert not hasattr(RuntimeMatrix, "from_auto")
    assert not hasattr(RuntimeMatrix, "auto")


def test_public_api_uses_camel_case_names():
    sig = inspect.signature(ElasticBit.compressMatrix)
    assert "calibrationData" in sig.parameters
    assert sig.parameters["decodePolicy"].default == "hardwareNative"
    assert inspect.signature(ElasticBit.loadMatrix).parameters["decodePolicy"].default == "hardwareNative"
    assert inspect.signature(RuntimeMatrix.compress).parameters["decodePolicy"].default == "hardwareNative"
    assert inspect.signature(RuntimeMatrix.load).parameters["decodePolicy"].default == "hardwareNative"
    assert inspect.signature(ElasticBit.compress).parameters["preserveOutputHead"].default is True
    assert hasattr(RuntimeMatrix, "setDecodePolicy")


def test_backend_api_reports_this_build():
    info = ElasticBit.backend()
    assert isinstance(info, BackendInfo)
    assert isinstance(info.available, bool)
    assert info.validated is False
    if info.available:
        assert info.prefill == "native"
        assert info.architecture == "gfx950"
        assert info.decodePlanner == "gfx950BitPlane"
        assert info.decodeEngine == "BitPlaneMFMA"
        assert info.decodeStatus == "experimental"
        assert info.decodeValidation == "unvalidated"
        assert info.weightWidths == tuple(range(3, 17))
    else:
        assert "ElasticBitBackend(unavailable" in str(info)


def test_semantic_output_head_detection_is_model_agnostic():
    class ToyDecoder(nn.Module):
        def __init__(self):
            super().__init__()
            self.embed = nn.Embedding(31, 8)
            self.block = nn.Linear(8, 8, bias=False)
            self.vocab_projection = nn.Linear(8, 31, bias=False)

        def get_output_embeddings(self):
            return self.vocab_projection

    model = ToyDecoder()
    assert _semanticOutputWeightIds(model) == {id(model.vocab_projection.weight)}


def test_compress_requires_cuda_model_and_fp16():
    model = nn.Sequential(nn.Linear(4, 4))
    with pytest.raises(RuntimeError, match="requires a CUDA model"):
        ElasticBit.compress(model, torch.randn(2, 4), 0.01)
    with pytest.raises(TypeError):
        ElasticBit.compress(object(), torch.randn(2, 4), 0.01)
    with pytest.raises(ValueError, match="decodePolicy"):
        ElasticBit.compress(model, torch.randn(2, 4), 0.01, decodePolicy="turbo")


def test_stage2_tools_are_explicitly_out_of_scope():
    with pytest.raises(NotImplementedError):
        ElasticBit.optimize(nn.Linear(2, 2))
    with pytest.raises(NotImplementedError):
        ElasticBit.reduce(nn.Linear(2, 2))


def test_normalize_backend():
    assert normalize_backend(None) == "auto"
    assert normalize_backend("NATIVE") == "native"
    assert normalize_backend("torch") == "pytorch"
    assert normalize_backend("hip") == "native"
    with pytest.raises(ValueError):
        normalize_backend("triton")


def test_elastic_linear_defaults_to_pytorch_auto_route():
    assert AUTO_OPERATOR_DEFAULTS["elastic_linear"] == "pytorch"


def test_set_module_backend_reaches_elastic_linear():
    import numpy as np

    m = mlb.RuntimeMatrix._compressSelectedCodes(np.zeros((4, 32), np.int16), np.ones(4, np.float32), 8, 0.01, 0.0)
    layer = _ElasticLinear(m, 32, 4, None)
    model = nn.Sequential(layer)
    assert layer.backend == "auto"
    set_module_backend(model, "native")
    assert layer.backend == "native"
    assert mlb.backend_report(model)[0]["requested"] == "native"


def test_native_request_without_native_route_raises():
    x = torch.randn(2, 8)
    with pytest.raises(RuntimeError, match="unavailable"):
        EXECUTION_PLANNER.select_operator("elastic_linear", x, requested_backend="native",
                                          native_available=False, training=False)


def test_auto_route_is_frozen_on_owner_until_explicit_reset():
    EXECUTION_PLANNER.clear()

    class Owner:
        pass

    owner = Owner()
    x = torch.randn(2, 8)
    first = EXECUTION_PLANNER.select_operator_once(owner, "unit_test_op", x, requested_backend="auto",
                                                   native_available=True, training=False, default_auto="native")
    assert first == "native"
    EXECUTION_PLANNER.set_operator_route("unit_test_op", x, "pytorch", training=False, reason="test-change")
    assert EXECUTION_PLANNER.select_operator_once(owner, "unit_test_op", x, requested_backend="auto",
                                                  native_available=True, training=False,
                                                  default_auto="native") == "native"
    EXECUTION_PLANNER.clear_owner_routes(owner)
    assert EXECUTION_PLANNER.select_operator_once(owner, "unit_test_op", x, requested_backend="auto",
                                                  native_available=True, training=False,
                                                  default_auto="native") == "pytorch"


def _fake_clock(monkeypatch):
    clock = {"now": 0.0}
    monkeypatch.setattr(planner_module, "time", SimpleNamespace(perf_counter=lambda: clock["now"]))
    return clock


def test_qualify_benchmarks_then_freezes_fastest_route(monkeypatch):
    planner = MLBricksExecutionPlanner()
    x = torch.randn(2, 4, 8)
    clock = _fake_clock(monkeypatch)

    class Owner:
        pass

    owner = Owner()

    def fast():
        clock["now"] += 0.0005
        return x

    def slow():
        clock["now"] += 0.003
        return x

    route = planner.qualify_operator_once(owner, "unit_element", x, {"native": slow, "pytorch": fast},
                                          native_available=True, training=False, default_auto="native",
                                          warmup=0, trials=3, switch_margin=0.0)
    assert route == "pytorch"
    assert planner.owner_routes(owner) == {("unit_element", False): "pytorch"}
    again = planner.qualify_operator_once(owner, "unit_element", x, {"native": fast, "pytorch": slow},
                                          native_available=True, training=False, default_auto="native",
                                          warmup=0, trials=1, switch_margin=0.0)
    assert again == "pytorch"
    # the cheap lookup _ElasticLinear.forward uses gives the same frozen answer
    assert planner.frozen_route(owner, "unit_element") == "pytorch"
    assert planner.frozen_route(owner, "unit_element", training=True) is None
    assert planner.frozen_route(Owner(), "unit_element") is None
    planner.clear_owner_routes(owner)
    assert planner.frozen_route(owner, "unit_element") is None


def test_qualify_hysteresis_keeps_default_inside_margin(monkeypatch):
    planner = MLBricksExecutionPlanner()
    x = torch.randn(4, 8)
    clock = _fake_clock(monkeypatch)

    class Owner:
        pass

    def native():
        clock["now"] += 0.00098
        return x

    def pytorch():
        clock["now"] += 0.001
        return x

    assert planner.qualify_operator_once(Owner(), "elastic_linear", x, {"native": native, "pytorch": pytorch},
                                         native_available=True, training=False, warmup=0, trials=3) == "pytorch"


def test_parity_gate_rejects_a_wrong_native_result(monkeypatch):
    planner = MLBricksExecutionPlanner()
    x = torch.randn(4, 8)
    _fake_clock(monkeypatch)

    class Owner:
        pass

    owner = Owner()
    route = planner.qualify_operator_once(owner, "elastic_linear", x,
                                          {"native": lambda: x + 1.0, "pytorch": lambda: x},
                                          native_available=True, training=False, default_auto="native")
    assert route == "pytorch"
    details = owner._mlbricks_frozen_auto_details[("elastic_linear", False)]
    assert details["reason"] == "correctness-gate:parity-failed;pytorch"


def test_parity_gate_freezes_pytorch_when_native_raises(monkeypatch):
    planner = MLBricksExecutionPlanner()
    x = torch.randn(4, 8)
    _fake_clock(monkeypatch)

    class Owner:
        pass

    def boom():
        raise RuntimeError("kernel failed")

    owner = Owner()
    assert planner.qualify_operator_once(owner, "elastic_linear", x, {"native": boom, "pytorch": lambda: x},
                                         native_available=True, training=False) == "pytorch"
    assert "native-error" in owner._mlbricks_frozen_auto_details[("elastic_linear", False)]["reason"]


def test_training_calls_stay_on_pytorch():
    planner = MLBricksExecutionPlanner()
    x = torch.randn(4, 8)

    class Owner:
        pass

    assert planner.qualify_operator_once(Owner(), "elastic_linear", x, {"native": lambda: x},
                                         native_available=True, training=True) == "pytorch"


def test_operator_decisions_report_the_heuristic_and_benchmarks_override_it():
    """As the reference's tests/test_unified_execution_planner.py: a first
    auto call records the operator default with a 'heuristic:' reason; a
    recorded benchmark replaces it and bumps the revision."""
    planner = MLBricksExecutionPlanner()
    x = torch.randn(1, 32, 16)
    assert planner.select_operator("elastic_linear", x, native_available=True, training=False) == "pytorch"
    rows = planner.operator_decisions()
    assert len(rows) == 1 and rows[0]["route"] == "pytorch"
    assert str(rows[0]["reason"]).startswith("heuristic:")
    assert rows[0]["key"][:2] == ("op", "elastic_linear")
    revision = planner.operator_revision
    assert planner.record_operator_benchmark("elastic_linear", x, {"native": 0.2, "pytorch": 0.8},
                                             training=False) == "native"
    assert planner.operator_revision == revision + 1
    assert planner.select_operator("elastic_linear", x, native_available=True, training=False) == "native"
    assert len(planner.operator_cache) == 1
    assert planner.operator_benchmarks[rows[0]["key"]] == {"native": 0.2, "pytorch": 0.8}
    with pytest.raises(ValueError):
        planner.record_operator_benchmark("elastic_linear", x, {"native": 0.0}, training=False)


def test_select_operator_cached_is_sticky_until_a_decision_changes(monkeypatch):
    planner = MLBricksExecutionPlanner()
    x = torch.randn(2, 32, 16)
    calls = {"n": 0}
    original = planner.select_operator

    def counted(*args, **kwargs):
        calls["n"] += 1
        return original(*args, **kwargs)

    monkeypatch.setattr(planner, "select_operator", counted)

    class Owner:
        pass

    owner = Owner()
    ask = dict(requested_backend="auto", native_available=True, training=False, extra=(16,), default_auto="native")
    assert planner.select_operator_cached(owner, "elastic_linear", x, **ask) == "native"
    assert planner.select_operator_cached(owner, "elastic_linear", x, **ask) == "native"
    assert calls["n"] == 1
    planner.record_operator_benchmark("elastic_linear", x, {"native": 0.8, "pytorch": 0.2}, training=False,
                                      extra=(16,))
    assert planner.select_operator_cached(owner, "elastic_linear", x, **ask) == "pytorch"
    assert calls["n"] == 2


def test_parity_gate_compares_nested_outputs_leaf_by_leaf(monkeypatch):
    planner = MLBricksExecutionPlanner()
    x = torch.randn(2, 4, 8)
    clock = _fake_clock(monkeypatch)

    class Owner:
        pass

    def native():
        clock["now"] += 0.001
        return (x + 1.0e-6, {"state": x * 0.5 + 1.0e-6})

    def pytorch():
        clock["now"] += 0.002
        return (x, {"state": x * 0.5})

    owner = Owner()
    assert planner.qualify_operator_once(owner, "nested", x, {"native": native, "pytorch": pytorch},
                                         native_available=True, training=False, warmup=0, trials=3,
                                         switch_margin=0.0) == "native"
    details = owner._mlbricks_frozen_auto_details[("nested", False)]
    assert details["parity"]["checked"] is True and details["parity"]["allclose"] is True
    assert details["parity"]["tensor_leaves"] == 2
    assert set(details["timings_ms"]) == {"native", "pytorch"}
    assert details["reason"].startswith("correctness-pass;benchmark-once:")
    # a different structure is a mismatch, whatever the speed
    other = Owner()
    assert planner.qualify_operator_once(other, "nested", x,
                                         {"native": lambda: [x, {"state": x}], "pytorch": lambda: (x, {"state": x})},
                                         native_available=True, training=False, default_auto="native") == "pytorch"
    assert other._mlbricks_frozen_auto_details[("nested", False)]["parity"]["allclose"] is False


def test_parity_gate_never_selects_native_when_the_reference_fails(monkeypatch):
    planner = MLBricksExecutionPlanner()
    x = torch.randn(2, 4, 8)
    _fake_clock(monkeypatch)

    class Owner:
        pass

    def broken():
        raise RuntimeError("reference failed")

    owner = Owner()
    assert planner.qualify_operator_once(owner, "elastic_linear", x, {"native": lambda: x, "pytorch": broken},
                                         native_available=True, training=False, default_auto="native") == "pytorch"
    details = owner._mlbricks_frozen_auto_details[("elastic_linear", False)]
    assert details["parity"]["checked"] is False and details["parity"]["allclose"] is None
    assert "pytorch_reference" in details["errors"]
    assert details["reason"] == "correctness-gate:reference-error;pytorch"


def test_legacy_backend_names_warn_when_asked():
    with pytest.warns(DeprecationWarning):
        assert normalize_backend("cuda", warn_legacy=True) == "native"
    assert normalize_backend(" Py-Torch ".replace("-", "")) == "pytorch"
