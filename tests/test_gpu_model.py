"""Model-level ElasticBit on the GPU, mirroring the reference's
tests/test_elasticbit_native.py (threshold contract, model compress / policy
switch / artifact round trip) plus planner routing of the HIP path."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mlbricks_amd.elasticbit._native  # noqa: F401  fails loudly when the library is missing


def _rel(a, b) -> float:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-12))


def test_threshold_contract_and_policy_switch(tmp_path):
    from mlbricks_amd import ElasticBit

    rng = np.random.default_rng(20260918)
    weights = rng.normal(0, 0.04, size=(96, 128)).astype(np.float32)
    calib = rng.normal(0, 1, size=(12, 128)).astype(np.float32)
    thr = 0.02
    analysis = ElasticBit.analyze(weights, calib, thr)
    assert 3 <= analysis.selectedBits <= 16
    assert analysis.selectedError <= thr + 1e-12
    matrix = ElasticBit.compressMatrix(weights, calib, thr)
    assert matrix.storageBits == analysis.selectedBits
    assert matrix.activateDType == "float16"
    assert matrix.executionPlanner == "gfx950BitPlane"
    x = calib[0]
    hw = np.asarray(matrix.forward(x))
    matrix.setDecodePolicy("fullPrecision")
    full = np.asarray(matrix.forward(x))
    assert _rel(hw, full) <= 2.0 * thr + 1e-3
    path = tmp_path / "matrix.mlb"
    matrix.setDecodePolicy("hardwareNative")
    matrix.save(path)
    loaded = ElasticBit.loadMatrix(path, decodePolicy="hardwareNative")
    # deterministic execution map: a reload is bitwise stable
    np.testing.assert_array_equal(np.asarray(loaded.forward(x)), hw)


def test_model_compress_switch_and_artifact(tmp_path):
    from mlbricks_amd import ElasticBit

    torch.manual_seed(20260918)
    model = torch.nn.Sequential(torch.nn.Linear(64, 96), torch.nn.GELU(),
                                torch.nn.Linear(96, 32)).cuda().half().eval()
    calib = [torch.randn(4, 64, device="cuda", dtype=torch.float16) for _ in range(2)]
    ElasticBit.compress(model, calib, 0.03)
    assert len(model.elasticbit.compressedNames) == 2
    prefill_x = torch.randn(40, 64, device="cuda", dtype=torch.float16)
    with torch.inference_mode():
        y = model(prefill_x)
    assert y.shape == (40, 32) and torch.isfinite(y).all()
    x = torch.randn(1, 64, device="cuda", dtype=torch.float16)
    with torch.inference_mode():
        model.elasticbit.setDecodePolicy("hardwareNative")
        hw = model(x).detach()
        model.elasticbit.setDecodePolicy("fullPrecision")
        full = model(x).detach()
    assert torch.nn.functional.cosine_similarity(hw.float(), full.float(), dim=-1).item() > 0.999
    artifact = tmp_path / "model.elasticbit"
    ElasticBit.save(model, artifact)
    shell = torch.nn.Sequential(torch.nn.Linear(64, 96), torch.nn.GELU(),
                                torch.nn.Linear(96, 32)).cuda().half().eval()
    ElasticBit.load(shell, artifact, decodePolicy="fullPrecision")
    with torch.inference_mode():
        restored = shell(x).detach()
    torch.testing.assert_close(restored, full, atol=0, rtol=0)


def test_compressed_layer_matches_uncompressed_linear():
    from mlbricks_amd import ElasticBit

    torch.manual_seed(1)
    lin = torch.nn.Linear(256, 512, bias=True).cuda().half()
    model = torch.nn.Sequential(lin).eval()
    ref_w = lin.weight.detach().clone()
    ref_b = lin.bias.detach().clone()
    ElasticBit.compress(model, torch.randn(32, 256, device="cuda", dtype=torch.float16), 0.01)
    layer = model[0]
    for M in (1, 8, 64):
        x = torch.randn(M, 256, device="cuda", dtype=torch.float16)
        with torch.inference_mode():
            y = model(x).float()
        ref = torch.nn.functional.linear(x.float(), ref_w.float(), ref_b.float())
        assert _rel(y.cpu(), ref.cpu()) <= 0.02          # the compression threshold plus fp16 output
    assert layer.matrix.storageBits <= 16


def test_planner_qualifies_and_freezes_the_native_route():
    from mlbricks_amd import EXECUTION_PLANNER, ElasticBit

    torch.manual_seed(2)
    model = torch.nn.Sequential(torch.nn.Linear(1024, 1024, bias=False)).cuda().half().eval()
    ElasticBit.compress(model, torch.randn(32, 1024, device="cuda", dtype=torch.float16), 0.01)
    layer = model[0]
    x = torch.randn(1, 1024, device="cuda", dtype=torch.float16)
    with torch.inference_mode():
        y = model(x)
    decode = EXECUTION_PLANNER.owner_routes(layer._routeOwners["decode"])
    assert decode == {("elastic_linear", False): "native"}
    details = layer._routeOwners["decode"]._mlbricks_frozen_auto_details[("elastic_linear", False)]
    assert details["parity"]["allclose"] is True
    with torch.inference_mode():
        assert torch.equal(model(x), y)
    layer.set_backend("pytorch")
    with torch.inference_mode():
        yp = model(x)
    assert _rel(yp.float().cpu(), y.float().cpu()) < 5e-3
    layer.set_backend("native")
    with torch.inference_mode():
        assert torch.equal(model(x), y)


def test_grad_mode_with_requires_grad_takes_pytorch_route():
    from mlbricks_amd import ElasticBit

    model = torch.nn.Sequential(torch.nn.Linear(64, 32, bias=False)).cuda().half()
    ElasticBit.compress(model, torch.randn(8, 64, device="cuda", dtype=torch.float16), 0.01)
    x = torch.randn(2, 64, device="cuda", dtype=torch.float16, requires_grad=True)
    y = model(x)
    y.float().sum().backward()
    assert x.grad is not None and x.grad.shape == x.shape


def test_attention_projections_with_zero_head_gate_in_one_launch():
    """A configs[4]-style attention block (bolt/enhanced_mqa.py:128-135):
    q 1024x1024, k and v 64x1024 and a zero-initialised 16x1024 head_gate
    with bias, each compressed by ElasticBit.compress.  The zero head_gate
    selects b = 3 with scale 1 and all-zero codes, so its output is its bias
    exactly.  RuntimeMatrix.forwardTorchMulti over the four equals each
    matrix's own native forward bit for bit, and the modules' forwards
    (whichever route the planner keeps) within the output tolerance."""
    from mlbricks_amd import ElasticBit
    from mlbricks_amd.elasticbit import RuntimeMatrix

    torch.manual_seed(0)
    layers = []
    for out_f, bias, zero in ((1024, False, False), (64, False, False), (64, False, False), (16, True, True)):
        lin = torch.nn.Linear(1024, out_f, bias=bias)
        if zero:
            torch.nn.init.zeros_(lin.weight)
        model = torch.nn.Sequential(lin).cuda().half().eval()
        ElasticBit.compress(model, torch.randn(32, 1024, generator=torch.Generator().manual_seed(out_f)).half(), 0.01)
        layers.append(model[0])
    gate = layers[3]
    assert gate.matrix.storageBits == 3
    scales, payload = gate.matrix._native._canonical()
    assert np.all(scales == 1.0)
    assert np.all(gate.matrix._native._unpackCodesTorch().cpu().numpy() == 0)
    for M in (1, 4, 16):
        x = torch.randn(M, 1024, generator=torch.Generator().manual_seed(M)).half().cuda()
        with torch.inference_mode():
            singles = [l.matrix._native.forwardTorch(x, bias=l.bias) for l in layers]
            modules = [l(x) for l in layers]
            fused = RuntimeMatrix.forwardTorchMulti([l.matrix for l in layers], x, [l.bias for l in layers])
        for j, (a, b, c) in enumerate(zip(fused, singles, modules)):
            assert torch.equal(a, b), (M, j)
            ref = float(c.float().abs().max())
            assert float((a.float() - c.float()).abs().max()) <= 2e-3 * max(ref, 1e-6), (M, j)
        assert torch.equal(fused[3], gate.bias.detach().expand(M, 16))
