"""CPU tests of the host-side package: public API, parameter ABI, registry, PyTorch backends
and helpers. Mirrors the reference's CPU-runnable tests (test_backends.py, test_primitives.py,
test_reference.py, test_poisson.py, test_extension_contract.py) and checks the package against
the oracle."""

from __future__ import annotations

import re
from math import pi
from pathlib import Path

import numpy as np
import pytest
import torch

import fused_hoad
from fused_hoad import (
    BACKENDS,
    DEFAULT_POISSON_MLP,
    POISSON_PARAMETER_COUNT,
    POISSON_PARAMETER_LAYOUT,
    MLPConfig,
    build_mlp,
    error_metrics,
    evaluate_poisson_residual,
    evaluate_residual,
    forward_laplacian,
    get_backend,
    gradient,
    manufactured_solution,
    manufactured_source,
    mlp_second_derivative,
    pack_poisson_parameters,
    unpack_poisson_parameters,
)
from fused_hoad.backends import FIXED_CONTRACT_BACKENDS, REFERENCE_BACKEND, TRAINABLE_BACKENDS
from oracle import jet, torch_ref

ROOT = Path(__file__).resolve().parents[1]
PRODUCT = ROOT / "expanded-gpu-optimization_amd"

CONFIGS = [
    DEFAULT_POISSON_MLP,
    MLPConfig(input_dim=3, hidden_dim=16, hidden_layers=2, activation="tanh"),
    MLPConfig(input_dim=2, hidden_dim=32, hidden_layers=3, activation="silu"),
]


def _model_and_coordinates(config, batch=64, dtype=torch.float64):
    torch.manual_seed(0)
    model = build_mlp(config).to(dtype=dtype)
    return model, torch.empty(batch, config.input_dim, dtype=dtype).uniform_(-1.0, 1.0)


def test_product_never_imports_the_oracle() -> None:
    for path in PRODUCT.rglob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", text, flags=re.MULTILINE), path


def test_layout_matches_abi_constants() -> None:
    offsets = [(s.weight_offset, s.bias_offset) for s in POISSON_PARAMETER_LAYOUT]
    assert offsets == [(0, 128), (192, 4288), (4352, 8448), (8512, 12608), (12672, 12736)]
    assert POISSON_PARAMETER_COUNT == 12737 == jet.PARAMETER_COUNT
    header = (PRODUCT / "csrc" / "mlp_abi.h").read_text()
    assert "kParameterCount == 12737" in header


def test_build_mlp_matches_the_seeded_reference_model() -> None:
    torch.manual_seed(0)
    packed = pack_poisson_parameters(build_mlp(DEFAULT_POISSON_MLP))
    assert torch.equal(packed, torch_ref.pack(torch_ref.reference_model(0)))


def test_pack_round_trip_and_differentiable_pack() -> None:
    torch.manual_seed(0)
    model = build_mlp(DEFAULT_POISSON_MLP)
    flat = pack_poisson_parameters(model)
    views = unpack_poisson_parameters(flat)
    assert torch.equal(views["layer2.weight"], model[4].weight)
    assert torch.equal(views["layer4.bias"], model[8].bias)
    diff = pack_poisson_parameters(model, differentiable=True)
    diff.sum().backward()
    assert all(torch.equal(p.grad, torch.ones_like(p)) for p in model.parameters())
    with pytest.raises(ValueError, match="12737"):
        unpack_poisson_parameters(torch.zeros(5))
    with pytest.raises(ValueError, match="linear layers"):
        pack_poisson_parameters(torch.nn.Sequential(torch.nn.Linear(2, 64)))


def test_layer_walk_and_flattened_binding_track_the_model() -> None:
    """The per-step module walk finds the linear layers in ``model.modules()`` order (nested,
    shared and ``None`` children included), and the flattened binding holds only while every
    parameter is a view of the packed buffer at its layout offset."""
    from torch import nn

    from fused_hoad.parameters import (
        _linear_layers,
        flatten_poisson_parameters_,
        flattened_poisson_binding,
        poisson_parameter_tensors,
    )

    shared = nn.Linear(3, 3)
    nested = nn.Sequential(
        nn.Linear(2, 2),
        nn.Sequential(shared, nn.Tanh(), nn.Sequential(nn.Linear(4, 4))),
        shared,
        nn.ModuleList([nn.Linear(5, 5), shared]),
    )
    nested.add_module("empty", None)
    for module in (nested, nn.Linear(2, 2), nn.Tanh(), build_mlp(DEFAULT_POISSON_MLP)):
        assert _linear_layers(module) == [m for m in module.modules() if isinstance(m, nn.Linear)]

    torch.manual_seed(0)
    model = build_mlp(DEFAULT_POISSON_MLP)
    assert flattened_poisson_binding(model) is None
    flat = flatten_poisson_parameters_(model)
    binding = flattened_poisson_binding(model)
    assert binding is not None and binding[0] is flat
    assert all(a is b for a, b in zip(binding[1], model.parameters(), strict=True))
    assert all(a is b for a, b in zip(poisson_parameter_tensors(model), model.parameters(), strict=True))
    with torch.no_grad():
        model[4].bias.data = model[4].bias.detach().clone()  # no longer a view of the buffer
    assert flattened_poisson_binding(model) is None
    flatten_poisson_parameters_(model)
    assert flattened_poisson_binding(model) is not None
    model[4] = nn.Linear(64, 64)  # a replaced layer is not in the buffer
    assert flattened_poisson_binding(model) is None
    model[4] = nn.Linear(64, 63)
    with pytest.raises(ValueError, match=r"layer2.weight must have shape \(64, 64\), got \(63, 64\)"):
        poisson_parameter_tensors(model)

    # A parametrized weight is not a registered parameter: it is read through the module (its
    # computed value), and gradients reach the parametrization's original.
    from torch.nn.utils import parametrize

    class Doubled(nn.Module):
        def forward(self, weight):
            return 2 * weight

    torch.manual_seed(0)
    model = build_mlp(DEFAULT_POISSON_MLP)
    before = model[2].weight.detach().clone()
    parametrize.register_parametrization(model[2], "weight", Doubled())
    assert torch.equal(poisson_parameter_tensors(model)[2], 2 * before)
    pack_poisson_parameters(model, differentiable=True).sum().backward()
    original = model[2].parametrizations.weight.original
    assert torch.equal(original.grad, torch.full_like(original, 2.0))


def test_bench_runs_on_one_gpu_only() -> None:
    """bench.py --gpus N with N > 1 exits (status 2) with a message, before touching a GPU."""
    import subprocess
    import sys

    result = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
        capture_output=True, text=True, timeout=300, cwd=ROOT,
    )
    assert result.returncode == 2
    assert "one GPU only" in result.stdout + result.stderr
    assert not result.stdout.strip()  # no JSON line


def test_registry_and_unknown_backend() -> None:
    assert REFERENCE_BACKEND in BACKENDS
    assert set(TRAINABLE_BACKENDS) <= set(BACKENDS)
    assert get_backend("forward_laplacian") is forward_laplacian
    with pytest.raises(KeyError, match="forward_laplacian"):
        get_backend("does-not-exist")
    # the extension is built in this tree, so the fixed-contract names are registered
    assert "fused_cuda" in FIXED_CONTRACT_BACKENDS and "fused_cuda_recompute" in BACKENDS


@pytest.mark.parametrize("config", CONFIGS, ids=lambda c: f"{c.activation}-{c.input_dim}d")
def test_forward_laplacian_matches_eager_in_float64(config) -> None:
    model, x = _model_and_coordinates(config)
    eu, el = get_backend("eager")(model, x)
    u, lap = forward_laplacian(model, x)
    assert u.shape == lap.shape == (x.shape[0], 1)
    torch.testing.assert_close(u, eu, atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(lap, el, atol=1e-10, rtol=1e-8)


@pytest.mark.parametrize("config", CONFIGS, ids=lambda c: f"{c.activation}-{c.input_dim}d")
def test_func_backend_matches_eager_in_float64(config) -> None:
    model, x = _model_and_coordinates(config)
    eu, el = get_backend("eager")(model, x)
    u, lap = get_backend("func")(model, x)
    assert u.shape == lap.shape == (x.shape[0], 1)
    torch.testing.assert_close(u, eu, atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(lap, el, atol=1e-10, rtol=1e-8)
    with pytest.raises(ValueError, match="batch, dimensions"):
        get_backend("func")(model, x[0])


@pytest.mark.parametrize("name", ["eager", "forward_laplacian"])
def test_graph_backends_call_their_base_backend_off_the_gpu(name: str) -> None:
    model, x = _model_and_coordinates(DEFAULT_POISSON_MLP, batch=16)
    want = get_backend(name)(model, x)
    got = get_backend(f"{name}_cudagraph")(model, x)
    for g, w in zip(got, want, strict=True):
        assert torch.equal(g, w)


def test_forward_laplacian_matches_oracle_jet() -> None:
    model, x = _model_and_coordinates(DEFAULT_POISSON_MLP, batch=40)
    flat = pack_poisson_parameters(model)
    u, lap = forward_laplacian(model, x)
    eu, el = jet.forward(flat.numpy(), x.numpy())
    np.testing.assert_allclose(u.detach().numpy().ravel(), eu, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(lap.detach().numpy().ravel(), el, rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("batch", [256, 1024])
def test_forward_laplacian_matches_eager_in_float32(batch: int) -> None:
    """1,024 points is BASELINE.json config 1 (the CPU residual), checked at its stated size
    with the north star's FP32 tolerance."""
    model, x = _model_and_coordinates(DEFAULT_POISSON_MLP, batch=batch, dtype=torch.float32)
    eu, expected = get_backend("eager")(model, x)
    u, actual = forward_laplacian(model, x)
    torch.testing.assert_close(u, eu, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(actual, expected, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("name", TRAINABLE_BACKENDS)
def test_parameter_gradients_match_eager(name: str) -> None:
    model, x = _model_and_coordinates(DEFAULT_POISSON_MLP, batch=32)

    def grads(backend):
        model.zero_grad()
        _, lap = get_backend(backend)(model, x)
        lap.pow(2).mean().backward()
        return [torch.zeros_like(p) if p.grad is None else p.grad.clone() for p in model.parameters()]

    for got, want in zip(grads(name), grads(REFERENCE_BACKEND), strict=True):
        torch.testing.assert_close(got, want, atol=1e-10, rtol=1e-8)


def test_recompute_backward_matches_oracle() -> None:
    from fused_hoad.backends.fused import _recompute_backward

    model, x = _model_and_coordinates(DEFAULT_POISSON_MLP, batch=20)
    flat = pack_poisson_parameters(model)
    gu = torch.randn(20, 1, dtype=torch.float64)
    gl = torch.randn(20, 1, dtype=torch.float64)
    gx, gp = _recompute_backward(x, flat, gu, gl, True, True)
    ep, ex = jet.backward(flat.numpy(), x.numpy(), gu.numpy(), gl.numpy())
    np.testing.assert_allclose(gp.numpy(), ep, rtol=1e-10, atol=1e-12 * np.abs(ep).max())
    np.testing.assert_allclose(gx.numpy(), ex, rtol=1e-10, atol=1e-12 * np.abs(ex).max())


def test_linear_model_has_zero_laplacian_and_relu_is_rejected() -> None:
    model = torch.nn.Sequential(torch.nn.Linear(2, 4), torch.nn.Linear(4, 1)).double()
    _, lap = forward_laplacian(model, torch.randn(8, 2, dtype=torch.float64))
    torch.testing.assert_close(lap, torch.zeros_like(lap))
    relu = torch.nn.Sequential(torch.nn.Linear(2, 4), torch.nn.ReLU(), torch.nn.Linear(4, 1))
    with pytest.raises(TypeError, match="ReLU"):
        forward_laplacian(relu, torch.randn(3, 2))


def test_quadratic_model_has_laplacian_six() -> None:
    class Quadratic(torch.nn.Module):
        def forward(self, x):
            return (x**2).sum(dim=1, keepdim=True)

    x = torch.randn(8, 3, dtype=torch.float64)
    out, lap = mlp_second_derivative(Quadratic(), x)
    torch.testing.assert_close(out, (x**2).sum(dim=1, keepdim=True))
    torch.testing.assert_close(lap, torch.full((8, 1), 6.0, dtype=torch.float64))
    with pytest.raises(ValueError, match="batch, dimensions"):
        mlp_second_derivative(torch.nn.Identity(), torch.randn(8))


def test_residual_operator_composes_and_error_metrics_known_values() -> None:
    class Sum(torch.nn.Module):
        def forward(self, x):
            return x.sum(dim=1, keepdim=True)

    out, res = evaluate_residual(Sum(), torch.randn(4, 3), lambda o, x: gradient(o, x))
    assert out.shape == (4, 1)
    torch.testing.assert_close(res, torch.ones(4, 3))
    m = error_metrics(torch.tensor([1.0, 4.0]), torch.tensor([1.0, 2.0]))
    assert (m.max_absolute, m.max_relative, m.mean_absolute) == (2.0, 1.0, 1.0)


def test_config_and_poisson_contract() -> None:
    with pytest.raises(ValueError, match="hidden_layers"):
        MLPConfig(input_dim=2, hidden_dim=16, hidden_layers=0)
    assert (DEFAULT_POISSON_MLP.input_dim, DEFAULT_POISSON_MLP.hidden_dim) == (2, 64)
    assert (DEFAULT_POISSON_MLP.hidden_layers, DEFAULT_POISSON_MLP.activation) == (4, "tanh")
    x = torch.tensor([[0.25, 0.5], [-0.5, 0.25]], dtype=torch.float64)
    torch.testing.assert_close(manufactured_source(x), -2.0 * pi**2 * manufactured_solution(x))
    edge = torch.tensor([[-1.0, -0.4], [1.0, 0.2], [0.3, -1.0], [-0.7, 1.0]], dtype=torch.float64)
    torch.testing.assert_close(manufactured_solution(edge), torch.zeros(4, 1, dtype=torch.float64), atol=1e-15, rtol=0)
    with pytest.raises(ValueError, match=r"\[batch, 2\]"):
        manufactured_solution(torch.randn(4, 3))


def test_manufactured_solution_has_negligible_residual() -> None:
    class Exact(torch.nn.Module):
        def forward(self, x):
            return manufactured_solution(x)

    torch.manual_seed(0)
    x = torch.empty(32, 2, dtype=torch.float64).uniform_(-1.0, 1.0)
    _, residual = evaluate_poisson_residual(Exact(), x)
    torch.testing.assert_close(residual, torch.zeros_like(residual), atol=1e-12, rtol=1e-12)


def test_pack_cache_tracks_model_identity_and_in_place_updates() -> None:
    from fused_hoad.backends.fused import _packed_parameters

    with torch.no_grad():
        first = build_mlp(DEFAULT_POISSON_MLP)
        packed = _packed_parameters(first)
        assert _packed_parameters(first) is packed
        first[0].weight.mul_(2.0)
        torch.testing.assert_close(_packed_parameters(first), pack_poisson_parameters(first))
        second = build_mlp(DEFAULT_POISSON_MLP)
        torch.testing.assert_close(_packed_parameters(second), pack_poisson_parameters(second))


def test_fused_laplacian_rejects_unknown_backward_mode() -> None:
    from fused_hoad.backends.fused import BACKWARD_MODES, fused_laplacian

    assert BACKWARD_MODES[0] == "cuda" and BACKWARD_MODES[-1] == "recompute"
    with pytest.raises(ValueError, match="backward must be one of"):
        fused_laplacian(build_mlp(DEFAULT_POISSON_MLP), torch.zeros(4, 2), backward="nope")


def test_poisson_training_loop_reduces_loss_on_cpu() -> None:
    from fused_hoad.training import boundary_points, poisson_loss_fn, relative_l2_error

    torch.manual_seed(0)
    model = build_mlp(MLPConfig(input_dim=2, hidden_dim=16, hidden_layers=2))
    interior = torch.rand(256, 2) * 2 - 1
    boundary = boundary_points(64, device="cpu")
    assert torch.all(boundary.abs().max(dim=1).values == 1.0)
    loss_fn = poisson_loss_fn(forward_laplacian, model, interior, boundary)
    opt = torch.optim.Adam(model.parameters(), lr=1e-2)
    first = loss_fn().item()
    for _ in range(30):
        opt.zero_grad()
        loss = loss_fn()
        loss.backward()
        opt.step()
    assert loss.item() < 0.9 * first
    assert 0.0 < relative_l2_error(model, resolution=11) < 10.0


def test_missing_extension_error_is_actionable(monkeypatch: pytest.MonkeyPatch) -> None:
    import builtins

    from fused_hoad import _extension

    real_import = builtins.__import__

    def no_extension(name, globals=None, locals=None, fromlist=(), level=0):
        if name == "fused_hoad" and fromlist and "_C" in fromlist:
            raise ImportError("simulated missing extension")
        return real_import(name, globals, locals, fromlist, level)

    monkeypatch.setattr(builtins, "__import__", no_extension)
    monkeypatch.delitem(__import__("sys").modules, "fused_hoad._C", raising=False)
    monkeypatch.delattr(fused_hoad, "_C", raising=False)
    with pytest.raises(RuntimeError, match="pip install -e . --no-build-isolation"):
        _extension.load_extension()
    assert not _extension.extension_available()
