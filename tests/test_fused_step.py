"""The fused Poisson + Adam training step (fhoad_poisson_adam_step / FusedPoissonAdam).

Checked against the float64 oracle (oracle/adam.py: jet forward/backward + Adam), against the
reference's own step on the same kernels (fused forward, autograd of the loss, fused backward,
torch.optim.Adam; benchmark_training.py:41-60), for bitwise determinism across runs and grid
sizes, and for HIP-graph replay.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from conftest import assert_scaled_close
from gpu_helpers import announce, coordinates, knobs, require_gpu_extension, to_numpy64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _extension():
    return require_gpu_extension()


def _model(seed: int = 0):
    from fused_hoad import DEFAULT_POISSON_MLP, build_mlp

    torch.manual_seed(seed)
    return build_mlp(DEFAULT_POISSON_MLP).cuda()


def _blocks():
    from fused_hoad.parameters import POISSON_PARAMETER_LAYOUT

    for spec in POISSON_PARAMETER_LAYOUT:
        yield f"{spec.name}.weight", spec.weight_offset, spec.bias_offset
        yield f"{spec.name}.bias", spec.bias_offset, spec.end_offset


@pytest.mark.parametrize("batch", [1, 63, 1000, 4096, 20000, 65536])
def test_one_step_matches_the_oracle(batch: int) -> None:
    """Loss, all 10 gradient blocks, the coordinate gradient and the Adam update of one step
    against the float64 oracle. 65,536 is BASELINE config 3 (whole rounds of 64-point tiles on
    every slot, coordinates requiring grad), the reference's per-block backward check at that
    size being /root/reference/tests/test_fused.py:194-218."""
    announce(f"fused Poisson+Adam step vs float64 oracle, batch={batch}")
    from oracle import adam
    from fused_hoad.training import FusedPoissonAdam

    model = _model()
    x = coordinates(batch, seed=5).requires_grad_(True)
    trainer = FusedPoissonAdam(model, x, lr=1e-3)
    p0 = to_numpy64(trainer.parameters)
    f = to_numpy64(trainer.source)
    loss = trainer.step()
    torch.cuda.synchronize()

    want = adam.poisson_adam_step(p0, to_numpy64(x), f, np.zeros_like(p0), np.zeros_like(p0), 1)
    assert float(loss) == pytest.approx(want["loss"], rel=2e-5)
    got_grad = to_numpy64(trainer.grad)
    for name, start, end in _blocks():
        assert_scaled_close(got_grad[start:end], want["grad_parameters"][start:end], 1e-4, name)
    assert_scaled_close(to_numpy64(trainer.grad_coordinates), want["grad_coordinates"], 1e-4, "coords")
    assert float(trainer.step_count) == 1.0

    # The update, given the kernel's own gradient: Adam in float64 from the same state.
    p1, m1, v1 = adam.adam_update(p0, got_grad, np.zeros_like(p0), np.zeros_like(p0), 1)
    np.testing.assert_allclose(to_numpy64(trainer.exp_avg), m1, rtol=1e-6, atol=1e-30)
    np.testing.assert_allclose(to_numpy64(trainer.exp_avg_sq), v1, rtol=1e-6, atol=1e-38)
    np.testing.assert_allclose(to_numpy64(trainer.parameters), p1, rtol=0, atol=2e-7 * np.abs(p0).max() + 1e-9)
    # the model holds the updated weights (views of the packed buffer)
    assert torch.equal(model[0].weight.reshape(-1), trainer.parameters[:128])


def test_several_steps_match_the_float64_oracle_with_weight_decay() -> None:
    announce("fused Poisson+Adam, 5 steps with weight decay vs float64 oracle, batch=3000")
    from oracle import adam
    from fused_hoad.training import FusedPoissonAdam

    model = _model(3)
    x = coordinates(3000, seed=6)
    kw = dict(lr=2e-3, betas=(0.85, 0.995), eps=1e-7, weight_decay=0.01)
    trainer = FusedPoissonAdam(model, x, **kw)
    p = to_numpy64(trainer.parameters)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for t in range(1, 6):
        loss = trainer.step()
        grad = to_numpy64(trainer.grad)  # the kernel's gradient at p, checked against the oracle
        want = adam.poisson_adam_step(p, to_numpy64(x), to_numpy64(trainer.source), m, v, t,
                                      lr=kw["lr"], beta1=kw["betas"][0], beta2=kw["betas"][1],
                                      eps=kw["eps"], weight_decay=kw["weight_decay"])
        assert float(loss) == pytest.approx(want["loss"], rel=2e-5)
        for name, start, end in _blocks():
            assert_scaled_close(grad[start:end], want["grad_parameters"][start:end], 1e-4, f"step {t} {name}")
        p, m, v = adam.adam_update(p, grad, m, v, t, lr=kw["lr"], beta1=kw["betas"][0],
                                   beta2=kw["betas"][1], eps=kw["eps"], weight_decay=kw["weight_decay"])
        got = to_numpy64(trainer.parameters)
        np.testing.assert_allclose(got, p, rtol=0, atol=1e-6 * np.abs(p).max())
        p = got  # continue from the kernel's own float32 state
        m, v = to_numpy64(trainer.exp_avg), to_numpy64(trainer.exp_avg_sq)


def test_matches_the_reference_training_step() -> None:
    """20 steps against the reference's step on the same kernels (fused forward, autograd of
    the loss, fused backward, torch.optim.Adam): loss curve within rtol 1e-3 (the reference's
    own loss-curve tolerance, test_fused.py:150) and weights close."""
    announce("FusedPoissonAdam vs fused_laplacian + autograd + torch Adam, 20 steps, batch=8192")
    from fused_hoad import manufactured_source
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.training import FusedPoissonAdam

    x = coordinates(8192, seed=7)
    source = manufactured_source(x)
    ref_model = _model()
    optimizer = torch.optim.Adam(ref_model.parameters(), lr=1e-3)
    ref_losses = []
    for _ in range(20):
        optimizer.zero_grad(set_to_none=True)
        _, lap = fused_laplacian(ref_model, x)
        loss = (lap - source).pow(2).mean()
        loss.backward()
        optimizer.step()
        ref_losses.append(loss.item())

    model = _model()
    trainer = FusedPoissonAdam(model, x, source, lr=1e-3)
    losses = [trainer.step().item() for _ in range(20)]
    np.testing.assert_allclose(losses, ref_losses, rtol=1e-3)
    for a, b in zip(model.parameters(), ref_model.parameters()):
        torch.testing.assert_close(a, b, rtol=0, atol=2e-5)


def test_step_is_bitwise_deterministic_and_grid_independent() -> None:
    announce("FusedPoissonAdam determinism: 2 runs + FUSED_HOAD_BWD_BLOCKS=7, batch=70000")
    from fused_hoad.training import FusedPoissonAdam

    x = coordinates(70000, seed=8)

    def run():
        trainer = FusedPoissonAdam(_model(), x)
        losses = torch.stack([trainer.step() for _ in range(3)])
        torch.cuda.synchronize()
        return losses, trainer.parameters.clone(), trainer.grad.clone(), trainer.exp_avg_sq.clone()

    first = run()
    second = run()
    os.environ["FUSED_HOAD_BWD_BLOCKS"] = "7"
    try:
        capped = run()
    finally:
        del os.environ["FUSED_HOAD_BWD_BLOCKS"]
    for a, b, c in zip(first, second, capped):
        assert torch.equal(a, b) and torch.equal(a, c)


def test_loss_equals_the_fused_forward_loss() -> None:
    announce("fused step loss vs (fused forward lap - f)^2 mean, batch=65536")
    from fused_hoad import fused_forward_laplacian
    from fused_hoad.training import FusedPoissonAdam

    model = _model()
    x = coordinates(65536, seed=9)
    trainer = FusedPoissonAdam(model, x)
    _, lap = fused_forward_laplacian(x, trainer.parameters)
    want = (lap.reshape(-1) - trainer.source).double().pow(2).mean().item()
    got = trainer.step().item()
    assert got == pytest.approx(want, rel=1e-5)


def test_graph_replay_matches_eager_steps() -> None:
    announce("FusedPoissonAdam graphed replay vs eager twin, 4 replays, batch=5000")
    from fused_hoad.training import FusedPoissonAdam

    x = coordinates(5000, seed=10)
    eager = FusedPoissonAdam(_model(), x)
    graphed = FusedPoissonAdam(_model(), x)
    replay = graphed.graphed(warmup=1)
    eager.step()  # the warmup step
    for i in range(4):
        loss = replay()
        want = eager.step()
        torch.cuda.synchronize()
        assert torch.equal(loss, want), f"replay {i}"
        assert torch.equal(graphed.parameters, eager.parameters), f"replay {i}"
        assert torch.equal(graphed.step_count, eager.step_count)
        torch.zeros(1000, device="cuda").sum().item()  # unrelated eager work between replays


def test_load_optimizer_state_continues_a_torch_adam_run() -> None:
    announce("FusedPoissonAdam continuing from torch Adam state, batch=4096")
    from fused_hoad import manufactured_source
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.training import FusedPoissonAdam

    x = coordinates(4096, seed=11)
    source = manufactured_source(x)

    def torch_step(model, optimizer):
        optimizer.zero_grad(set_to_none=True)
        _, lap = fused_laplacian(model, x)
        (lap - source).pow(2).mean().backward()
        optimizer.step()

    model = _model()
    optimizer = torch.optim.Adam(model.parameters(), lr=1e-3)
    for _ in range(3):
        torch_step(model, optimizer)
    twin = _model()
    twin.load_state_dict(model.state_dict())
    twin_optimizer = torch.optim.Adam(twin.parameters(), lr=1e-3)
    twin_optimizer.load_state_dict(optimizer.state_dict())

    trainer = FusedPoissonAdam(model, x, source)
    trainer.load_optimizer_state(optimizer)
    assert float(trainer.step_count) == 3.0
    trainer.step()
    torch_step(twin, twin_optimizer)
    for a, b in zip(model.parameters(), twin.parameters()):
        torch.testing.assert_close(a, b, rtol=0, atol=1e-6)


def test_flattened_model_feeds_the_forward_without_a_stale_copy() -> None:
    announce("flattened parameters: no-grad fused_laplacian sees each fused update")
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.training import FusedPoissonAdam

    model = _model()
    x = coordinates(2048, seed=12)
    trainer = FusedPoissonAdam(model, x)
    with torch.no_grad():
        _, before = fused_laplacian(model, x)
        trainer.step()
        _, after = fused_laplacian(model, x)
    from fused_hoad import fused_forward_laplacian, pack_poisson_parameters

    _, want = fused_forward_laplacian(x, pack_poisson_parameters(model))
    assert not torch.equal(before, after)
    assert torch.equal(after, want)
    # parameters' .grad are views of the trainer's summed gradient
    assert model[0].weight.grad.data_ptr() == trainer.grad.data_ptr()


def test_argument_errors() -> None:
    announce("fused step argument errors")
    from fused_hoad import _C

    x = coordinates(10)
    p = torch.zeros(12737, device="cuda")
    f = torch.zeros(10, device="cuda")
    step = torch.zeros(1, device="cuda")
    with pytest.raises(RuntimeError, match="source must have 10 values"):
        _C.poisson_adam_step(x, f[:9], p, p.clone(), p.clone(), step, 1e-3, 0.9, 0.999, 1e-8, 0.0)
    with pytest.raises(RuntimeError, match="exp_avg must have 12737 values"):
        _C.poisson_adam_step(x, f, p, p[:5], p.clone(), step, 1e-3, 0.9, 0.999, 1e-8, 0.0)
    with pytest.raises(RuntimeError, match="at least one point"):
        _C.poisson_adam_step(x[:0], f[:0], p, p.clone(), p.clone(), step, 1e-3, 0.9, 0.999, 1e-8, 0.0)
    with pytest.raises(RuntimeError, match="betas"):
        _C.poisson_adam_step(x, f, p, p.clone(), p.clone(), step, 1e-3, 1.5, 0.999, 1e-8, 0.0)


def _boundary(count: int, seed: int):
    from fused_hoad.training import boundary_points

    return boundary_points(count, device="cpu", generator=torch.Generator().manual_seed(seed)).cuda()


@pytest.mark.parametrize(
    "batch,nb",
    [(1000, 100), (100, 1), (100, 63), (64, 64), (100, 65), (12000, 288), (12000, 289), (20000, 1024),
     (65537, 1025)],
)
def test_pinn_step_with_boundary_matches_the_oracle(batch: int, nb: int) -> None:
    announce(f"fused PINN+Adam step (boundary term) vs float64 oracle, batch={batch}, boundary={nb}")
    from oracle import adam
    from fused_hoad.training import FusedPoissonAdam

    model = _model(2)
    x = coordinates(batch, seed=14)
    xb = _boundary(nb, 14)
    trainer = FusedPoissonAdam(model, x, boundary=xb, boundary_weight=100.0, lr=1e-3)
    p0 = to_numpy64(trainer.parameters)
    loss = trainer.step()
    torch.cuda.synchronize()
    want = adam.poisson_adam_step(p0, to_numpy64(x), to_numpy64(trainer.source), np.zeros_like(p0),
                                  np.zeros_like(p0), 1, boundary=to_numpy64(xb), boundary_weight=100.0)
    assert float(loss) == pytest.approx(want["loss"], rel=2e-5)
    got_grad = to_numpy64(trainer.grad)
    for name, start, end in _blocks():
        assert_scaled_close(got_grad[start:end], want["grad_parameters"][start:end], 1e-4, name)
    p1, _, _ = adam.adam_update(p0, got_grad, np.zeros_like(p0), np.zeros_like(p0), 1)
    np.testing.assert_allclose(to_numpy64(trainer.parameters), p1, rtol=0, atol=2e-7 * np.abs(p0).max() + 1e-9)


def test_pinn_step_matches_the_reference_pinn_loss_path() -> None:
    """20 PINN steps against the reference's poisson_loss_fn (training.py:66-88) on the fused
    backend with torch.optim.Adam, as train_poisson.py runs it: loss curve within rtol 1e-3."""
    announce("FusedPoissonAdam(boundary) vs poisson_loss_fn(fused_cuda) + torch Adam, 20 steps")
    from fused_hoad import get_backend
    from fused_hoad.training import FusedPoissonAdam, poisson_loss_fn

    x = coordinates(16384, seed=15)
    xb = _boundary(1024, 15)
    ref_model = _model()
    optimizer = torch.optim.Adam(ref_model.parameters(), lr=1e-3)
    loss_fn = poisson_loss_fn(get_backend("fused_cuda"), ref_model, x, xb)
    ref_losses = []
    for _ in range(20):
        optimizer.zero_grad(set_to_none=True)
        loss = loss_fn()
        loss.backward()
        optimizer.step()
        ref_losses.append(loss.item())

    model = _model()
    trainer = FusedPoissonAdam(model, x, boundary=xb, boundary_weight=100.0, lr=1e-3)
    losses = [trainer.step().item() for _ in range(20)]
    np.testing.assert_allclose(losses, ref_losses, rtol=1e-3)
    for a, b in zip(model.parameters(), ref_model.parameters()):
        torch.testing.assert_close(a, b, rtol=0, atol=2e-5)


def test_pinn_step_is_bitwise_deterministic_and_grid_independent() -> None:
    announce("FusedPoissonAdam(boundary) determinism: 2 runs + FUSED_HOAD_BWD_BLOCKS=5")
    from fused_hoad.training import FusedPoissonAdam

    x = coordinates(16384, seed=16)
    xb = _boundary(1024, 16)

    def run():
        trainer = FusedPoissonAdam(_model(), x, boundary=xb)
        losses = torch.stack([trainer.step() for _ in range(3)])
        torch.cuda.synchronize()
        return losses, trainer.parameters.clone(), trainer.grad.clone()

    first = run()
    second = run()
    os.environ["FUSED_HOAD_BWD_BLOCKS"] = "5"
    try:
        capped = run()
    finally:
        del os.environ["FUSED_HOAD_BWD_BLOCKS"]
    for a, b, c in zip(first, second, capped):
        assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("batch,nb", [(1000, 100), (4096, 0), (12000, 288)])
def test_split_gradient_kernel_agrees_with_the_tiled_one(batch: int, nb: int) -> None:
    """Small batches run backward_split_kernel; forced either way, the two gradient kernels
    give the same loss and gradient up to rounding (1e-5 of each block's scale)."""
    announce(f"fused step, split vs tiled gradient kernel, batch={batch}, boundary={nb}")
    from fused_hoad.training import FusedPoissonAdam

    x = coordinates(batch, seed=17)
    xb = _boundary(nb, 17) if nb else None
    results = []
    for split in ("1", "0"):
        trainer = FusedPoissonAdam(_model(3), x, boundary=xb)
        with knobs(FUSED_HOAD_BWD_SPLIT=split):
            loss = trainer.step()
        torch.cuda.synchronize()
        results.append((float(loss), to_numpy64(trainer.grad)))
    (loss_s, grad_s), (loss_t, grad_t) = results
    assert loss_s == pytest.approx(loss_t, rel=1e-6)
    for name, start, end in _blocks():
        assert_scaled_close(grad_s[start:end], grad_t[start:end], 1e-5, name)
