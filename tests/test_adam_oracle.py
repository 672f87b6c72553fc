"""Pins the training-step oracle (oracle/adam.py) on the CPU.

Adam is checked against torch.optim.Adam itself in float64 (the optimizer the reference's
training benchmark uses, benchmark_training.py:41) and against the closed form of the first
step; planted mistakes in a copy of the update must fail those same checks. The loss seed is
checked against torch autograd of ``(lap - f).pow(2).mean()`` (benchmark_training.py:46-48).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import adam, jet, torch_ref


def _torch_adam_trajectory(p0, grads, **kw):
    """Parameters after each torch.optim.Adam step, float64 on the CPU, given the gradients."""
    p = torch.nn.Parameter(torch.tensor(p0, dtype=torch.float64))
    opt = torch.optim.Adam([p], foreach=False, **kw)
    out = []
    for g in grads:
        p.grad = torch.tensor(g, dtype=torch.float64)
        opt.step()
        out.append(p.detach().numpy().copy())
    state = opt.state[p]
    return out, state["exp_avg"].numpy(), state["exp_avg_sq"].numpy()


@pytest.mark.parametrize(
    "kw",
    [
        dict(lr=1e-3),
        dict(lr=3e-2, betas=(0.8, 0.99), eps=1e-6),
        dict(lr=1e-3, weight_decay=0.1),
    ],
)
def test_adam_update_matches_torch_adam(kw) -> None:
    rng = np.random.default_rng(0)
    p0 = rng.normal(size=257)
    grads = [rng.normal(size=257) * 10.0 ** rng.uniform(-6, 1, size=257) for _ in range(7)]
    want, want_m, want_v = _torch_adam_trajectory(p0, grads, **kw)
    beta1, beta2 = kw.get("betas", (0.9, 0.999))
    args = dict(lr=kw["lr"], beta1=beta1, beta2=beta2, eps=kw.get("eps", 1e-8),
                weight_decay=kw.get("weight_decay", 0.0))
    p, m, v = p0, np.zeros_like(p0), np.zeros_like(p0)
    for t, (g, w) in enumerate(zip(grads, want), start=1):
        p, m, v = adam.adam_update(p, g, m, v, t, **args)
        np.testing.assert_allclose(p, w, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(m, want_m, rtol=1e-13, atol=0)
    np.testing.assert_allclose(v, want_v, rtol=1e-13, atol=0)


def _first_step_closed_form(update) -> None:
    """From zero state the bias-corrected moments are g and g^2, so p1 = p0 - lr g / (|g| + eps)."""
    rng = np.random.default_rng(1)
    p0 = rng.normal(size=64)
    g = rng.normal(size=64)
    p1, _, _ = update(p0, g, np.zeros(64), np.zeros(64), 1, lr=0.01, beta1=0.9, beta2=0.999,
                      eps=1e-8, weight_decay=0.0)
    np.testing.assert_allclose(p1, p0 - 0.01 * g / (np.abs(g) + 1e-8), rtol=1e-12, atol=1e-15)


def test_adam_first_step_closed_form() -> None:
    _first_step_closed_form(adam.adam_update)


def _no_bias_correction(p, g, m, v, t, *, lr, beta1, beta2, eps, weight_decay):
    m = beta1 * m + (1 - beta1) * g
    v = beta2 * v + (1 - beta2) * g * g
    return p - lr * m / (np.sqrt(v) + eps), m, v


def _swapped_betas(p, g, m, v, t, *, lr, beta1, beta2, eps, weight_decay):
    return adam.adam_update(p, g, m, v, t, lr=lr, beta1=beta2, beta2=beta1, eps=eps,
                            weight_decay=weight_decay)


def test_planted_missing_bias_correction_fails_the_closed_form() -> None:
    with pytest.raises(AssertionError):
        _first_step_closed_form(_no_bias_correction)


@pytest.mark.parametrize("mistake", [_no_bias_correction, _swapped_betas])
def test_planted_adam_mistakes_fail_the_torch_trajectory(mistake) -> None:
    # (the first step from zero state does not depend on the betas, so a beta mistake shows
    # only over several steps)
    rng = np.random.default_rng(2)
    p0 = rng.normal(size=33)
    grads = [rng.normal(size=33) for _ in range(3)]
    want, _, _ = _torch_adam_trajectory(p0, grads, lr=1e-3)
    p, m, v = p0, np.zeros(33), np.zeros(33)
    for t, g in enumerate(grads, start=1):
        p, m, v = mistake(p, g, m, v, t, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
                          weight_decay=0.0)
    assert not np.allclose(p, want[-1], rtol=1e-9, atol=0)


def test_poisson_seed_matches_autograd_of_the_loss() -> None:
    rng = np.random.default_rng(3)
    lap = torch.tensor(rng.normal(size=(37, 1)), requires_grad=True)
    f = torch.tensor(rng.normal(size=(37, 1)))
    loss = (lap - f).pow(2).mean()
    loss.backward()
    want_loss, want_grad = loss.item(), lap.grad.numpy().reshape(-1)
    got_loss, got_grad = adam.poisson_seed(lap.detach().numpy(), f.numpy())
    assert got_loss == pytest.approx(want_loss, rel=1e-14)
    np.testing.assert_allclose(got_grad, want_grad, rtol=1e-14, atol=0)


def test_poisson_adam_step_matches_a_torch_training_step() -> None:
    """The whole oracle step against the reference's step in float64 on the CPU: the PyTorch
    forward Laplacian of the packed buffer, the loss, autograd, torch.optim.Adam."""
    from fused_hoad.problems.poisson import manufactured_source

    flat = torch_ref.pack(torch_ref.reference_model(0)).double()
    gen = torch.Generator().manual_seed(4)
    x = (torch.rand(300, 2, generator=gen, dtype=torch.float64) * 2 - 1)
    f = manufactured_source(x)

    leaf = torch.nn.Parameter(flat.clone())
    opt = torch.optim.Adam([leaf], lr=1e-3, foreach=False)
    _, lap = torch_ref.forward_laplacian(leaf, x)
    loss = (lap - f).pow(2).mean()
    loss.backward()
    grad = leaf.grad.detach().numpy().copy()
    opt.step()

    out = adam.poisson_adam_step(flat.numpy(), x.numpy(), f.numpy(), np.zeros(jet.PARAMETER_COUNT),
                                 np.zeros(jet.PARAMETER_COUNT), 1, lr=1e-3)
    assert out["loss"] == pytest.approx(loss.item(), rel=1e-12)
    np.testing.assert_allclose(out["grad_parameters"], grad, rtol=1e-9, atol=1e-12 * np.abs(grad).max())
    np.testing.assert_allclose(out["params"], leaf.detach().numpy(), rtol=1e-12, atol=1e-14)


def test_pinn_step_with_boundary_matches_a_torch_training_step() -> None:
    """The oracle's PINN step (boundary term included) against the reference's loss of
    training.py:66-88 in float64 on the CPU: forward Laplacian on the interior, a plain MLP
    forward on the boundary, autograd, torch.optim.Adam."""
    from fused_hoad.problems.poisson import manufactured_source
    from fused_hoad.training import boundary_points

    flat = torch_ref.pack(torch_ref.reference_model(1)).double()
    gen = torch.Generator().manual_seed(5)
    x = torch.rand(200, 2, generator=gen, dtype=torch.float64) * 2 - 1
    xb = boundary_points(70, device="cpu", dtype=torch.float64, generator=gen)
    f = manufactured_source(x)

    leaf = torch.nn.Parameter(flat.clone())
    opt = torch.optim.Adam([leaf], lr=1e-3, foreach=False)
    _, lap = torch_ref.forward_laplacian(leaf, x)
    loss = (lap - f).pow(2).mean() + 100.0 * torch_ref._mlp(leaf, xb).pow(2).mean()
    loss.backward()
    grad = leaf.grad.detach().numpy().copy()
    opt.step()

    zeros = np.zeros(jet.PARAMETER_COUNT)
    out = adam.poisson_adam_step(flat.numpy(), x.numpy(), f.numpy(), zeros, zeros, 1,
                                 boundary=xb.numpy(), boundary_weight=100.0, lr=1e-3)
    assert out["loss"] == pytest.approx(loss.item(), rel=1e-12)
    np.testing.assert_allclose(out["grad_parameters"], grad, rtol=1e-9, atol=1e-12 * np.abs(grad).max())
    np.testing.assert_allclose(out["params"], leaf.detach().numpy(), rtol=1e-12, atol=1e-14)
    # the boundary term matters: without it the gradient differs
    plain = adam.poisson_adam_step(flat.numpy(), x.numpy(), f.numpy(), zeros, zeros, 1, lr=1e-3)
    assert not np.allclose(plain["grad_parameters"], grad, rtol=1e-3, atol=0)
