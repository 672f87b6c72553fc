"""Pins the oracle (oracle/jet.py, oracle/torch_ref.py) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle (a dropped term, a wrong sign,
a transposed weight) fails at least one of them:
* nested eager autograd in float64: an independent algorithm for u, the Laplacian and every
  gradient (the reference's own cross-implementation test, test_backends.py:47-88);
* float64 central finite differences of u (for the Laplacian) and of the loss (for gradients);
* closed forms: zero hidden weights give a constant network with zero Laplacian and zero
  gradients for every block below the zeroed layer;
* a planted mistake in a copy of the oracle is caught.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import jet, torch_ref


def _flat(seed: int, scale: float = 1.0) -> np.ndarray:
    model = torch_ref.reference_model(seed)
    return torch_ref.pack(model).double().numpy() * scale


def _coords(batch: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).uniform(-1.0, 1.0, (batch, 2))


@pytest.mark.parametrize("seed,scale", [(0, 1.0), (1, 3.0), (2, 0.5)])
def test_forward_matches_nested_autograd_float64(seed: int, scale: float) -> None:
    flat = _flat(seed, scale)
    x = _coords(50, seed)
    u, lap = jet.forward(flat, x)
    ue, le = torch_ref.eager_laplacian(torch.tensor(flat), torch.tensor(x))
    np.testing.assert_allclose(u, ue.detach().numpy().ravel(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lap, le.detach().numpy().ravel(), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("seed,scale", [(0, 1.0), (1, 3.0)])
def test_torch_forward_laplacian_matches_numpy_jet(seed: int, scale: float) -> None:
    flat = _flat(seed, scale)
    x = _coords(40, seed + 7)
    u, lap = jet.forward(flat, x)
    ut, lt = torch_ref.forward_laplacian(torch.tensor(flat), torch.tensor(x))
    np.testing.assert_allclose(ut.numpy().ravel(), u, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(lt.numpy().ravel(), lap, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed,scale", [(0, 1.0), (1, 3.0)])
def test_stacked_forward_laplacian_matches_numpy_jet(seed: int, scale: float) -> None:
    """The reference's op structure (stacked jet, in-place row fix-ups), timed as the CPU
    baseline, against the float64 closed form; and in float32 against the per-component form
    to rounding."""
    flat = _flat(seed, scale)
    x = _coords(40, seed + 9)
    u, lap = jet.forward(flat, x)
    us, ls = torch_ref.forward_laplacian_stacked(torch.tensor(flat), torch.tensor(x))
    np.testing.assert_allclose(us.numpy().ravel(), u, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(ls.numpy().ravel(), lap, rtol=1e-12, atol=1e-12)
    f32, x32 = torch.tensor(flat, dtype=torch.float32), torch.tensor(x, dtype=torch.float32)
    for got, want in zip(torch_ref.forward_laplacian_stacked(f32, x32), torch_ref.forward_laplacian(f32, x32)):
        torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-4)


def test_stacked_forward_laplacian_planted_mistake_is_caught(monkeypatch: pytest.MonkeyPatch) -> None:
    """A dropped curvature term (the L row's in-place add) in the stacked form is caught."""
    flat = _flat(0)
    x = _coords(16, 5)
    _, lap = jet.forward(flat, x)
    real_add = torch.Tensor.add_

    def dropped(self, other, *args, **kwargs):
        return self if self.shape[1:] == (1, 64) else real_add(self, other, *args, **kwargs)

    monkeypatch.setattr(torch.Tensor, "add_", dropped)
    _, wrong = torch_ref.forward_laplacian_stacked(torch.tensor(flat), torch.tensor(x))
    monkeypatch.undo()
    assert not np.allclose(wrong.numpy().ravel(), lap, rtol=1e-6, atol=1e-8)


def _eager_gradients(flat: np.ndarray, x: np.ndarray, gu: np.ndarray, gl: np.ndarray):
    p = torch.tensor(flat, requires_grad=True)
    xt = torch.tensor(x, requires_grad=True)
    with torch.enable_grad():
        xx = xt.clone()
        u = torch_ref._mlp(p, xx)
        (grad,) = torch.autograd.grad(u.sum(), xx, create_graph=True)
        lap = 0.0
        for d in range(2):
            (second,) = torch.autograd.grad(grad[:, d].sum(), xx, create_graph=True)
            lap = lap + second[:, d]
        loss = (torch.tensor(gu) * u.ravel()).sum() + (torch.tensor(gl) * lap).sum()
        gp, gx = torch.autograd.grad(loss, (p, xt))
    return gp.numpy(), gx.numpy()


def _backward_matches(backward_fn, seed: int = 0, scale: float = 1.0) -> bool:
    flat = _flat(seed, scale)
    x = _coords(24, seed + 3)
    rng = np.random.default_rng(seed + 11)
    gu, gl = rng.standard_normal(24), rng.standard_normal(24)
    gp, gx = backward_fn(flat, x, gu, gl)
    ep, ex = _eager_gradients(flat, x, gu, gl)
    return bool(
        np.allclose(gp, ep, rtol=1e-9, atol=1e-11 * np.abs(ep).max())
        and np.allclose(gx, ex, rtol=1e-9, atol=1e-11 * np.abs(ex).max())
    )


@pytest.mark.parametrize("seed,scale", [(0, 1.0), (1, 3.0), (2, 0.5)])
def test_backward_matches_nested_autograd_float64(seed: int, scale: float) -> None:
    assert _backward_matches(jet.backward, seed, scale)


def test_torch_recompute_backward_matches_numpy_adjoint() -> None:
    flat = _flat(1, 3.0)
    x = _coords(30, 5)
    rng = np.random.default_rng(9)
    gu, gl = rng.standard_normal(30), rng.standard_normal(30)
    gp, gx = jet.backward(flat, x, gu, gl)
    tp, tx = torch_ref.recompute_backward(
        torch.tensor(flat), torch.tensor(x), torch.tensor(gu), torch.tensor(gl)
    )
    np.testing.assert_allclose(tp.numpy(), gp, rtol=1e-10, atol=1e-12 * np.abs(gp).max())
    np.testing.assert_allclose(tx.numpy(), gx, rtol=1e-10, atol=1e-12 * np.abs(gx).max())


def test_laplacian_matches_finite_differences() -> None:
    flat = _flat(0)
    x = _coords(16, 1)
    h = 1e-3
    u0, lap = jet.forward(flat, x)
    fd = np.zeros_like(u0)
    for d in range(2):
        step = np.zeros_like(x)
        step[:, d] = h
        fd += (jet.forward(flat, x + step)[0] - 2 * u0 + jet.forward(flat, x - step)[0]) / h**2
    np.testing.assert_allclose(lap, fd, rtol=0, atol=1e-5 * np.abs(lap).max())


def test_gradients_match_finite_differences() -> None:
    flat = _flat(0)
    x = _coords(12, 2)
    rng = np.random.default_rng(4)
    gu, gl = rng.standard_normal(12), rng.standard_normal(12)
    gp, gx = jet.backward(flat, x, gu, gl)

    def loss(p, xx):
        u, lap = jet.forward(p, xx)
        return float(gu @ u + gl @ lap)

    eps = 1e-6
    # one index from every block of the layout, plus random ones
    picks = [0, 1, 127, 128, 191, 192, 4287, 4288, 4351, 4352, 8511, 8512, 12607, 12608, 12671,
             12672, 12735, 12736]
    picks += list(rng.choice(jet.PARAMETER_COUNT, 30, replace=False))
    for k in picks:
        e = np.zeros_like(flat)
        e[k] = eps
        fd = (loss(flat + e, x) - loss(flat - e, x)) / (2 * eps)
        assert abs(fd - gp[k]) <= 1e-6 * max(1.0, abs(gp[k])), (k, fd, gp[k])
    for p_idx in (0, 5, 11):
        for d in range(2):
            e = np.zeros_like(x)
            e[p_idx, d] = eps
            fd = (loss(flat, x + e) - loss(flat, x - e)) / (2 * eps)
            assert abs(fd - gx[p_idx, d]) <= 1e-6 * max(1.0, abs(gx[p_idx, d]))


def test_zero_hidden_weights_give_constant_network() -> None:
    params = jet.unpack(_flat(0))
    params.w[0][:] = 0.0  # cuts every path from the inputs through hidden layer 1
    flat = jet.pack(params)
    x = _coords(20, 3)
    u, lap = jet.forward(flat, x)
    expected_u = np.tanh(params.w[2] @ np.tanh(params.w[1] @ np.tanh(params.b[0]) + params.b[1]) + params.b[2])
    assert np.all(lap == 0.0)
    np.testing.assert_allclose(u, expected_u @ params.w_out + params.b_out, rtol=1e-14)
    rng = np.random.default_rng(0)
    gp, gx = jet.backward(flat, x, rng.standard_normal(20), rng.standard_normal(20))
    grads = jet.unpack(gp)
    assert np.all(grads.w0 == 0.0) and np.all(grads.b0 == 0.0) and np.all(gx == 0.0)


def test_planted_mistake_is_caught(monkeypatch: pytest.MonkeyPatch) -> None:
    """Drop the q s3 curvature term from the tanh adjoint: the autograd check must fail."""
    real = jet.tanh_jet_adjoint

    def wrong(z, hbar):
        zv, zj0, zj1, zl = z
        vb, j0b, j1b, lb = hbar
        a = np.tanh(zv)
        s = 1.0 - a * a
        s2 = -2.0 * a * s
        zvb = vb * s + (j0b * zj0 + j1b * zj1) * s2 + lb * (zl * s2)
        return zvb, j0b * s + 2.0 * lb * s2 * zj0, j1b * s + 2.0 * lb * s2 * zj1, lb * s

    assert _backward_matches(jet.backward)
    monkeypatch.setattr(jet, "tanh_jet_adjoint", wrong)
    assert not _backward_matches(jet.backward)
    monkeypatch.setattr(jet, "tanh_jet_adjoint", real)


def test_planted_transpose_is_caught(monkeypatch: pytest.MonkeyPatch) -> None:
    """Use W instead of W^T for hbar: the autograd check must fail."""
    original = jet.backward

    def transposed_backward(flat, coords, gu, gl):
        p = jet.unpack(flat)
        p.w = [w.T.copy() for w in p.w]
        gp, gx = original(jet.pack(p), coords, gu, gl)
        return gp, gx

    assert not _backward_matches(transposed_backward)


def test_pack_unpack_round_trip_and_offsets() -> None:
    flat = np.arange(jet.PARAMETER_COUNT, dtype=np.float64)
    params = jet.unpack(flat)
    assert params.w0[63, 1] == 127 and params.b0[0] == 128 and params.w[0][0, 0] == 192
    assert params.b[0][0] == 4288 and params.w[1][0, 0] == 4352 and params.b[2][63] == 12671
    assert params.w_out[0] == 12672 and params.b_out == 12736
    np.testing.assert_array_equal(jet.pack(params), flat)


# ---- the CPU training-step baseline: poisson_source and eager_train_step ----


def test_poisson_source_is_the_laplacian_of_the_manufactured_solution() -> None:
    """f = -2 pi^2 sin(pi x) sin(pi y) is pinned by known values and by a float64 five-point
    finite-difference Laplacian of u* = sin(pi x) sin(pi y) (truncation error
    h^2 / 12 * 2 pi^4 |u*| < 2e-5 at h = 1e-3), which a wrong sign or factor fails."""
    pi2 = np.pi**2
    known = torch.tensor([[0.5, 0.5], [-0.5, 0.5], [0.5, -0.5], [0.0, 0.3], [0.7, 1.0], [-1.0, -1.0]],
                         dtype=torch.float64)
    np.testing.assert_allclose(torch_ref.poisson_source(known).numpy().ravel(),
                               [-2 * pi2, 2 * pi2, 2 * pi2, 0.0, 0.0, 0.0], rtol=1e-15, atol=1e-13)

    def solution(p):
        return np.sin(np.pi * p[:, 0]) * np.sin(np.pi * p[:, 1])

    def laplacian_fd(p, h=1e-3):
        total = -4.0 * solution(p)
        for d in range(2):
            step = np.zeros_like(p)
            step[:, d] = h
            total += solution(p + step) + solution(p - step)
        return total / h**2

    x = _coords(200, 21)
    got = torch_ref.poisson_source(torch.tensor(x)).numpy().ravel()
    assert torch_ref.poisson_source(torch.tensor(x)).shape == (200, 1)
    np.testing.assert_allclose(got, laplacian_fd(x), rtol=0, atol=5e-5)
    # planted mistakes (sign, pi instead of pi^2) fail the same check
    assert not np.allclose(-got, laplacian_fd(x), rtol=0, atol=5e-5)
    assert not np.allclose(got / np.pi, laplacian_fd(x), rtol=0, atol=5e-5)


def _eager_step_matches_the_oracle(step_fn=None) -> bool:
    """One eager_train_step in float64 (Adam lr 1e-3 from zero state) against
    oracle/adam.poisson_adam_step: the loss, the 12,737 gradients and the updated parameters.
    Returns False on a mismatch or when the step cannot run."""
    from oracle import adam

    model = torch_ref.reference_model(0).double()
    x = torch.tensor(_coords(256, 22))
    source = torch_ref.poisson_source(x)
    p0 = torch_ref.pack(model).numpy().copy()
    optimizer = torch.optim.Adam(model.parameters(), lr=1e-3)
    try:
        loss = (step_fn or torch_ref.eager_train_step)(model, x, source, optimizer)
    except RuntimeError:
        return False
    # b_out does not reach the Laplacian, so autograd leaves its .grad unset (the oracle: 0)
    grads = torch.cat([(t.grad if t.grad is not None else torch.zeros_like(t)).reshape(-1)
                       for m in model if isinstance(m, torch.nn.Linear) for t in (m.weight, m.bias)]).numpy()
    want = adam.poisson_adam_step(p0, x.numpy(), source.numpy().ravel(), np.zeros_like(p0),
                                  np.zeros_like(p0), 1)
    return bool(
        abs(float(loss) - want["loss"]) <= 1e-12 * abs(want["loss"])
        and np.allclose(grads, want["grad_parameters"], rtol=0, atol=1e-11 * np.abs(want["grad_parameters"]).max())
        and np.allclose(torch_ref.pack(model).numpy(), want["params"], rtol=0, atol=1e-13)
    )


def test_eager_train_step_matches_the_float64_oracle_step() -> None:
    assert _eager_step_matches_the_oracle()


def test_eager_train_step_planted_mistakes_are_caught(monkeypatch: pytest.MonkeyPatch) -> None:
    """Two mistakes planted in the step's nested autograd: dropping create_graph from the
    second-derivative passes (the loss no longer reaches the weights) and dropping the y
    second derivative from the Laplacian. The oracle-step check must reject both."""
    real_grad = torch.autograd.grad

    def planted(mistake):
        calls = []

        def grad(outputs, inputs, *args, **kwargs):
            calls.append(None)
            nested = len(calls) > 1  # calls 2 and 3 are the second derivatives (d = 0, 1)
            if mistake == "create_graph" and nested:
                kwargs["create_graph"] = False
            result = real_grad(outputs, inputs, *args, **kwargs)
            if mistake == "y_term" and len(calls) == 3:
                result = tuple(r * 0.0 for r in result)
            return result

        return grad

    for mistake in ("create_graph", "y_term"):
        monkeypatch.setattr(torch.autograd, "grad", planted(mistake))
        assert not _eager_step_matches_the_oracle(), mistake
        monkeypatch.setattr(torch.autograd, "grad", real_grad)
    assert _eager_step_matches_the_oracle()
