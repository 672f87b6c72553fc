"""PyTorch restatement of the reference's CPU path for the fused-Laplacian hot path.

TEST INFRASTRUCTURE ONLY (checker and CPU baseline). Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may use it; the product
never imports it.

* ``forward_laplacian``: the PyTorch forward Laplacian the north star's forward tolerance
  (atol 1e-5 / rtol 1e-4) is stated against, /root/reference/src/fused_hoad/backends/
  forward_laplacian.py:28-132. The reference stacks (v, J, L) into one [batch, 4, 64] tensor;
  this restatement keeps the four components as separate [batch, 64] tensors, which is the
  same arithmetic (one matmul per component).
* ``forward_laplacian_stacked``: the same jet in the reference's op structure (one stacked
  [batch, 4, 64] tensor, in-place row fix-ups), timed as the CPU baseline's headline.
* ``recompute_backward``: the reference backward (autograd through the PyTorch jet),
  /root/reference/src/fused_hoad/backends/fused.py:76-101.
* ``eager_laplacian``: nested ``autograd.grad`` Laplacian, /root/reference/src/fused_hoad/
  autodiff.py:16-40 and reference.py:9-20; an algorithm independent of the jet.
* ``reference_model`` / ``pack``: the seeded model of /root/reference/src/fused_hoad/models.py:
  15-26 with /root/reference/src/fused_hoad/problems/poisson.py:15-21, packed as in
  parameters.py:55-84.
* ``poisson_source``, ``eager_train_step``: the training-step definition of
  /root/reference/benchmarks/benchmark_training.py:36-65 (loss mean((lap - f)^2), Adam).

Pinned in tests/test_oracle.py against the numpy closed forms of oracle/jet.py, float64 finite
differences and the known answers of the reference's own tests.
"""

from __future__ import annotations

from math import pi

import torch
from torch import Tensor, nn

HIDDEN_BASE = 192
HIDDEN_STRIDE = 4160
OUTPUT_BASE = 12672
PARAMETER_COUNT = 12737


def reference_model(seed: int = 0) -> nn.Sequential:
    """``torch.manual_seed(seed)`` then the 2 -> 64x4 -> 1 tanh MLP with default init."""
    torch.manual_seed(seed)
    layers: list[nn.Module] = []
    width = 2
    for _ in range(4):
        layers += [nn.Linear(width, 64), nn.Tanh()]
        width = 64
    layers.append(nn.Linear(64, 1))
    return nn.Sequential(*layers)


def pack(model: nn.Module) -> Tensor:
    """Detached packed [12737] copy of the model's parameters."""
    with torch.no_grad():
        return torch.cat(
            [t.detach().reshape(-1) for m in model if isinstance(m, nn.Linear) for t in (m.weight, m.bias)]
        )


def _blocks(flat: Tensor):
    w0 = flat[:128].view(64, 2)
    b0 = flat[128:192]
    hidden = []
    for layer in range(3):
        base = HIDDEN_BASE + layer * HIDDEN_STRIDE
        hidden.append((flat[base : base + 4096].view(64, 64), flat[base + 4096 : base + 4160]))
    return w0, b0, hidden, flat[OUTPUT_BASE : OUTPUT_BASE + 64], flat[OUTPUT_BASE + 64]


def _tanh_jet(zv: Tensor, zj0: Tensor, zj1: Tensor, zl: Tensor):
    a = torch.tanh(zv)
    s = 1.0 - a * a
    return a, s * zj0, s * zj1, s * zl + (-2.0 * a * s) * (zj0 * zj0 + zj1 * zj1)


def forward_laplacian(flat: Tensor, coords: Tensor) -> tuple[Tensor, Tensor]:
    """(u, lap), each [batch, 1], by forward-mode jet propagation (differentiable)."""
    w0, b0, hidden, w_out, b_out = _blocks(flat)
    x = coords[:, 0:1]
    y = coords[:, 1:2]
    zv = x * w0[:, 0] + y * w0[:, 1] + b0
    zj0 = w0[:, 0].expand_as(zv)
    zj1 = w0[:, 1].expand_as(zv)
    jet = _tanh_jet(zv, zj0, zj1, torch.zeros_like(zv))
    for weight, bias in hidden:
        wt = weight.t()
        jet = _tanh_jet(jet[0] @ wt + bias, jet[1] @ wt, jet[2] @ wt, jet[3] @ wt)
    u = jet[0] @ w_out.unsqueeze(1) + b_out
    lap = jet[3] @ w_out.unsqueeze(1)
    return u, lap


def forward_laplacian_stacked(flat: Tensor, coords: Tensor) -> tuple[Tensor, Tensor]:
    """(u, lap), each [batch, 1], in the reference's op structure, for timing its CPU path:
    one [batch, 4, width] jet (rows v, J0, J1, L), one matmul per layer with the bias added
    to the value row in place, and the tanh jet as ``s * z`` with the L row and the value row
    fixed up in place (/root/reference/src/fused_hoad/backends/forward_laplacian.py:52-67,
    120-132). The arithmetic is that of forward_laplacian grouped differently, so float32
    results agree to rounding."""
    w0, b0, hidden, w_out, b_out = _blocks(flat)
    batch = coords.shape[0]
    jet = coords.new_zeros(batch, 4, 2)
    jet[:, 0] = coords
    jet[:, 1, 0] = 1.0
    jet[:, 2, 1] = 1.0
    layers = [(w0, b0), *hidden, (w_out.unsqueeze(0), b_out.reshape(1))]
    for index, (weight, bias) in enumerate(layers):
        z = jet @ weight.t()
        z[:, 0].add_(bias)
        if index + 1 == len(layers):
            return z[:, 0], z[:, 3]
        a = torch.tanh(z[:, :1])
        s = 1.0 - a * a
        jet = s * z
        jet[:, 3:].add_((-2.0 * a * s) * (z[:, 1:3] * z[:, 1:3]).sum(dim=1, keepdim=True))
        jet[:, :1].copy_(a)
    raise AssertionError("unreachable")


def recompute_backward(flat: Tensor, coords: Tensor, grad_output: Tensor, grad_laplacian: Tensor):
    """(grad_parameters[12737], grad_coordinates[batch, 2]) by autograd through the jet."""
    with torch.enable_grad():
        p = flat.detach().requires_grad_(True)
        x = coords.detach().requires_grad_(True)
        u, lap = forward_laplacian(p, x)
        gp, gx = torch.autograd.grad(
            (u, lap), (p, x), (grad_output.reshape(-1, 1), grad_laplacian.reshape(-1, 1))
        )
    return gp, gx


def _mlp(flat: Tensor, x: Tensor) -> Tensor:
    w0, b0, hidden, w_out, b_out = _blocks(flat)
    h = torch.tanh(x @ w0.t() + b0)
    for weight, bias in hidden:
        h = torch.tanh(h @ weight.t() + bias)
    return h @ w_out.unsqueeze(1) + b_out


def eager_laplacian(flat: Tensor, coords: Tensor, *, create_graph: bool = False):
    """(u, lap) by nested autograd: one gradient, then one more pass per input dimension."""
    with torch.enable_grad():
        x = coords.detach().clone().requires_grad_(True)
        u = _mlp(flat, x)
        (grad,) = torch.autograd.grad(u.sum(), x, create_graph=True)
        lap = torch.zeros_like(u)
        for d in range(2):
            (second,) = torch.autograd.grad(
                grad[:, d].sum(), x, create_graph=create_graph or flat.requires_grad, retain_graph=True
            )
            lap = lap + second[:, d : d + 1]
    return u, lap


def poisson_source(coords: Tensor) -> Tensor:
    """f = -2 pi^2 sin(pi x) sin(pi y), [batch, 1]."""
    return -2.0 * pi**2 * torch.sin(pi * coords[:, 0:1]) * torch.sin(pi * coords[:, 1:2])


def eager_train_step(model: nn.Sequential, coords: Tensor, source: Tensor, optimizer) -> Tensor:
    """One reference-style step: nested-autograd Laplacian, loss mean((lap - f)^2),
    backward, optimizer step (benchmark_training.py:46-57 with the eager backend)."""
    optimizer.zero_grad(set_to_none=True)
    x = coords.detach().clone().requires_grad_(True)
    u = model(x)
    (grad,) = torch.autograd.grad(u.sum(), x, create_graph=True)
    lap = torch.zeros_like(u)
    for d in range(2):
        (second,) = torch.autograd.grad(grad[:, d].sum(), x, create_graph=True, retain_graph=True)
        lap = lap + second[:, d : d + 1]
    loss = (lap - source).pow(2).mean()
    loss.backward()
    optimizer.step()
    return loss.detach()
