"""Forward-mode Laplacian in PyTorch: one forward pass, no nested autograd.

Each hidden state carries a second-order jet per point (Li et al., 2023), stacked as one
``[batch, dims + 2, width]`` tensor: row 0 the value v, rows 1..dims the input gradient J,
row dims + 1 the Laplacian L. A linear layer is then one matmul (the bias only touches the
value row) and an activation ``act`` maps the jet as

    v' = act(z_v),   J' = act'(z_v) z_J,   L' = act'(z_v) z_L + act''(z_v) sum_d z_J[d]^2.

This is the general PyTorch backend of the public API (behaviour of
/root/reference/src/fused_hoad/backends/forward_laplacian.py:28-132) and the jet the
``"recompute"`` backward differentiates; the fused kernels implement the same math.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence

import torch
from torch import Tensor, nn

# value, first and second derivative of an activation at z
Derivatives = Callable[[Tensor], tuple[Tensor, Tensor, Tensor]]


def _tanh_derivatives(z: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    a = torch.tanh(z)
    slope = 1.0 - a * a
    return a, slope, -2.0 * a * slope


def _silu_derivatives(z: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    sig = torch.sigmoid(z)
    one_minus = 1.0 - sig
    return z * sig, sig * (1.0 + z * one_minus), sig * one_minus * (2.0 + z * (1.0 - 2.0 * sig))


_DERIVATIVES: dict[type, Derivatives] = {nn.Tanh: _tanh_derivatives, nn.SiLU: _silu_derivatives}


def _affine(jet: Tensor, weight: Tensor, bias: Tensor | None) -> Tensor:
    out = torch.matmul(jet, weight.t())
    if bias is not None:
        # Derivatives of a constant vanish: only the value row gets the bias. matmul does not
        # save its output for backward, so the in-place add is autograd-safe.
        out.select(1, 0).add_(bias)
    return out


def _activate(jet: Tensor, derivatives: Derivatives) -> Tensor:
    value, grads, lap = jet[:, :1], jet[:, 1:-1], jet[:, -1:]
    f, df, d2f = derivatives(value)
    new_lap = df * lap + d2f * (grads * grads).sum(dim=1, keepdim=True)
    return torch.cat((f, df * grads, new_lap), dim=1)


def _initial_jet(coordinates: Tensor) -> Tensor:
    if coordinates.ndim != 2:
        raise ValueError("coordinates must have shape [batch, dimensions]")
    if not coordinates.is_floating_point():
        raise TypeError("coordinates must use a floating-point dtype")
    batch, dims = coordinates.shape
    eye = torch.eye(dims, dtype=coordinates.dtype, device=coordinates.device)
    return torch.cat(
        (
            coordinates.unsqueeze(1),
            eye.unsqueeze(0).expand(batch, dims, dims),
            coordinates.new_zeros(batch, 1, dims),
        ),
        dim=1,
    )


def _run(jet: Tensor, steps: Sequence) -> tuple[Tensor, Tensor]:
    for step in steps:
        jet = _affine(jet, *step) if isinstance(step, tuple) else _activate(jet, step)
    return jet[:, 0], jet[:, -1]


def _check_model(model: nn.Module) -> list[nn.Module]:
    if not isinstance(model, nn.Sequential):
        raise TypeError("forward_laplacian requires an nn.Sequential MLP")
    modules = list(model)
    for module in modules:
        if not isinstance(module, nn.Linear) and type(module) not in _DERIVATIVES:
            raise TypeError(f"unsupported module for forward_laplacian: {type(module).__name__}")
    if not modules or not isinstance(modules[-1], nn.Linear):
        raise TypeError("forward_laplacian requires the MLP to end with nn.Linear")
    if modules[-1].out_features != 1:
        raise ValueError("model output must have shape [batch, 1]")
    return modules


def forward_laplacian(model: nn.Module, coordinates: Tensor) -> tuple[Tensor, Tensor]:
    """``(u, Laplacian u)`` of a tanh/SiLU MLP, each ``[batch, 1]``, in one forward pass."""
    steps = [
        (m.weight, m.bias) if isinstance(m, nn.Linear) else _DERIVATIVES[type(m)]
        for m in _check_model(model)
    ]
    return _run(_initial_jet(coordinates), steps)


def tanh_mlp_forward_laplacian(
    linears: Sequence[tuple[Tensor, Tensor | None]], coordinates: Tensor
) -> tuple[Tensor, Tensor]:
    """Forward Laplacian of a tanh MLP given raw ``(weight, bias)`` pairs (tanh between
    consecutive pairs, none after the last)."""
    steps: list = []
    for index, pair in enumerate(linears):
        if index:
            steps.append(_tanh_derivatives)
        steps.append(pair)
    return _run(_initial_jet(coordinates), steps)
