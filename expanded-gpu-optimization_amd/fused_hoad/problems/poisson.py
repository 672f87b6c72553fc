"""The 2-D Poisson problem the fused path trains on: Laplacian(u) = f on [-1, 1]^2, with the
manufactured solution u* = sin(pi x) sin(pi y), so f = -2 pi^2 u*.

Public names, defaults and error messages are those of
/root/reference/src/fused_hoad/problems/poisson.py:15-68 (the default MLP of the fused kernels,
the solution and source used by every benchmark, the eager-autograd residual).
"""

from __future__ import annotations

from collections.abc import Callable
from functools import partial
from math import pi

import torch
from torch import Tensor, nn

from fused_hoad.autodiff import laplacian
from fused_hoad.residuals import evaluate_residual
from fused_hoad.specs import MLPConfig

Source = Tensor | Callable[[Tensor], Tensor]

# The fixed network of the fused kernels: 2 -> 64 -> 64 -> 64 -> 64 -> 1, tanh.
DEFAULT_POISSON_MLP = MLPConfig(
    input_dim=2, hidden_dim=64, hidden_layers=4, output_dim=1, activation="tanh"
)


def _columns(coordinates: Tensor) -> tuple[Tensor, Tensor]:
    """The x and y columns, each ``[batch, 1]``, of ``[batch, 2]`` coordinates."""
    if coordinates.ndim != 2 or coordinates.shape[1] != 2:
        raise ValueError("Poisson coordinates must have shape [batch, 2]")
    return coordinates[:, 0:1], coordinates[:, 1:2]


def manufactured_solution(coordinates: Tensor) -> Tensor:
    """``u* = sin(pi x) sin(pi y)``, ``[batch, 1]``; zero on the boundary of the square."""
    x, y = _columns(coordinates)
    return torch.sin(pi * x) * torch.sin(pi * y)


def manufactured_source(coordinates: Tensor) -> Tensor:
    """``f = Laplacian(u*) = -2 pi^2 u*``, ``[batch, 1]``."""
    return -2.0 * pi**2 * manufactured_solution(coordinates)


def poisson_residual(output: Tensor, coordinates: Tensor, source: Source = manufactured_source) -> Tensor:
    """``Laplacian(output) - f`` at each point, by nested autograd. ``source`` is the ``[batch,
    1]`` values of f or a function of the coordinates that returns them."""
    _columns(coordinates)
    if output.ndim != 2 or output.shape != (coordinates.shape[0], 1):
        raise ValueError("Poisson output must have shape [batch, 1]")
    f = source(coordinates) if callable(source) else source
    if f.shape != output.shape:
        raise ValueError("Poisson source must have shape [batch, 1]")
    return laplacian(output, coordinates) - f


def evaluate_poisson_residual(
    model: nn.Module, coordinates: Tensor, source: Source = manufactured_source
) -> tuple[Tensor, Tensor]:
    """``(model(x), Laplacian(model)(x) - f(x))`` on a differentiable copy of the coordinates."""
    return evaluate_residual(model, coordinates, partial(poisson_residual, source=source))
