"""2-D Poisson problem on [-1, 1]^2 with manufactured solution u = sin(pi x) sin(pi y).

Behaviour of /root/reference/src/fused_hoad/problems/poisson.py:15-68.
"""

from collections.abc import Callable
from math import pi

import torch
from torch import Tensor, nn

from fused_hoad.autodiff import laplacian
from fused_hoad.residuals import evaluate_residual
from fused_hoad.specs import MLPConfig

Source = Tensor | Callable[[Tensor], Tensor]

DEFAULT_POISSON_MLP = MLPConfig(
    input_dim=2, hidden_dim=64, hidden_layers=4, output_dim=1, activation="tanh"
)


def _check(coordinates: Tensor) -> None:
    if coordinates.ndim != 2 or coordinates.shape[1] != 2:
        raise ValueError("Poisson coordinates must have shape [batch, 2]")


def manufactured_solution(coordinates: Tensor) -> Tensor:
    """``sin(pi x) sin(pi y)``, shape ``[batch, 1]``."""
    _check(coordinates)
    return torch.sin(pi * coordinates[:, 0:1]) * torch.sin(pi * coordinates[:, 1:2])


def manufactured_source(coordinates: Tensor) -> Tensor:
    """``f = Laplacian(u) = -2 pi^2 sin(pi x) sin(pi y)`` for the manufactured solution."""
    return -2.0 * pi**2 * manufactured_solution(coordinates)


def poisson_residual(output: Tensor, coordinates: Tensor, source: Source = manufactured_source) -> Tensor:
    """``Laplacian(output) - source`` by nested autograd."""
    _check(coordinates)
    if output.ndim != 2 or output.shape != (coordinates.shape[0], 1):
        raise ValueError("Poisson output must have shape [batch, 1]")
    values = source(coordinates) if callable(source) else source
    if values.shape != output.shape:
        raise ValueError("Poisson source must have shape [batch, 1]")
    return laplacian(output, coordinates) - values


def evaluate_poisson_residual(
    model: nn.Module, coordinates: Tensor, source: Source = manufactured_source
) -> tuple[Tensor, Tensor]:
    """``(model(x), Laplacian(model)(x) - f(x))``."""
    return evaluate_residual(model, coordinates, lambda out, x: poisson_residual(out, x, source))
