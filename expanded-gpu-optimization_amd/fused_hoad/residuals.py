"""Apply a residual operator to a model's output on fresh differentiable coordinates.

The operator sees ``(output, x)`` with ``x`` a leaf that requires grad, so it can take input
derivatives of the output (``fused_hoad.autodiff``). Both the model's output and the
operator's result must be ``[batch, k]`` matrices over the same points.

Public names, arguments and error messages are those of
/root/reference/src/fused_hoad/residuals.py:8-26.
"""

from __future__ import annotations

from collections.abc import Callable

from torch import Tensor, nn

from fused_hoad.autodiff import differentiable_coordinates

ResidualOperator = Callable[[Tensor, Tensor], Tensor]


def _per_point_matrix(tensor: Tensor, batch: int, message: str) -> Tensor:
    if tensor.ndim != 2 or tensor.shape[0] != batch:
        raise ValueError(message)
    return tensor


def evaluate_residual(
    model: nn.Module, coordinates: Tensor, operator: ResidualOperator
) -> tuple[Tensor, Tensor]:
    """``(model(x), operator(model(x), x))`` with ``x`` a differentiable copy of
    ``coordinates``."""
    x = differentiable_coordinates(coordinates)
    batch = x.shape[0]
    output = _per_point_matrix(model(x), batch, "model output must have shape [batch, outputs]")
    residual = _per_point_matrix(operator(output, x), batch, "residual must have shape [batch, terms]")
    return output, residual
