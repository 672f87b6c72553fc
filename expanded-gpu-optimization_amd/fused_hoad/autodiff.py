"""Higher-order autodiff operators on batched scalar fields (nested ``autograd.grad``).

Behaviour of /root/reference/src/fused_hoad/autodiff.py:7-40.
"""

import torch
from torch import Tensor


def differentiable_coordinates(coordinates: Tensor) -> Tensor:
    """Validate ``[batch, dims]`` floating coordinates and return a fresh differentiable leaf."""
    if coordinates.ndim != 2:
        raise ValueError("coordinates must have shape [batch, dimensions]")
    if not coordinates.is_floating_point():
        raise TypeError("coordinates must use a floating-point dtype")
    return coordinates.detach().clone().requires_grad_(True)


def gradient(output: Tensor, coordinates: Tensor, *, create_graph: bool = True) -> Tensor:
    """Per-sample input gradient ``[batch, dims]`` of a ``[batch, 1]`` field."""
    if output.ndim != 2 or output.shape != (coordinates.shape[0], 1):
        raise ValueError("output must have shape [batch, 1]")
    (grad,) = torch.autograd.grad(output.sum(), coordinates, create_graph=create_graph)
    return grad


def diagonal_hessian(output: Tensor, coordinates: Tensor) -> Tensor:
    """``[batch, dims]`` diagonal of the per-sample input Hessian (no mixed partials)."""
    first = gradient(output, coordinates)
    columns = []
    for d in range(coordinates.shape[1]):
        (second,) = torch.autograd.grad(
            first[:, d].sum(), coordinates, create_graph=True, retain_graph=True
        )
        columns.append(second[:, d])
    return torch.stack(columns, dim=1)


def laplacian(output: Tensor, coordinates: Tensor) -> Tensor:
    """``[batch, 1]`` Laplacian of a batched scalar field."""
    return diagonal_hessian(output, coordinates).sum(dim=1, keepdim=True)
