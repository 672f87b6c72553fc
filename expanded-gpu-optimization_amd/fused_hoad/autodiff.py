"""Input derivatives of batched scalar fields, built from one primitive: a seeded reverse pass.

A field here is a ``[batch, 1]`` tensor computed point by point from ``[batch, dims]``
coordinates, so the reverse pass of ``field`` seeded with ``seed`` (one weight per field entry)
returns, for every point ``b``, ``seed[b] * d field[b] / d coordinates[b, :]``: seeding with
ones gives the per-point gradient, and seeding the gradient's ``d``-th column with ones (and
the other columns with zeros) gives the ``d``-th column of the per-point Hessian, of which only
the diagonal entry is kept.

Public names, arguments, results and error messages are those of
/root/reference/src/fused_hoad/autodiff.py:7-40, which the eager backend, the residual helpers
and the reference's tests use.
"""

from __future__ import annotations

import torch
from torch import Tensor


def differentiable_coordinates(coordinates: Tensor) -> Tensor:
    """A fresh leaf copy of ``[batch, dims]`` floating-point coordinates that requires grad."""
    if coordinates.ndim != 2:
        raise ValueError("coordinates must have shape [batch, dimensions]")
    if not coordinates.is_floating_point():
        raise TypeError("coordinates must use a floating-point dtype")
    return coordinates.detach().clone().requires_grad_(True)


def _seeded_pass(field: Tensor, coordinates: Tensor, seed: Tensor, *, create_graph: bool,
                 retain_graph: bool | None = None) -> Tensor:
    """Reverse pass of ``field`` seeded with ``seed``, differentiated against ``coordinates``."""
    (derivative,) = torch.autograd.grad(
        field, coordinates, grad_outputs=seed, create_graph=create_graph, retain_graph=retain_graph
    )
    return derivative


def gradient(output: Tensor, coordinates: Tensor, *, create_graph: bool = True) -> Tensor:
    """``[batch, dims]`` gradient of a ``[batch, 1]`` field at each point."""
    if output.ndim != 2 or output.shape != (coordinates.shape[0], 1):
        raise ValueError("output must have shape [batch, 1]")
    return _seeded_pass(output, coordinates, torch.ones_like(output), create_graph=create_graph)


def diagonal_hessian(output: Tensor, coordinates: Tensor) -> Tensor:
    """``[batch, dims]`` second derivatives ``d2 u / dx_d2`` at each point (the Hessian's
    diagonal; one reverse pass per dimension, no mixed partials are kept)."""
    first = gradient(output, coordinates)
    dims = first.shape[1]
    diagonal = []
    for d in range(dims):
        unit_column = torch.zeros_like(first)
        unit_column[:, d] = 1
        column = _seeded_pass(first, coordinates, unit_column, create_graph=True, retain_graph=True)
        diagonal.append(column[:, d])
    return torch.stack(diagonal, dim=1)


def laplacian(output: Tensor, coordinates: Tensor) -> Tensor:
    """``[batch, 1]`` Laplacian: the per-point sum of ``diagonal_hessian``."""
    return diagonal_hessian(output, coordinates).sum(dim=1, keepdim=True)
