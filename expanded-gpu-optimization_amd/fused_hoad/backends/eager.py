"""Eager autograd backend: nested ``autograd.grad`` Laplacian, the registry's oracle."""

from torch import Tensor, nn

from fused_hoad.reference import mlp_second_derivative


def eager_laplacian(model: nn.Module, coordinates: Tensor) -> tuple[Tensor, Tensor]:
    """``(u, Laplacian u)`` with one gradient pass plus one per input dimension
    (/root/reference/src/fused_hoad/backends/eager.py:8-10)."""
    return mlp_second_derivative(model, coordinates)
