"""Correctness-first eager-autograd evaluation used as an oracle."""

from torch import Tensor, nn

from fused_hoad.autodiff import laplacian
from fused_hoad.residuals import evaluate_residual


def mlp_second_derivative(model: nn.Module, coordinates: Tensor) -> tuple[Tensor, Tensor]:
    """``(u, Laplacian u)`` of a scalar-output model by nested eager autograd
    (/root/reference/src/fused_hoad/reference.py:9-20)."""

    def operator(output: Tensor, x: Tensor) -> Tensor:
        if output.shape[1] != 1:
            raise ValueError("model output must have shape [batch, 1]")
        return laplacian(output, x)

    return evaluate_residual(model, coordinates, operator)
