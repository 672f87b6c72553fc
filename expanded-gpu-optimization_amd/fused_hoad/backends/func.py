"""``torch.func`` backend: the Laplacian as a sum of per-point second directional derivatives.

Registered as ``"func"``, like /root/reference/src/fused_hoad/backends/func.py:8-19, and
trainable like it (autograd reaches the weights through the ``torch.func`` transforms). Each
point's trace is formed from D forward-over-reverse products ``e_d . (H e_d)``, one per
coordinate axis, rather than from the whole D x D Hessian.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn
from torch.func import functional_call, grad, jvp, vmap


def func_laplacian(model: nn.Module, coordinates: Tensor) -> tuple[Tensor, Tensor]:
    """``(u, Laplacian u)``, both ``[batch, 1]``, of a scalar-output ``model``."""
    if coordinates.ndim != 2:
        raise ValueError("coordinates must have shape [batch, dimensions]")
    state = dict(model.named_parameters())
    state.update(model.named_buffers())
    axes = torch.eye(coordinates.shape[1], dtype=coordinates.dtype, device=coordinates.device)

    def field(point: Tensor) -> Tensor:
        return functional_call(model, state, (point.unsqueeze(0),)).reshape(())

    slope = grad(field)

    def trace(point: Tensor) -> Tensor:
        total = None
        for d in range(axes.shape[0]):
            _, curvature = jvp(slope, (point,), (axes[d],))  # H e_d
            total = curvature[d] if total is None else total + curvature[d]
        return total

    return model(coordinates), vmap(trace)(coordinates).unsqueeze(1)
