"""Training-step helpers: whole-step graph capture and the Poisson PINN loss.

Behaviour of /root/reference/src/fused_hoad/training.py:9-88. On ROCm ``torch.cuda.CUDAGraph``
records a HIP graph.
"""

from collections.abc import Callable

import torch
from torch import Tensor


def cuda_graph_step(
    loss_fn: Callable[[], Tensor], optimizer: torch.optim.Optimizer, *, warmup: int = 3
) -> Callable[[], Tensor]:
    """Capture ``loss_fn() -> backward -> optimizer.step()`` as one graph and return a replay
    function that returns the (static) loss tensor.

    Warm up on a side stream, drop grads so backward allocates them in the graph's pool, then
    capture. The optimizer must be built with ``capturable=True``; inputs closed over by
    ``loss_fn`` are static (copy new data into them in place between replays).
    """
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            optimizer.zero_grad(set_to_none=True)
            loss_fn().backward()
            optimizer.step()
    torch.cuda.current_stream().wait_stream(side)

    graph = torch.cuda.CUDAGraph()
    optimizer.zero_grad(set_to_none=True)
    with torch.cuda.graph(graph):
        static_loss = loss_fn()
        static_loss.backward()
        optimizer.step()

    def replay() -> Tensor:
        graph.replay()
        return static_loss

    return replay


def boundary_points(count: int, *, device, dtype=torch.float32, generator=None) -> Tensor:
    """``count`` points uniform on the boundary of ``[-1, 1]^2`` (sides x=-1, x=1, y=-1, y=1)."""
    t = torch.rand(count, device=device, dtype=dtype, generator=generator) * 2 - 1
    side = torch.randint(0, 4, (count,), device=device, generator=generator)
    fixed = torch.where(side % 2 == 0, -1.0, 1.0).to(dtype)
    x_fixed = side < 2
    return torch.stack((torch.where(x_fixed, fixed, t), torch.where(x_fixed, t, fixed)), dim=1)


def relative_l2_error(model: torch.nn.Module, *, resolution: int = 101) -> float:
    """Relative L2 error of ``model`` against ``sin(pi x) sin(pi y)`` on a uniform grid."""
    from fused_hoad.problems.poisson import manufactured_solution

    reference = next(model.parameters())
    axis = torch.linspace(-1.0, 1.0, resolution, device=reference.device, dtype=reference.dtype)
    grid = torch.cartesian_prod(axis, axis)
    with torch.no_grad():
        exact = manufactured_solution(grid)
        return ((model(grid) - exact).norm() / exact.norm()).item()


def poisson_loss_fn(
    backend: Callable,
    model: torch.nn.Module,
    interior: Tensor,
    boundary: Tensor,
    *,
    boundary_weight: float = 100.0,
) -> Callable[[], Tensor]:
    """Closure for the PINN loss ``mean((Lap u - f)^2) + boundary_weight * mean(u_boundary^2)``;
    ``backend(model, interior)`` supplies ``(u, Lap u)``, the boundary term is a plain forward."""
    from fused_hoad.problems.poisson import manufactured_source

    source = manufactured_source(interior)

    def loss_fn() -> Tensor:
        _, lap = backend(model, interior)
        return (lap - source).pow(2).mean() + boundary_weight * model(boundary).pow(2).mean()

    return loss_fn
