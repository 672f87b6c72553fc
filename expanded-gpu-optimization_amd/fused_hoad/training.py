"""Training-step helpers: whole-step graph capture, the Poisson PINN loss, and the fused
Poisson + Adam step.

``cuda_graph_step``, ``boundary_points``, ``relative_l2_error`` and ``poisson_loss_fn`` have the
behaviour of /root/reference/src/fused_hoad/training.py:9-88 (on ROCm ``torch.cuda.CUDAGraph``
records a HIP graph). ``FusedPoissonAdam`` has no counterpart there: it runs the training step
of /root/reference/benchmarks/benchmark_training.py:41-60 as one native call.
"""

from __future__ import annotations

from collections.abc import Callable

import torch
from torch import Tensor, nn

from fused_hoad._extension import poisson_adam_step
from fused_hoad.parameters import (
    POISSON_PARAMETER_LAYOUT,
    _linear_layers,
    flatten_poisson_parameters_,
)


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

    # The graph reads and writes the optimizer's state and the tensors loss_fn closes over by
    # address: the replay function holds them, so they outlive any caller that keeps only it
    # (freed, their memory would be handed to other tensors under the replays).
    replay.owners = (loss_fn, optimizer)
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


class FusedPoissonAdam:
    """The Poisson training step with Adam as one native call of two gfx950 kernels.

    Each ``step()`` does what this does with the fused backend and ``torch.optim.Adam``
    (/root/reference/benchmarks/benchmark_training.py:41-60)::

        optimizer.zero_grad(set_to_none=True)
        _, lap = fused_laplacian(model, coordinates)
        (lap - source).pow(2).mean().backward()
        optimizer.step()

    or, given ``boundary`` points, the PINN step of
    /root/reference/benchmarks/train_poisson.py:30-45 with the loss of ``poisson_loss_fn``,
    ``mean((lap - source)^2) + boundary_weight * mean(model(boundary)^2)``. It returns the loss
    (a 0-dim device tensor, the loss before the update). The gradient kernel re-runs the forward
    jet, so no separate forward launch is needed; it forms the residual (or the boundary value)
    and its adjoint seed in registers. The reduction kernel sums the weight gradient in a fixed
    order and applies Adam to each element in the same thread. Results are bitwise
    reproducible.

    The model's parameters are moved into one packed buffer (``self.parameters``, the kernel
    ABI layout) and become views of it, so the model always holds the current weights. Adam's
    moments live in the same layout (``exp_avg``, ``exp_avg_sq``) with the step count on the
    device (``step_count``), so a step can be captured in a HIP graph (``graphed``).
    ``keep_grads`` leaves the summed gradient in ``self.grad`` and, as views of it, in every
    parameter's ``.grad``; with ``coordinates.requires_grad`` the coordinate gradient goes to
    ``self.grad_coordinates``. The coordinates, the source and the boundary points are read in
    place on every step: to train on new points, copy them into ``self.coordinates``,
    ``self.source`` and ``self.boundary``.
    """

    def __init__(
        self,
        model: nn.Module,
        coordinates: Tensor,
        source: Tensor | None = None,
        *,
        boundary: Tensor | None = None,
        boundary_weight: float = 100.0,
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 0.0,
        keep_grads: bool = True,
    ) -> None:
        from fused_hoad.problems.poisson import manufactured_source

        if not lr >= 0.0 or not eps >= 0.0 or not weight_decay >= 0.0 or not boundary_weight >= 0.0:
            raise ValueError("lr, eps, weight_decay and boundary_weight must be non-negative")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError("betas must lie in [0, 1)")
        if coordinates.ndim != 2 or coordinates.shape[1] != 2 or coordinates.shape[0] == 0:
            raise ValueError("coordinates must have shape [batch, 2] with batch > 0")
        self.model = model
        self.parameters = flatten_poisson_parameters_(model)
        if self.parameters.device != coordinates.device:
            raise ValueError("the model and the coordinates must be on the same device")
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.coordinates = coordinates.detach().contiguous()
        if source is None:
            source = manufactured_source(self.coordinates)
        if source.numel() != coordinates.shape[0]:
            raise ValueError("source must hold one value per point")
        self.source = source.detach().reshape(-1).contiguous()
        if boundary is not None and (boundary.ndim != 2 or boundary.shape[1] != 2):
            raise ValueError("boundary must have shape [count, 2]")
        self.boundary = None if boundary is None else boundary.detach().contiguous()
        self.boundary_weight = boundary_weight
        self.exp_avg = torch.zeros_like(self.parameters)
        self.exp_avg_sq = torch.zeros_like(self.parameters)
        self.step_count = torch.zeros(1, dtype=torch.float32, device=self.parameters.device)
        self.grad = torch.zeros_like(self.parameters) if keep_grads else None
        self.grad_coordinates = (
            torch.zeros_like(self.coordinates) if coordinates.requires_grad else None
        )
        self._grad_views: list[tuple[Tensor, Tensor]] = []
        if self.grad is not None:
            for layer, spec in zip(_linear_layers(model), POISSON_PARAMETER_LAYOUT, strict=True):
                self._grad_views.append(
                    (layer.weight, self.grad[spec.weight_offset : spec.bias_offset].view(
                        spec.out_features, spec.in_features))
                )
                self._grad_views.append((layer.bias, self.grad[spec.bias_offset : spec.end_offset]))

    def _launch(self) -> Tensor:
        return poisson_adam_step(
            self.coordinates,
            self.source,
            self.parameters,
            self.exp_avg,
            self.exp_avg_sq,
            self.step_count,
            lr=self.lr,
            betas=self.betas,
            eps=self.eps,
            weight_decay=self.weight_decay,
            grad_parameters=self.grad,
            grad_coordinates=self.grad_coordinates,
            boundary=self.boundary,
            boundary_weight=self.boundary_weight,
        )

    def step(self) -> Tensor:
        """One training step; returns the loss at the parameters on entry."""
        loss = self._launch()
        if self._grad_views and self._grad_views[0][0].grad is not self._grad_views[0][1]:
            for parameter, view in self._grad_views:
                parameter.grad = view
        return loss

    __call__ = step

    def graphed(self, warmup: int = 1) -> Callable[[], Tensor]:
        """Capture one step as a HIP graph and return its replay function (which returns the
        static loss tensor). ``warmup`` eager steps run first, on a side stream, and count as
        training steps, as in ``cuda_graph_step``."""
        current = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(current)
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.step()
        current.wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_loss = self._launch()
        self.step_graph = graph

        def replay() -> Tensor:
            graph.replay()
            return static_loss

        # The graph works on this trainer's buffers by address (parameters, Adam moments, step
        # count, workspace): the replay function holds the trainer so that they outlive it.
        replay.trainer = self
        return replay

    def load_optimizer_state(self, optimizer: torch.optim.Optimizer) -> None:
        """Take Adam's moments and step count from a ``torch.optim.Adam`` over this model's
        parameters (parameters the optimizer has not stepped start from zero state)."""
        steps = set()
        with torch.no_grad():
            for layer, spec in zip(_linear_layers(self.model), POISSON_PARAMETER_LAYOUT, strict=True):
                for tensor, start, end in (
                    (layer.weight, spec.weight_offset, spec.bias_offset),
                    (layer.bias, spec.bias_offset, spec.end_offset),
                ):
                    state = optimizer.state.get(tensor, {})
                    if "exp_avg" in state:
                        self.exp_avg[start:end].copy_(state["exp_avg"].reshape(-1))
                        self.exp_avg_sq[start:end].copy_(state["exp_avg_sq"].reshape(-1))
                        steps.add(float(state["step"]))
        if len(steps) > 1:
            raise ValueError("the optimizer's parameters are at different step counts")
        self.step_count.fill_(steps.pop() if steps else 0.0)
