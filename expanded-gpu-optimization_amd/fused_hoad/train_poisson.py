"""Train the 2-D Poisson PINN end to end and report wall time, final loss, relative L2 error
and time to a target error, per backend.

Behaviour of /root/reference/benchmarks/train_poisson.py:
* 5000 Adam steps (lr 1e-3) on 16K interior and 1K boundary points drawn from a seeded
  device generator;
* the loss `mean((Lap u - f)^2) + 100 mean(u_boundary^2)`;
* relative L2 against the analytic solution every `--eval-every` steps with the clock paused;
* the first evaluation below `--target` gives the time to target.

Backends are the reference's registry names that are trainable here (`eager`,
`forward_laplacian`, `fused_cuda`, `fused_cuda_bwd_v1`, `fused_cuda_recompute`), all stepped
through autograd and torch.optim.Adam. `fused_step` is this build's fused training step
(`FusedPoissonAdam`: loss, gradients and Adam in two kernels).

    python -m fused_hoad.train_poisson --backends fused_step fused_cuda --seeds 0 1 2
"""

from __future__ import annotations

import argparse
import contextlib
import hashlib
import statistics
import time
from collections.abc import Callable, Iterator

import torch

from fused_hoad import BACKENDS, DEFAULT_POISSON_MLP, build_mlp, get_backend
from fused_hoad.training import (
    FusedPoissonAdam,
    boundary_points,
    cuda_graph_step,
    poisson_loss_fn,
    relative_l2_error,
)

FUSED_STEP = "fused_step"
_TRAINABLE = ("eager", "forward_laplacian", "fused_cuda", "fused_cuda_bwd_v1", "fused_cuda_recompute")


class _TrainingClock:
    """Wall time spent training: starts at construction (after a device sync) and leaves out
    what runs inside ``paused()``, which yields the training seconds so far."""

    def __init__(self) -> None:
        torch.cuda.synchronize()
        self.seconds = 0.0
        self._resumed = time.perf_counter()

    @contextlib.contextmanager
    def paused(self) -> Iterator[float]:
        torch.cuda.synchronize()
        self.seconds += time.perf_counter() - self._resumed
        try:
            yield self.seconds
        finally:
            self._resumed = time.perf_counter()


def _stepper(name: str, model: torch.nn.Module, interior: torch.Tensor, boundary: torch.Tensor,
             lr: float, graph: bool) -> tuple[Callable[[], torch.Tensor], int]:
    """One training step of backend `name` (optionally replayed from a captured HIP graph) and
    the number of steps already taken while building it: a captured step's warmup iterations
    update the model like any other (1 for the fused step, 3 for ``cuda_graph_step``)."""
    if name == FUSED_STEP:
        trainer = FusedPoissonAdam(model, interior, boundary=boundary, lr=lr)
        return (trainer.graphed(warmup=1), 1) if graph else (trainer.step, 0)
    optimizer = torch.optim.Adam(model.parameters(), lr=lr, capturable=graph)
    loss_fn = poisson_loss_fn(get_backend(name), model, interior, boundary)
    if graph:
        return cuda_graph_step(loss_fn, optimizer), 3

    def eager_step() -> torch.Tensor:
        optimizer.zero_grad(set_to_none=True)
        loss = loss_fn()
        loss.backward()
        optimizer.step()
        return loss

    return eager_step, 0


def _weights_digest(model: torch.nn.Module) -> str:
    """First 12 hex digits of the SHA-256 of the parameters' float32 bytes in model order."""
    flat = torch.cat([p.detach().reshape(-1) for p in model.parameters()]).cpu()
    return hashlib.sha256(flat.numpy().tobytes()).hexdigest()[:12]


def train(name: str, args: argparse.Namespace, seed: int, graph: bool) -> dict:
    """Train one backend from `seed` for `args.steps` steps, evaluating the relative L2 error
    every `args.eval_every` steps outside the timed region. Returns the training seconds
    (building the step and any capture warmup included), the last step's loss, the final
    relative L2, a hash of the weights, and the training seconds and step count at the first
    evaluation below `args.target` (None if none was)."""
    # Seeded draws in the reference's order: model, then interior and boundary points from one
    # device generator.
    torch.manual_seed(seed)
    model = build_mlp(DEFAULT_POISSON_MLP).cuda()
    generator = torch.Generator(device="cuda").manual_seed(seed)
    interior = torch.rand(args.interior, 2, device="cuda", generator=generator) * 2 - 1
    boundary = boundary_points(args.boundary, device="cuda", generator=generator)

    clock = _TrainingClock()
    step, taken = _stepper(name, model, interior, boundary, args.lr, graph)
    loss: torch.Tensor | None = None
    first_hit: tuple[float, int] | None = None
    while taken < args.steps:
        window = min(args.eval_every, args.steps - taken)
        for _ in range(window):
            loss = step()
        taken += window
        with clock.paused() as elapsed:
            if first_hit is None and relative_l2_error(model) < args.target:
                first_hit = (elapsed, taken)
    return {
        "seconds": clock.seconds,
        "loss": float("nan") if loss is None else loss.detach().item(),
        "rel_l2": relative_l2_error(model),
        "weights": _weights_digest(model),
        "hit_seconds": None if first_hit is None else first_hit[0],
        "hit_step": None if first_hit is None else first_hit[1],
    }


def main(argv: list[str] | None = None) -> None:
    choices = [FUSED_STEP] + [n for n in _TRAINABLE if n in BACKENDS]
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--backends", nargs="+", choices=choices, default=[FUSED_STEP, "fused_cuda"])
    parser.add_argument("--steps", type=int, default=5_000)
    parser.add_argument("--interior", type=int, default=16_384)
    parser.add_argument("--boundary", type=int, default=1_024)
    parser.add_argument("--lr", type=float, default=1e-3)
    parser.add_argument("--seeds", type=int, nargs="+", default=[0])
    parser.add_argument("--cuda-graph", action="store_true", help="also run each backend captured as a HIP graph")
    parser.add_argument("--target", type=float, default=5e-3, help="relative L2 for time to target")
    parser.add_argument("--eval-every", type=int, default=250)
    args = parser.parse_args(argv)
    if args.steps < 1 or args.eval_every < 1 or args.interior < 1 or args.boundary < 0:
        parser.error("steps, eval-every and interior must be positive, boundary non-negative")
    if not torch.cuda.is_available():
        raise SystemExit("train_poisson needs a GPU")

    props = torch.cuda.get_device_properties(0)
    print(f"device: {props.name} ({getattr(props, 'gcnArchName', '?')}), torch {torch.__version__}")
    print(f"steps={args.steps} interior={args.interior} boundary={args.boundary} lr={args.lr} "
          f"loss=mean(res^2)+100*mean(u_b^2); seconds exclude rel-L2 evaluation every "
          f"{args.eval_every} steps; target {args.target}")
    print(f"{'backend':>22} {'graph':>5} {'seed':>4} {'seconds':>8} {'final loss':>12} {'rel L2':>10} "
          f"{'weights':>12} {'s to target':>11} {'step':>5}", flush=True)
    for name in args.backends:
        for graph in ((False, True) if args.cuda_graph else (False,)):
            runs = []
            for seed in args.seeds:
                r = train(name, args, seed, graph)
                runs.append(r)
                hit = "never" if r["hit_seconds"] is None else f"{r['hit_seconds']:.3f}"
                print(f"{name:>22} {'yes' if graph else 'no':>5} {seed:>4} {r['seconds']:>8.3f} "
                      f"{r['loss']:>12.5e} {r['rel_l2']:>10.3e} {r['weights']:>12} {hit:>11} "
                      f"{r['hit_step'] or '-':>5}", flush=True)
            if len(runs) > 1:
                hits = [r["hit_seconds"] for r in runs if r["hit_seconds"] is not None]
                print(f"{name:>22} {'yes' if graph else 'no':>5} {'med':>4} "
                      f"{statistics.median(r['seconds'] for r in runs):>8.3f} {'':>12} "
                      f"{statistics.median(r['rel_l2'] for r in runs):>10.3e} {'':>12} "
                      f"{(f'{statistics.median(hits):.3f}' if hits else 'never'):>11}", flush=True)


if __name__ == "__main__":
    main()
