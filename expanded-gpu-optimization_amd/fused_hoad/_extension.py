"""Access to the compiled MI355X extension ``fused_hoad._C``.

Mirrors /root/reference/src/fused_hoad/_extension.py:8-65. The extension is the only way into
the kernels: when it is not built, every fused entry point raises; nothing falls back to
another implementation.
"""

from __future__ import annotations

from types import ModuleType

from torch import Tensor

_BUILD_HINT = (
    "The fused_hoad HIP extension is not built. Build it for gfx950 in-tree with "
    "`python -m fused_hoad._build` (run from expanded-gpu-optimization_amd/), the equivalent "
    "of the reference's `pip install -e . --no-build-isolation`."
)


def load_extension() -> ModuleType:
    """Return the compiled extension or raise an actionable ``RuntimeError``."""
    try:
        from fused_hoad import _C
    except ImportError as exc:
        raise RuntimeError(_BUILD_HINT) from exc
    return _C


def extension_available() -> bool:
    """Whether ``fused_hoad._C`` (and the HIP library it links) can be imported."""
    try:
        load_extension()
    except RuntimeError:
        return False
    return True


def fused_forward_laplacian(
    coordinates: Tensor, parameters: Tensor, version: int = 2
) -> tuple[Tensor, Tensor]:
    """``(u, Laplacian u)``, each ``[batch, 1]``, from the gfx950 forward kernel.

    ``version`` 0..5 is accepted for compatibility with the reference's variants; every
    value runs the same kernel.
    """
    output, laplacian = load_extension().fused_forward_laplacian(coordinates, parameters, version)
    return output, laplacian


def fused_forward_laplacian_backward(
    coordinates: Tensor,
    parameters: Tensor,
    grad_output: Tensor,
    grad_laplacian: Tensor,
    version: int = 6,
) -> tuple[Tensor, Tensor]:
    """``(grad_parameters[12737], grad_coordinates[batch, 2])`` from the gfx950 backward.

    Upstream gradients may be ``[batch]`` or ``[batch, 1]``. ``version`` 1..6 is accepted for
    compatibility; every value runs the same deterministic kernels.
    """
    grad_parameters, grad_coordinates = load_extension().fused_forward_laplacian_backward(
        coordinates,
        parameters,
        grad_output.reshape(-1).contiguous(),
        grad_laplacian.reshape(-1).contiguous(),
        version,
    )
    return grad_parameters, grad_coordinates


def poisson_adam_step(
    coordinates: Tensor,
    source: Tensor,
    parameters: Tensor,
    exp_avg: Tensor,
    exp_avg_sq: Tensor,
    step: Tensor,
    *,
    lr: float,
    betas: tuple[float, float],
    eps: float,
    weight_decay: float,
    grad_parameters: Tensor | None = None,
    grad_coordinates: Tensor | None = None,
    boundary: Tensor | None = None,
    boundary_weight: float = 100.0,
) -> Tensor:
    """One fused Poisson PINN + Adam step (two gfx950 kernels); updates ``parameters``,
    ``exp_avg``, ``exp_avg_sq`` and ``step`` in place and returns the loss at entry:
    ``mean((Lap u - f)^2)`` over ``coordinates``, plus ``boundary_weight * mean(u^2)`` over
    ``boundary`` when given."""
    return load_extension().poisson_adam_step(
        coordinates,
        source,
        parameters,
        exp_avg,
        exp_avg_sq,
        step,
        float(lr),
        float(betas[0]),
        float(betas[1]),
        float(eps),
        float(weight_decay),
        grad_parameters,
        grad_coordinates,
        boundary,
        float(boundary_weight),
    )
