"""Interchangeable implementations of ``model -> (u, Laplacian(u))``.

Every backend takes a dense MLP and ``[batch, dims]`` coordinates and returns the output and
its input Laplacian, both ``[batch, 1]``. ``eager`` is the registry's oracle. The ``*_cudagraph``
entries replay a HIP graph of their base backend (inference only; the base backend off the
GPU). The ``fused_*`` entries run the gfx950 kernels; they are registered only when the
extension is built.
Registry keys follow /root/reference/src/fused_hoad/backends/__init__.py:22-67; every
``fused_cuda*`` name maps onto the one forward kernel and the one backward kernel pair.
"""

from collections.abc import Callable
from functools import partial

from torch import Tensor, nn

from fused_hoad._extension import extension_available
from fused_hoad.backends.eager import eager_laplacian
from fused_hoad.backends.forward_laplacian import forward_laplacian
from fused_hoad.backends.func import func_laplacian
from fused_hoad.backends.graphs import cuda_graphed

Backend = Callable[[nn.Module, Tensor], tuple[Tensor, Tensor]]

BACKENDS: dict[str, Backend] = {
    "eager": eager_laplacian,
    "eager_cudagraph": cuda_graphed(eager_laplacian),
    "func": func_laplacian,
    "forward_laplacian": forward_laplacian,
    "forward_laplacian_cudagraph": cuda_graphed(forward_laplacian),
}

TRAINABLE_BACKENDS = ("eager", "func", "forward_laplacian")

FIXED_CONTRACT_BACKENDS: tuple[str, ...] = ()
if extension_available():
    from fused_hoad.backends.fused import fused_laplacian

    _FUSED = {
        "fused_cuda_v0": partial(fused_laplacian, version=0),
        "fused_cuda_v1": partial(fused_laplacian, version=1),
        "fused_cuda": fused_laplacian,
        "fused_cuda_tf32": partial(fused_laplacian, version=3),
        "fused_cuda_tf32_pipelined": partial(fused_laplacian, version=4),
        "fused_cuda_tf32_16warp": partial(fused_laplacian, version=5),
        "fused_cuda_bwd_v1": partial(fused_laplacian, backward="cuda_v1"),
        "fused_cuda_bwd_v3": partial(fused_laplacian, backward="cuda_v3"),
        "fused_cuda_bwd_v5": partial(fused_laplacian, backward="cuda_v5"),
        "fused_cuda_bwd_v4": partial(fused_laplacian, backward="cuda_v4"),
        "fused_cuda_bwd_v2": partial(fused_laplacian, backward="cuda_v2"),
        "fused_cuda_recompute": partial(fused_laplacian, backward="recompute"),
    }
    BACKENDS.update(_FUSED)
    FIXED_CONTRACT_BACKENDS = tuple(_FUSED)

REFERENCE_BACKEND = "eager"


def get_backend(name: str) -> Backend:
    """The backend registered under ``name``."""
    try:
        return BACKENDS[name]
    except KeyError:
        raise KeyError(f"unknown backend {name!r}; available: {', '.join(sorted(BACKENDS))}") from None


__all__ = [
    "BACKENDS",
    "FIXED_CONTRACT_BACKENDS",
    "REFERENCE_BACKEND",
    "TRAINABLE_BACKENDS",
    "Backend",
    "cuda_graphed",
    "eager_laplacian",
    "forward_laplacian",
    "func_laplacian",
    "get_backend",
]
