"""Fused backend: the whole forward Laplacian in one gfx950 kernel launch.

Fixed to the Poisson contract (2 -> 64x4 -> 1 tanh, FP32, on the GPU). The forward is one
kernel; the backward is the fused HIP kernel pair (default) or, when asked for by name, the
reference's PyTorch recompute-and-differentiate path. Behaviour follows
/root/reference/src/fused_hoad/backends/fused.py:24-138. One mode the reference does not have,
``"saved"``, keeps the forward's hidden-layer outputs (3 KB per point) so that the HIP
backward reads them instead of re-running the forward.
"""

from __future__ import annotations

import weakref

import torch
from torch import Tensor, nn

from fused_hoad._extension import (
    fused_forward_laplacian,
    fused_forward_laplacian_backward,
    load_extension,
)
from fused_hoad.backends.forward_laplacian import tanh_mlp_forward_laplacian
from fused_hoad.parameters import (
    POISSON_PARAMETER_LAYOUT,
    flattened_poisson_binding,
    flattened_poisson_parameters,
    pack_poisson_parameters,
    poisson_parameter_tensors,
    unpack_poisson_parameters,
)

# Backward modes. Every "cuda*" name runs the same fused HIP backward (the reference's kernel
# versions are kept as names only); "recompute" is the PyTorch reference backward; "saved" is
# the HIP backward reading the layer outputs the forward kept (bitwise the same gradients as
# "cuda", with 3 KB per point held from the forward to the backward).
_CUDA_BACKWARD_VERSIONS = {
    "cuda": 6,
    "cuda_v1": 1,
    "cuda_v2": 2,
    "cuda_v3": 3,
    "cuda_v4": 4,
    "cuda_v5": 5,
}
BACKWARD_MODES = (*_CUDA_BACKWARD_VERSIONS, "recompute")  # the reference's names
SAVED_MODE = "saved"
_ACCEPTED_MODES = (*BACKWARD_MODES, SAVED_MODE)

_cache: dict[str, object] = {}


class FusedForwardLaplacian(torch.autograd.Function):
    """Fused-kernel forward; fused-kernel (or, by name, recompute) backward, over a packed
    parameter buffer (the reference's public Function, same arguments). ``fused_laplacian``
    runs it for the ``"recompute"`` mode of a model as built; its ``"cuda*"`` and ``"saved"``
    modes run the C++ Function behind ``_C._model_laplacian``, which gives bitwise the same
    results."""

    @staticmethod
    def forward(ctx, coordinates: Tensor, parameters: Tensor, version: int, backward: str):
        ctx.backward_mode = backward
        if backward == SAVED_MODE:
            output, laplacian, saved = load_extension()._forward_saving(coordinates, parameters, version)
            ctx.save_for_backward(coordinates, parameters, saved)
            return output, laplacian
        ctx.save_for_backward(coordinates, parameters)
        return fused_forward_laplacian(coordinates, parameters, version)

    @staticmethod
    def backward(ctx, grad_output: Tensor, grad_laplacian: Tensor):
        coordinates, parameters, *saved = ctx.saved_tensors
        needs_coordinates, needs_parameters = ctx.needs_input_grad[:2]
        mode = ctx.backward_mode
        if mode == SAVED_MODE:
            grad_parameters, grad_coordinates = load_extension()._backward(
                coordinates,
                parameters,
                grad_output.reshape(-1).contiguous(),
                grad_laplacian.reshape(-1).contiguous(),
                needs_coordinates,
                6,
                saved[0],
            )
            return grad_coordinates, grad_parameters if needs_parameters else None, None, None
        if mode in _CUDA_BACKWARD_VERSIONS:
            grad_parameters, grad_coordinates = fused_forward_laplacian_backward(
                coordinates, parameters, grad_output, grad_laplacian, _CUDA_BACKWARD_VERSIONS[mode]
            )
            return (
                grad_coordinates if needs_coordinates else None,
                grad_parameters if needs_parameters else None,
                None,
                None,
            )
        grad_coordinates, grad_parameters = _recompute_backward(
            coordinates, parameters, grad_output, grad_laplacian, needs_coordinates, needs_parameters
        )
        return grad_coordinates, grad_parameters, None, None


class FlattenedFusedLaplacian(torch.autograd.Function):
    """The ``"recompute"`` mode for a model whose parameters are views of one packed buffer
    (``flatten_poisson_parameters_``): the kernel reads that buffer directly, the autograd
    inputs are the model's ten parameters themselves, and the backward (the PyTorch reference
    backward) hands each one a view of the packed gradient. The ``"cuda*"`` and ``"saved"``
    modes run the C++ autograd Function behind ``_C._model_laplacian``, which does the same
    without the Python Function's per-step host work. An output the loss does
    not use reaches the backward as ``None`` and is read as zero."""

    @staticmethod
    def forward(ctx, coordinates: Tensor, flat: Tensor, version: int, *parameters: Tensor):
        ctx.set_materialize_grads(False)
        # The parameters are saved too (no copy): each view of the buffer has its own version
        # counter, so an in-place update between forward and backward raises PyTorch's
        # in-place-modification error when the backward unpacks them, as nn.Linear would.
        ctx.save_for_backward(coordinates, flat, *parameters)
        return fused_forward_laplacian(coordinates, flat, version)

    @staticmethod
    def backward(ctx, grad_output: Tensor | None, grad_laplacian: Tensor | None):
        coordinates, flat, *_ = ctx.saved_tensors
        needs_coordinates = ctx.needs_input_grad[0]
        needs_parameters = any(ctx.needs_input_grad[3:])
        if grad_output is None and grad_laplacian is None:
            return (None,) * (3 + len(POISSON_PARAMETER_LAYOUT) * 2)
        zeros = torch.zeros(coordinates.shape[0], 1, dtype=flat.dtype, device=flat.device)
        grad_coordinates, grad_flat = _recompute_backward(
            coordinates,
            flat,
            zeros if grad_output is None else grad_output,
            zeros if grad_laplacian is None else grad_laplacian,
            needs_coordinates,
            True,
        )
        grads: list[Tensor | None] = []
        for spec, needs in zip(POISSON_PARAMETER_LAYOUT, _pairs(ctx.needs_input_grad[3:]), strict=True):
            grads.append(
                grad_flat[spec.weight_offset : spec.bias_offset].view(spec.out_features, spec.in_features)
                if needs[0] else None
            )
            grads.append(grad_flat[spec.bias_offset : spec.end_offset] if needs[1] else None)
        if not needs_parameters:
            grads = [None] * len(grads)
        return (grad_coordinates if needs_coordinates else None, None, None, *grads)


def _pairs(flags):
    return [(flags[i], flags[i + 1]) for i in range(0, len(flags), 2)]


def _recompute_backward(
    coordinates: Tensor,
    parameters: Tensor,
    grad_output: Tensor,
    grad_laplacian: Tensor,
    needs_coordinates: bool,
    needs_parameters: bool,
) -> tuple[Tensor | None, Tensor | None]:
    """The reference backward: rebuild the jet in PyTorch from the packed buffer and
    differentiate it with autograd (/root/reference/src/fused_hoad/backends/fused.py:76-101)."""
    with torch.enable_grad():
        x = coordinates.detach().requires_grad_(needs_coordinates)
        flat = parameters.detach().requires_grad_(needs_parameters)
        views = unpack_poisson_parameters(flat)
        linears = [
            (views[f"{spec.name}.weight"], views[f"{spec.name}.bias"])
            for spec in POISSON_PARAMETER_LAYOUT
        ]
        outputs = tanh_mlp_forward_laplacian(linears, x)
        wanted = [tensor for tensor, needed in ((x, needs_coordinates), (flat, needs_parameters)) if needed]
        grads = list(
            torch.autograd.grad(outputs, wanted, (grad_output, grad_laplacian), allow_unused=True)
        )
    grad_coordinates = grads.pop(0) if needs_coordinates else None
    grad_parameters = grads.pop(0) if needs_parameters else None
    return grad_coordinates, grad_parameters


def _packed_parameters(model: nn.Module) -> Tensor:
    """Differentiable pack while training; otherwise one cached pack per weight update.

    The parameter list is cached per model behind a weakref (a recycled ``id`` cannot return
    another model's buffer); a call then only compares the parameters' version counters.
    """
    model_ref = _cache.get("model")
    if model_ref is None or model_ref() is not model:
        _cache.clear()
        _cache.update(model=weakref.ref(model), parameters=list(model.parameters()))
    parameters: list[Tensor] = _cache["parameters"]  # type: ignore[assignment]
    if torch.is_grad_enabled() and any(p.requires_grad for p in parameters):
        return pack_poisson_parameters(model, differentiable=True)
    flat = flattened_poisson_parameters(model)
    if flat is not None:  # the parameters are views of a packed buffer: no copy, never stale
        return flat
    versions = [p._version for p in parameters]
    if versions != _cache.get("versions"):
        _cache.update(versions=versions, packed=pack_poisson_parameters(model))
    return _cache["packed"]  # type: ignore[return-value]


def fused_laplacian(
    model: nn.Module, coordinates: Tensor, version: int = 2, backward: str = "cuda"
) -> tuple[Tensor, Tensor]:
    """``(u, Laplacian u)`` of the fixed Poisson MLP from one gfx950 kernel launch.

    ``backward`` selects the gradient path when autograd is active: any ``"cuda*"`` mode runs
    the fused HIP backward; ``"recompute"`` runs the PyTorch reference backward; ``"saved"``
    runs the fused HIP backward on the layer outputs the forward kept (3 KB per point until the
    backward), which spares it the forward re-run and gives bitwise the same gradients.
    """
    if backward not in _ACCEPTED_MODES:
        raise ValueError(f"backward must be one of {_ACCEPTED_MODES}")
    if torch.is_grad_enabled():
        # A flattened model's parameters are views of its packed buffer: no pack at all.
        binding = flattened_poisson_binding(model)
        flat, tensors = binding if binding is not None else (None, poisson_parameter_tensors(model))
        coordinates = coordinates.contiguous()
        if coordinates.requires_grad or any(t.requires_grad for t in tensors):
            if backward != "recompute":
                u, lap = load_extension()._model_laplacian(
                    coordinates, flat, version, _CUDA_BACKWARD_VERSIONS.get(backward, 6),
                    backward == SAVED_MODE, tensors,
                )
                return u, lap
            if flat is not None:
                return FlattenedFusedLaplacian.apply(coordinates, flat, version, *tensors)
        elif flat is not None:
            return fused_forward_laplacian(coordinates, flat, version)
    parameters = _packed_parameters(model)
    if parameters.requires_grad or coordinates.requires_grad:
        return FusedForwardLaplacian.apply(coordinates.contiguous(), parameters, version, backward)
    return fused_forward_laplacian(coordinates.contiguous(), parameters, version)
