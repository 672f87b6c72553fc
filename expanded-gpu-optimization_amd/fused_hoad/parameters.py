"""Packed 12,737-float parameter ABI of the fixed Poisson MLP.

Layout (identical to /root/reference/src/fused_hoad/parameters.py:28-48 and
/root/reference/csrc/mlp_abi.cuh:8-17): for each linear layer in order, its weight
``[out, in]`` row-major followed by its bias ``[out]``::

    layer0  W[64, 2]  @0       b[64] @128
    layer1  W[64, 64] @192     b[64] @4288
    layer2  W[64, 64] @4352    b[64] @8448
    layer3  W[64, 64] @8512    b[64] @12608
    layer4  W[1, 64]  @12672   b[1]  @12736      (12,737 floats)

The kernels read this buffer directly; nothing else about the model crosses the boundary.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor, nn

_SHAPES = ((64, 2), (64, 64), (64, 64), (64, 64), (1, 64))


@dataclass(frozen=True, slots=True)
class ParameterSlice:
    """Where one linear layer's weight and bias live in the packed buffer."""

    name: str
    out_features: int
    in_features: int
    weight_offset: int
    bias_offset: int

    @property
    def weight_elements(self) -> int:
        return self.out_features * self.in_features

    @property
    def end_offset(self) -> int:
        return self.bias_offset + self.out_features


def _layout() -> tuple[ParameterSlice, ...]:
    slices = []
    cursor = 0
    for index, (rows, cols) in enumerate(_SHAPES):
        slices.append(ParameterSlice(f"layer{index}", rows, cols, cursor, cursor + rows * cols))
        cursor += rows * cols + rows
    return tuple(slices)


POISSON_PARAMETER_LAYOUT: tuple[ParameterSlice, ...] = _layout()
POISSON_PARAMETER_COUNT: int = POISSON_PARAMETER_LAYOUT[-1].end_offset


def _linear_layers(model: nn.Module) -> list[nn.Linear]:
    """The model's ``nn.Linear`` modules in ``model.modules()`` order (pre-order, each module
    once), walked through ``_modules`` directly: half the host time of ``modules()``, which
    builds every module's name on the way. The autograd path walks the model every step."""
    layers: list[nn.Linear] = [model] if isinstance(model, nn.Linear) else []
    _collect_linear(model, {model}, layers)
    return layers


def _collect_linear(module: nn.Module, seen: set[nn.Module], layers: list[nn.Linear]) -> None:
    for child in module._modules.values():
        if child is None or child in seen:
            continue
        seen.add(child)
        if isinstance(child, nn.Linear):
            layers.append(child)
        _collect_linear(child, seen, layers)


def poisson_parameter_tensors(model: nn.Module) -> list[Tensor]:
    """The model's ten weights and biases in packed-layout order, checked against the layout
    (the pack's errors and messages)."""
    layers = _linear_layers(model)
    if len(layers) != len(POISSON_PARAMETER_LAYOUT):
        raise ValueError(f"expected {len(POISSON_PARAMETER_LAYOUT)} linear layers")
    tensors: list[Tensor] = []
    for layer, spec in zip(layers, POISSON_PARAMETER_LAYOUT, strict=True):
        weight, bias = _weight_and_bias(layer)
        expected = (spec.out_features, spec.in_features)
        if weight.shape != expected:
            raise ValueError(
                f"{spec.name}.weight must have shape {expected}, got {tuple(weight.shape)}"
            )
        if bias is None or bias.shape != (spec.out_features,):
            raise ValueError(f"{spec.name}.bias must have shape ({spec.out_features},)")
        tensors += (weight, bias)
    return tensors


def _weight_and_bias(layer: nn.Linear) -> tuple[Tensor, Tensor | None]:
    """``(layer.weight, layer.bias)``, read from the registered parameters when they are there
    (Module.__getattr__ costs about half a microsecond per read, and the autograd path reads
    every layer on every step)."""
    registered = layer._parameters
    weight = registered.get("weight")
    if weight is None:
        weight = layer.weight
    bias = registered.get("bias") if "bias" in registered else layer.bias
    return weight, bias


def _segments(model: nn.Module) -> list[Tensor]:
    return [tensor.reshape(-1) for tensor in poisson_parameter_tensors(model)]


def pack_poisson_parameters(model: nn.Module, *, differentiable: bool = False) -> Tensor:
    """Pack the fixed 2x64x64x64x64x1 MLP into the kernel ABI layout.

    ``differentiable=True`` returns a ``torch.cat`` of the parameters, so a gradient on the
    packed buffer flows back to the model; otherwise a detached contiguous copy.
    (Behaviour of /root/reference/src/fused_hoad/parameters.py:55-84.)
    """
    segments = _segments(model)
    if differentiable:
        return torch.cat(segments)
    with torch.no_grad():
        return torch.cat([segment.detach() for segment in segments]).contiguous()


def unpack_poisson_parameters(parameters: Tensor) -> dict[str, Tensor]:
    """Shaped views ``layerN.weight`` / ``layerN.bias`` into a packed buffer."""
    if parameters.ndim != 1 or parameters.numel() != POISSON_PARAMETER_COUNT:
        raise ValueError(f"parameters must have shape [{POISSON_PARAMETER_COUNT}]")
    views: dict[str, Tensor] = {}
    for spec in POISSON_PARAMETER_LAYOUT:
        weight = parameters[spec.weight_offset : spec.bias_offset]
        views[f"{spec.name}.weight"] = weight.view(spec.out_features, spec.in_features)
        views[f"{spec.name}.bias"] = parameters[spec.bias_offset : spec.end_offset]
    return views


def flatten_poisson_parameters_(model: nn.Module) -> Tensor:
    """Move the model's parameters into one packed ABI buffer, in place, and return it.

    Each ``weight`` / ``bias`` becomes a view of the returned buffer (still a leaf
    ``nn.Parameter``), so the model, any optimizer over ``model.parameters()`` and the fused
    kernels all see the same memory and the pack costs nothing afterwards. Calling it again
    on a flattened model returns the same buffer; after ``model.to(...)`` or a reassigned
    parameter it flattens anew.
    """
    existing = flattened_poisson_parameters(model)
    if existing is not None:
        return existing
    flat = pack_poisson_parameters(model)
    with torch.no_grad():
        for layer, spec in zip(_linear_layers(model), POISSON_PARAMETER_LAYOUT, strict=True):
            layer.weight.data = flat[spec.weight_offset : spec.bias_offset].view(
                spec.out_features, spec.in_features
            )
            layer.bias.data = flat[spec.bias_offset : spec.end_offset]
    model._fused_hoad_packed = flat
    return flat


def flattened_poisson_parameters(model: nn.Module) -> Tensor | None:
    """The packed buffer the model's parameters are views of, or ``None`` if they are not
    (never flattened, moved, or a parameter reassigned since)."""
    binding = flattened_poisson_binding(model)
    return None if binding is None else binding[0]


def flattened_poisson_binding(model: nn.Module) -> tuple[Tensor, list[Tensor]] | None:
    """``(packed buffer, the ten parameters in layout order)`` for a model whose parameters are
    views of the buffer at their layout offsets, else ``None``; one walk over the modules (the
    autograd path calls it every step)."""
    flat = getattr(model, "_fused_hoad_packed", None)
    if flat is None:
        return None
    base = flat.data_ptr()
    item = flat.element_size()
    tensors: list[Tensor] = []
    layers = _linear_layers(model)
    if len(layers) != len(POISSON_PARAMETER_LAYOUT):
        return None
    for layer, spec in zip(layers, POISSON_PARAMETER_LAYOUT):
        # The registered parameters themselves (what ``layer.weight`` returns, without
        # Module.__getattr__); a layer that keeps them elsewhere is not a flattened one.
        weight = layer._parameters.get("weight")
        bias = layer._parameters.get("bias")
        if (
            weight is None
            or bias is None
            or weight.data_ptr() != base + item * spec.weight_offset
            or bias.data_ptr() != base + item * spec.bias_offset
        ):
            return None
        tensors += (weight, bias)
    if tensors[0].device != flat.device:
        return None
    return flat, tensors
