"""Elementwise error summaries for comparing backends."""

from dataclasses import dataclass

import torch
from torch import Tensor


@dataclass(frozen=True, slots=True)
class ErrorMetrics:
    max_absolute: float
    max_relative: float
    mean_absolute: float


def error_metrics(actual: Tensor, expected: Tensor) -> ErrorMetrics:
    """Max absolute, max relative (against ``max(|expected|, eps)``) and mean absolute error."""
    if actual.shape != expected.shape:
        raise ValueError(f"shape mismatch: {actual.shape} != {expected.shape}")
    if actual.numel() == 0:
        raise ValueError("cannot compare empty tensors")
    absolute = (actual - expected).abs()
    floor = torch.finfo(expected.dtype).eps
    relative = absolute / expected.abs().clamp_min(floor)
    return ErrorMetrics(
        max_absolute=absolute.max().item(),
        max_relative=relative.max().item(),
        mean_absolute=absolute.mean().item(),
    )
