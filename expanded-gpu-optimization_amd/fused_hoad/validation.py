"""Error summary of one tensor against another, for comparing backends.

``error_metrics`` reduces on the tensors' device and brings the three figures to the host in
one transfer (one synchronization for GPU tensors instead of one per figure). Public names,
fields and error messages are those of /root/reference/src/fused_hoad/validation.py:8-33; the
relative error divides by ``|expected|`` floored at the dtype's machine epsilon, as there.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor


@dataclass(frozen=True, slots=True)
class ErrorMetrics:
    max_absolute: float
    max_relative: float
    mean_absolute: float


def error_metrics(actual: Tensor, expected: Tensor) -> ErrorMetrics:
    """Largest absolute and relative elementwise error, and the mean absolute error."""
    if actual.shape != expected.shape:
        raise ValueError(f"shape mismatch: {actual.shape} != {expected.shape}")
    if actual.numel() == 0:
        raise ValueError("cannot compare empty tensors")
    error = (actual - expected).abs()
    scale = expected.abs().clamp_min(torch.finfo(expected.dtype).eps)
    figures = torch.stack((error.max(), (error / scale).max(), error.mean())).tolist()
    return ErrorMetrics(*figures)
