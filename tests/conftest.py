"""Shared test setup: import paths, the ``gpu`` marker and small helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = ROOT / "expanded-gpu-optimization_amd"
for path in (ROOT, PACKAGE_ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP extension"
    )


def assert_scaled_close(actual, expected, tolerance: float, what: str = "") -> None:
    """max |actual - expected| <= tolerance * max |expected| (sums over many points are
    compared against the gradient block's own scale, as in the reference's tests)."""
    scale = float(abs(expected).max())
    error = float(abs(actual - expected).max())
    assert error <= tolerance * scale, f"{what}: max error {error:.3e} vs scale {scale:.3e}"
