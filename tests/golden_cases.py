"""Loader for the committed golden fixtures (tests/golden/fused_hoad_golden.npz)."""

from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).with_name("golden") / "fused_hoad_golden.npz"
CASE_NAMES = ("single_point", "ragged_tile", "workgroup_tile", "ragged_batch", "saturated")


def load_case(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN, allow_pickle=False) as data:
        key = str(data[f"{name}/params_key"])
        case = {field: data[f"{name}/{field}"] for field in (
            "coordinates", "grad_output", "grad_laplacian", "u", "laplacian",
            "grad_parameters", "grad_coordinates")}
        case["parameters"] = data[key]
    return case
