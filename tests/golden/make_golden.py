"""Write tests/golden/fused_hoad_golden.npz: small input/output vectors for the hot path.

Inputs are float32 (what the kernels consume): packed parameters of the seeded reference
model (``torch.manual_seed(seed)`` + default ``nn.Linear`` init, optionally scaled), coordinates
uniform in [-1, 1]^2 and upstream gradients from a seeded numpy generator. Expected outputs
are the float64 oracle (oracle/jet.py) evaluated on exactly those float32 values. The
fixtures are cross-checked against nested eager autograd in tests/test_golden.py.

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import jet, torch_ref  # noqa: E402

CASES = (
    # name, model seed, weight scale, batch, data seed
    ("single_point", 0, 1.0, 1, 10),
    ("ragged_tile", 0, 1.0, 17, 11),
    ("workgroup_tile", 0, 1.0, 64, 12),
    ("ragged_batch", 0, 1.0, 100, 13),
    ("saturated", 1, 3.0, 33, 14),
)


def main() -> None:
    arrays: dict[str, np.ndarray] = {}
    params = {}
    for name, seed, scale, batch, data_seed in CASES:
        key = f"params_s{seed}_x{scale:g}"
        if key not in params:
            flat = (torch_ref.pack(torch_ref.reference_model(seed)).numpy() * np.float32(scale)).astype(np.float32)
            params[key] = flat
            arrays[key] = flat
        flat = params[key]
        rng = np.random.default_rng(data_seed)
        coords = rng.uniform(-1.0, 1.0, (batch, 2)).astype(np.float32)
        gu = rng.standard_normal(batch).astype(np.float32)
        gl = rng.standard_normal(batch).astype(np.float32)
        u, lap = jet.forward(flat.astype(np.float64), coords.astype(np.float64))
        gp, gx = jet.backward(flat.astype(np.float64), coords.astype(np.float64), gu, gl)
        arrays[f"{name}/params_key"] = np.array(key)
        arrays[f"{name}/coordinates"] = coords
        arrays[f"{name}/grad_output"] = gu
        arrays[f"{name}/grad_laplacian"] = gl
        arrays[f"{name}/u"] = u
        arrays[f"{name}/laplacian"] = lap
        arrays[f"{name}/grad_parameters"] = gp
        arrays[f"{name}/grad_coordinates"] = gx
    out = Path(__file__).with_name("fused_hoad_golden.npz")
    np.savez_compressed(out, **arrays)
    print(f"wrote {out} ({out.stat().st_size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
