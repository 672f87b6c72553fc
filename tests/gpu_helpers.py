"""Helpers shared by the GPU tests: the GPU and the built extension are required (a missing
extension is a failure, never a skip), and every case prints what it runs before touching
the GPU."""

from __future__ import annotations

import contextlib
import os
import sys

import numpy as np
import torch

from oracle import torch_ref


def require_gpu_extension():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from fused_hoad._extension import load_extension

    return load_extension()  # raises when the HIP extension is not built


def announce(what: str) -> None:
    print(f"[gpu case] {what}", file=sys.stderr, flush=True)


def packed(seed: int = 0, scale: float = 1.0, device: str = "cuda") -> torch.Tensor:
    flat = torch_ref.pack(torch_ref.reference_model(seed)) * scale
    return flat.to(device).contiguous()


def coordinates(batch: int, seed: int = 0, device: str = "cuda") -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    return (torch.rand(batch, 2, generator=gen) * 2 - 1).to(device)


def upstream(batch: int, seed: int = 0, device: str = "cuda"):
    gen = torch.Generator().manual_seed(seed + 1000)
    gu = torch.randn(batch, 1, generator=gen).to(device)
    gl = torch.randn(batch, 1, generator=gen).to(device)
    return gu, gl


def to_numpy64(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().double().numpy()


@contextlib.contextmanager
def knobs(**values: str):
    """Set the kernels' experiment knobs (environment variables read on every call) for the
    duration of a block, restoring the previous values afterwards."""
    saved = {k: os.environ.get(k) for k in values}
    os.environ.update(values)
    try:
        yield
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
