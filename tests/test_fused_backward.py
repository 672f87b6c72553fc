"""GPU parity of the gfx950 backward kernels (through fused_hoad._C and the C ABI).

Tolerance: max |error| <= 1e-4 x max |expected| for the whole parameter gradient, for each of
the 10 weight/bias blocks separately, and for the coordinate gradient (the north star's bar;
the reference's test_fused.py:185-218). Expected values come from the PyTorch reference
backward (autograd through the jet, oracle/torch_ref.py) in FP32 on the GPU, and from the
float64 closed-form oracle (oracle/jet.py).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from conftest import assert_scaled_close
from golden_cases import CASE_NAMES, load_case
from gpu_helpers import announce, coordinates, knobs, packed, require_gpu_extension, to_numpy64, upstream
from oracle import jet, torch_ref

pytestmark = pytest.mark.gpu

BLOCKS = [
    ("layer0.weight", 0, 128), ("layer0.bias", 128, 192),
    ("layer1.weight", 192, 4288), ("layer1.bias", 4288, 4352),
    ("layer2.weight", 4352, 8448), ("layer2.bias", 8448, 8512),
    ("layer3.weight", 8512, 12608), ("layer3.bias", 12608, 12672),
    ("layer4.weight", 12672, 12736), ("layer4.bias", 12736, 12737),
]


@pytest.fixture(scope="module", autouse=True)
def _extension():
    return require_gpu_extension()


def _fused_backward(x, p, gu, gl, version=6):
    from fused_hoad._extension import fused_forward_laplacian_backward

    return fused_forward_laplacian_backward(x, p, gu, gl, version)


def _pair(batch: int, seed: int = 0, scale: float = 1.0):
    p = packed(seed, scale)
    x = coordinates(batch, seed=seed + batch)
    gu, gl = upstream(batch, seed=seed + batch)
    actual = _fused_backward(x, p, gu, gl)
    expected = torch_ref.recompute_backward(p, x, gu, gl)
    return actual, expected


@pytest.mark.parametrize(
    "batch", [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 1000, 1024, 16385, 65536, 65537]
)
def test_backward_matches_recompute(batch: int) -> None:
    announce(f"backward vs recompute, batch={batch}")
    (gp, gx), (ep, ex) = _pair(batch)
    assert gp.shape == (12737,) and gx.shape == (batch, 2)
    assert_scaled_close(gp, ep, 1e-4, "grad_parameters")
    assert_scaled_close(gx, ex, 1e-4, "grad_coordinates")


def test_backward_matches_recompute_with_saturated_tanh() -> None:
    announce("backward vs recompute, weights x3, batch=4096")
    (gp, gx), (ep, ex) = _pair(4096, seed=1, scale=3.0)
    assert_scaled_close(gp, ep, 1e-4, "grad_parameters")
    assert_scaled_close(gx, ex, 1e-4, "grad_coordinates")


@pytest.mark.parametrize("seed,scale", [(0, 1.0), (1, 3.0)])
def test_backward_matches_per_parameter_block(seed: int, scale: float) -> None:
    announce(f"backward per block, seed={seed} scale={scale}, batch=2048")
    (gp, _), (ep, _) = _pair(2048, seed=seed, scale=scale)
    for name, lo, hi in BLOCKS:
        assert_scaled_close(gp[lo:hi], ep[lo:hi], 1e-4, name)


def test_backward_matches_float64_oracle_per_block() -> None:
    announce("backward vs float64 oracle per block, batch=3000")
    p = packed(2)
    x = coordinates(3000, seed=2)
    gu, gl = upstream(3000, seed=2)
    gp, gx = _fused_backward(x, p, gu, gl)
    ep, ex = jet.backward(to_numpy64(p), to_numpy64(x), to_numpy64(gu), to_numpy64(gl))
    gp64 = to_numpy64(gp)
    for name, lo, hi in BLOCKS:
        assert_scaled_close(gp64[lo:hi], ep[lo:hi], 1e-4, name)
    assert_scaled_close(to_numpy64(gx), ex, 1e-4, "grad_coordinates")


@pytest.mark.parametrize("name", CASE_NAMES)
def test_backward_matches_golden_fixture(name: str) -> None:
    announce(f"backward vs golden fixture {name}")
    case = load_case(name)
    p = torch.from_numpy(case["parameters"]).cuda()
    x = torch.from_numpy(case["coordinates"]).cuda()
    gu = torch.from_numpy(case["grad_output"]).cuda()
    gl = torch.from_numpy(case["grad_laplacian"]).cuda()
    gp, gx = _fused_backward(x, p, gu, gl)
    gp64 = to_numpy64(gp)
    for block, lo, hi in BLOCKS:
        assert_scaled_close(gp64[lo:hi], case["grad_parameters"][lo:hi], 1e-4, block)
    assert_scaled_close(to_numpy64(gx), case["grad_coordinates"], 1e-4, "grad_coordinates")


def test_backward_many_tiles_per_slot() -> None:
    announce("backward vs recompute, batch=262144 (16 workgroup tiles per slot)")
    (gp, gx), (ep, ex) = _pair(262144, seed=4)
    for name, lo, hi in BLOCKS:
        assert_scaled_close(gp[lo:hi], ep[lo:hi], 1e-4, name)
    assert_scaled_close(gx, ex, 1e-4, "grad_coordinates")


def test_backward_is_bitwise_deterministic_across_runs_grids_and_versions() -> None:
    announce("backward determinism: repeats, FUSED_HOAD_BWD_BLOCKS, versions, batch=65536")
    p = packed(0)
    x = coordinates(65536, seed=6)
    gu, gl = upstream(65536, seed=6)
    ref_p, ref_x = _fused_backward(x, p, gu, gl)
    saved = os.environ.pop("FUSED_HOAD_BWD_BLOCKS", None)
    try:
        for blocks in (None, 1, 7, 64, 100, 256):
            if blocks is None:
                os.environ.pop("FUSED_HOAD_BWD_BLOCKS", None)
            else:
                os.environ["FUSED_HOAD_BWD_BLOCKS"] = str(blocks)
            gp, gx = _fused_backward(x, p, gu, gl)
            assert torch.equal(gp, ref_p), f"grad_parameters changed with {blocks} blocks"
            assert torch.equal(gx, ref_x), f"grad_coordinates changed with {blocks} blocks"
        os.environ.pop("FUSED_HOAD_BWD_BLOCKS", None)
        for version in range(1, 7):
            gp, gx = _fused_backward(x, p, gu, gl, version)
            assert torch.equal(gp, ref_p) and torch.equal(gx, ref_x)
    finally:
        os.environ.pop("FUSED_HOAD_BWD_BLOCKS", None)
        if saved is not None:
            os.environ["FUSED_HOAD_BWD_BLOCKS"] = saved


def test_backward_past_the_last_whole_round() -> None:
    """70,001 points are 4 whole rounds of 64-point tiles on 256 slots plus 4,465 points, which
    run as 16-point tiles shared by the workgroup's 4 waves: against the recompute backward,
    and bitwise the same for every grid."""
    announce("backward past the last whole round, batch=70001, FUSED_HOAD_BWD_BLOCKS in {1, 7, 256}")
    p = packed(0)
    x = coordinates(70001, seed=11)
    gu, gl = upstream(70001, seed=11)
    ref_p, ref_x = _fused_backward(x, p, gu, gl)
    ep, ex = torch_ref.recompute_backward(p, x, gu, gl)
    for name, lo, hi in BLOCKS:
        assert_scaled_close(ref_p[lo:hi], ep[lo:hi], 1e-4, name)
    assert_scaled_close(ref_x, ex, 1e-4, "grad_coordinates")
    for blocks in ("1", "7", "256"):
        with knobs(FUSED_HOAD_BWD_BLOCKS=blocks):
            gp, gx = _fused_backward(x, p, gu, gl)
        assert torch.equal(gp, ref_p) and torch.equal(gx, ref_x), f"changed with {blocks} blocks"


@pytest.mark.parametrize("batch", [1, 17, 1000, 4096, 12288])
def test_split_backward_agrees_with_the_tiled_kernel(batch: int) -> None:
    """Up to 768 16-point tiles the backward runs backward_split_kernel (rows split over a
    workgroup's waves). It does backward_kernel's arithmetic with the sums over points grouped
    differently, so the two agree to rounding: 1e-5 of each block's scale, ten times tighter
    than the parity bar."""
    announce(f"backward split kernel vs tiled kernel, batch={batch}")
    p = packed(0)
    x = coordinates(batch, seed=31)
    gu, gl = upstream(batch, seed=31)
    with knobs(FUSED_HOAD_BWD_SPLIT="1"):
        sp, sx = _fused_backward(x, p, gu, gl)
    with knobs(FUSED_HOAD_BWD_SPLIT="0"):
        tp, tx = _fused_backward(x, p, gu, gl)
    for name, lo, hi in BLOCKS:
        assert_scaled_close(sp[lo:hi], tp[lo:hi], 1e-5, name)
    assert_scaled_close(sx, tx, 1e-5, "grad_coordinates")


@pytest.mark.parametrize("batch", [12288, 12289])
def test_backward_on_both_sides_of_the_kernel_threshold(batch: int) -> None:
    """12,288 points (768 16-point tiles) still run backward_split_kernel, 12,289 run
    backward_kernel; both meet the parity bar against the recompute backward."""
    announce(f"backward at the split-kernel threshold, batch={batch}, vs recompute")
    (gp, gx), (ep, ex) = _pair(batch, seed=8)
    for name, lo, hi in BLOCKS:
        assert_scaled_close(gp[lo:hi], ep[lo:hi], 1e-4, name)
    assert_scaled_close(gx, ex, 1e-4, "grad_coordinates")


def test_split_backward_many_tiles_per_slot_and_saturated_tanh() -> None:
    announce("backward split kernel forced at batch=20000 (several tiles per slot), weights x3, vs recompute")
    with knobs(FUSED_HOAD_BWD_SPLIT="1"):
        (gp, gx), (ep, ex) = _pair(20000, seed=5, scale=3.0)
    for name, lo, hi in BLOCKS:
        assert_scaled_close(gp[lo:hi], ep[lo:hi], 1e-4, name)
    assert_scaled_close(gx, ex, 1e-4, "grad_coordinates")


def test_split_backward_is_bitwise_deterministic_across_grids() -> None:
    announce("backward split kernel determinism: repeats and FUSED_HOAD_BWD_BLOCKS, batch=4096")
    p = packed(0)
    x = coordinates(4096, seed=33)
    gu, gl = upstream(4096, seed=33)
    ref_p, ref_x = _fused_backward(x, p, gu, gl)
    for blocks in ("1", "7", "100", "256"):
        with knobs(FUSED_HOAD_BWD_BLOCKS=blocks):
            gp, gx = _fused_backward(x, p, gu, gl)
        assert torch.equal(gp, ref_p) and torch.equal(gx, ref_x), f"changed with {blocks} blocks"


def test_backward_handles_empty_batch() -> None:
    announce("backward, empty batch")
    p = packed(0)
    empty = torch.empty(0, 2, device="cuda")
    gp, gx = _fused_backward(empty, p, torch.empty(0, 1, device="cuda"), torch.empty(0, 1, device="cuda"))
    assert gx.shape == (0, 2)
    assert torch.count_nonzero(gp) == 0


def test_backward_rejects_bad_upstream_gradients() -> None:
    announce("backward rejects bad upstream gradients")
    from fused_hoad import _C

    p = packed(0)
    x = coordinates(8)
    good = torch.zeros(8, device="cuda")
    with pytest.raises(RuntimeError, match=r"\[batch\] values"):
        _C.fused_forward_laplacian_backward(x, p, torch.zeros(7, device="cuda"), good)
    with pytest.raises(RuntimeError, match="float32"):
        _C.fused_forward_laplacian_backward(x, p, good.double(), good)
    with pytest.raises(RuntimeError, match="version"):
        _C.fused_forward_laplacian_backward(x, p, good, good, 0)
