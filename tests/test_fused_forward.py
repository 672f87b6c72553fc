"""GPU parity of the gfx950 forward kernel (through fused_hoad._C and the C ABI).

Tolerances: against the PyTorch forward Laplacian in FP32 (oracle/torch_ref.py, the
reference's forward_laplacian.py restated) atol 1e-5 / rtol 1e-4, the north star's bar and
the reference's test_fused.py:27-35; against the float64 oracle with saturating weights
max |error| <= 1e-4 max |expected| (test_fused.py:38-49).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_cases import CASE_NAMES, load_case
from gpu_helpers import announce, coordinates, knobs, packed, require_gpu_extension, to_numpy64
from oracle import jet, torch_ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _extension():
    return require_gpu_extension()


def _fused(x, p, version=2):
    from fused_hoad import fused_forward_laplacian

    return fused_forward_laplacian(x, p, version)


# the reference's tile edges (test_fused.py:28) plus this kernel's: 16-point wave tiles, and
# ragged large batches (a partial last tile, workgroups with unequal tile counts); 1,024 and
# 16,384 are BASELINE.json configs 1 and 2
@pytest.mark.parametrize(
    "batch",
    [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 1000, 1024, 4097, 16384, 16401, 65536, 65537,
     70000, 100000, 262145],
)
def test_forward_matches_torch_forward_laplacian(batch: int) -> None:
    announce(f"forward vs torch forward Laplacian, batch={batch}")
    p = packed(0)
    x = coordinates(batch, seed=batch)
    eu, el = torch_ref.forward_laplacian(p, x)
    u, lap = _fused(x, p)
    assert u.shape == lap.shape == (batch, 1)
    torch.testing.assert_close(u, eu, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(lap, el, atol=1e-5, rtol=1e-4)


def test_forward_matches_float64_oracle_with_saturated_tanh() -> None:
    announce("forward vs float64 oracle, weights x3, batch=4096")
    p = packed(1, 3.0)
    x = coordinates(4096, seed=1)
    eu, el = jet.forward(to_numpy64(p), to_numpy64(x))
    u, lap = _fused(x, p)
    for got, want in ((u, eu), (lap, el)):
        err = np.abs(to_numpy64(got).ravel() - want).max()
        assert err <= 1e-4 * np.abs(want).max(), err


@pytest.mark.parametrize("name", CASE_NAMES)
def test_forward_matches_golden_fixture(name: str) -> None:
    announce(f"forward vs golden fixture {name}")
    case = load_case(name)
    p = torch.from_numpy(case["parameters"]).cuda()
    x = torch.from_numpy(case["coordinates"]).cuda()
    u, lap = _fused(x, p)
    np.testing.assert_allclose(to_numpy64(u).ravel(), case["u"], atol=1e-5, rtol=1e-4)
    np.testing.assert_allclose(to_numpy64(lap).ravel(), case["laplacian"], atol=1e-5, rtol=1e-4)


def test_forward_large_batch_matches_torch() -> None:
    announce("forward vs torch forward Laplacian, batch=1048576")
    p = packed(0)
    x = coordinates(1 << 20, seed=3)
    u, lap = _fused(x, p)
    eu, el = torch_ref.forward_laplacian(p, x)
    torch.testing.assert_close(u, eu, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(lap, el, atol=1e-5, rtol=1e-4)


def test_forward_is_bitwise_reproducible_and_version_independent() -> None:
    announce("forward determinism and versions 0..5, batch=65536")
    p = packed(0)
    x = coordinates(65536, seed=5)
    first = _fused(x, p)
    for version in range(6):
        again = _fused(x, p, version)
        assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])


@pytest.mark.parametrize("batch", [1000, 65536])
def test_forward_workgroup_shape_does_not_change_results(batch: int) -> None:
    """12 waves per workgroup (default) and 8 (FUSED_HOAD_FWD_WAVES=8) only distribute tiles
    differently; every tile's arithmetic is the same, so the outputs are bitwise equal."""
    announce(f"forward 12-wave vs 8-wave workgroups, batch={batch}")
    p = packed(0)
    x = coordinates(batch, seed=17)
    with knobs(FUSED_HOAD_FWD_SPLIT="0"):
        u12, l12 = _fused(x, p)
        with knobs(FUSED_HOAD_FWD_WAVES="8"):
            u8, l8 = _fused(x, p)
    torch.cuda.synchronize()
    assert torch.equal(u12, u8) and torch.equal(l12, l8)


@pytest.mark.parametrize(
    "batch,scale",
    [(1, 1.0), (15, 1.0), (16, 1.0), (17, 1.0), (1000, 1.0), (4096, 1.0), (8192, 3.0), (20000, 1.0)],
)
def test_split_forward_is_bitwise_equal_to_the_tiled_kernel(batch: int, scale: float) -> None:
    """The small-batch kernel (one tile over a workgroup's 4 waves, rows split by wave) runs
    the tiled kernel's MFMA chains and tanh updates in the same order, so the outputs are
    bitwise equal; 20000 points force several tiles per workgroup through its exchange
    buffers, and scale 3 saturates the tanh."""
    announce(f"forward split kernel vs tiled kernel, batch={batch}, weights x{scale}")
    p = packed(0) * scale
    x = coordinates(batch, seed=23)
    with knobs(FUSED_HOAD_FWD_SPLIT="0"):
        u_tiled, l_tiled = _fused(x, p)
    with knobs(FUSED_HOAD_FWD_SPLIT="1"):
        u_split, l_split = _fused(x, p)
    torch.cuda.synchronize()
    assert torch.equal(u_tiled, u_split) and torch.equal(l_tiled, l_split)


@pytest.mark.parametrize(
    "batch,scale,waves",
    [(16401, 1.0, "12"), (65537, 1.0, "12"), (70000, 3.0, "12"), (100000, 1.0, "12"),
     (262145, 1.0, "12"), (70000, 1.0, "8"), (81904, 1.0, "12"), (81904, 3.0, "8")],
)
def test_forward_split_rest_is_bitwise_equal_to_whole_tiles(batch: int, scale: float, waves: str) -> None:
    """Past the last whole round (one 16-point tile per SIMD), the tiled kernel runs the
    remaining tiles with their rows split over each workgroup's last four waves, which meet at
    an LDS counter; FUSED_HOAD_FWD_SPLIT_REST=0 runs them as whole tiles. The split tiles run
    the whole tiles' MFMA chains and tanh updates in the same order, so the outputs are bitwise
    equal. 16,401 points leave two split tiles after one round; 70,000 points put two split
    tiles on some workgroups (two passes through both exchange buffers); 81,904 points leave
    1,023 split tiles, four on all but one workgroup (twelve meetings a quad); scale 3
    saturates the tanh; 8-wave workgroups use waves 4-7 as the quad."""
    announce(f"forward split rest tiles vs whole tiles, batch={batch}, weights x{scale}, waves={waves}")
    p = packed(0) * scale
    x = coordinates(batch, seed=29)
    with knobs(FUSED_HOAD_FWD_WAVES=waves, FUSED_HOAD_FWD_SPLIT="0"):
        u_split, l_split = _fused(x, p)
        with knobs(FUSED_HOAD_FWD_SPLIT_REST="0"):
            u_whole, l_whole = _fused(x, p)
    torch.cuda.synchronize()
    assert torch.equal(u_split, u_whole) and torch.equal(l_split, l_whole)


def test_quad_meeting_timeout_is_reported_and_marks_its_tiles() -> None:
    """A split rest tile's four waves meet at an LDS counter with a bounded wait. With the test
    knob FUSED_HOAD_QUAD_SPIN_LIMIT=0 every meeting gives up at once (every kernel still runs to
    its end): the split tiles' u and Laplacian come back NaN, every whole tile's are bitwise the
    default ones, and _check_device raises once, naming the timeout, then passes again. With the
    default bound the status word stays clear and the outputs do not change."""
    from fused_hoad import _C

    batch = 70000  # 4,375 tiles: 279 split tiles past four whole rounds on 256 CUs
    announce(f"forward quad meeting timeout knob, batch={batch}")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = (batch + 15) // 16
    grid = min(tiles, cus)
    whole = tiles - tiles % (4 * grid) if tiles >= 4 * grid else tiles
    assert whole < tiles, "the batch must leave split tiles on this device"
    p = packed(0)
    x = coordinates(batch, seed=31)
    device = torch.device("cuda:0")
    _C._check_device(device)  # clear anything earlier
    with knobs(FUSED_HOAD_FWD_SPLIT="0"):
        u_ref, l_ref = _fused(x, p)
        _C._check_device(device)
        with knobs(FUSED_HOAD_QUAD_SPIN_LIMIT="0"):
            u, lap = _fused(x, p)
        with pytest.raises(RuntimeError, match="gave up waiting for its quad"):
            _C._check_device(device)
        _C._check_device(device)  # cleared by the check that reported it
        split = slice(whole * 16, batch)
        assert torch.isnan(u[split]).all() and torch.isnan(lap[split]).all()
        assert torch.equal(u[: whole * 16], u_ref[: whole * 16])
        assert torch.equal(lap[: whole * 16], l_ref[: whole * 16])
        u2, l2 = _fused(x, p)
        _C._check_device(device)
    assert torch.equal(u2, u_ref) and torch.equal(l2, l_ref)


def test_forward_handles_empty_batch() -> None:
    announce("forward, empty batch")
    u, lap = _fused(torch.empty(0, 2, device="cuda"), packed(0))
    assert u.shape == lap.shape == (0, 1)


@pytest.mark.parametrize(
    ("make", "message"),
    [
        (lambda: torch.zeros(4, 2, device="cuda", dtype=torch.float64), "float32"),
        (lambda: torch.zeros(4, 3, device="cuda"), r"\[batch, 2\]"),
        (lambda: torch.zeros(4, 2), "CUDA"),
        (lambda: torch.zeros(2, 4, device="cuda").t(), "contiguous"),
    ],
)
def test_forward_rejects_invalid_coordinates(make, message: str) -> None:
    announce(f"forward rejects invalid coordinates ({message})")
    with pytest.raises(RuntimeError, match=message):
        _fused(make(), packed(0))


def test_forward_rejects_bad_parameters_and_version() -> None:
    announce("forward rejects bad parameters / version")
    x = torch.zeros(4, 2, device="cuda")
    with pytest.raises(RuntimeError, match="version"):
        _fused(x, packed(0), 7)
    with pytest.raises(RuntimeError, match=r"\[12737\]"):
        _fused(x, torch.zeros(12736, device="cuda"))


def test_backend_repacks_after_in_place_weight_update() -> None:
    announce("fused_cuda backend repacks after an in-place update")
    from fused_hoad import DEFAULT_POISSON_MLP, build_mlp, forward_laplacian, get_backend

    torch.manual_seed(0)
    model = build_mlp(DEFAULT_POISSON_MLP).cuda().requires_grad_(False)
    x = coordinates(256, seed=8)
    run = get_backend("fused_cuda")
    run(model, x)
    with torch.no_grad():
        model[0].weight.mul_(0.5)
    _, lap = run(model, x)
    _, expected = forward_laplacian(model, x)
    torch.testing.assert_close(lap, expected, atol=1e-5, rtol=1e-4)
