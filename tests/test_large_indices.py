"""Batches past 2^31 points (the reference's "maximum sizes" edge case; its kernels take the
batch as int64, /root/reference/csrc/fused_residual.cu:587-643 and fused_backward.cu:859-934).

Every point, tile and coordinate index in the kernels and the host code is 64-bit. One ragged
batch of 2^31 + 4,099 points is run through the forward (about 35 GB on the device) and the
backward (about 52 GB); points past index 2^31, and a window across it, are checked against
separate small calls on the same points:
* the forward is lane-local per point, so the big call must give bitwise the small call's
  u and Laplacian;
* the backward gets upstream gradients that are zero except at three points past 2^31 (in
  three different slots), so its parameter gradient is those three points' gradient, summed in
  another order than the small call sums it (1e-5 of each block's scale), and its coordinate
  gradient is zero everywhere else;
* the fused training step (lr 0, so the weights stay put) with a random source term: its loss
  against a float64 sum of (lap - f)^2 over the forward's Laplacian, and its gradient against
  the backward call seeded with grad_lap = 2 (lap - f) / B (the same tiles and slots).
"""

from __future__ import annotations

import pytest
import torch

from conftest import assert_scaled_close
from gpu_helpers import announce, packed, require_gpu_extension

pytestmark = pytest.mark.gpu

# The ten weight and bias blocks of the packed parameters (mlp_abi layout).
BLOCKS = [
    ("layer0.weight", 0, 128), ("layer0.bias", 128, 192),
    ("layer1.weight", 192, 4288), ("layer1.bias", 4288, 4352),
    ("layer2.weight", 4352, 8448), ("layer2.bias", 8448, 8512),
    ("layer3.weight", 8512, 12608), ("layer3.bias", 12608, 12672),
    ("layer4.weight", 12672, 12736), ("layer4.bias", 12736, 12737),
]

TWO_31 = 1 << 31
BIG = TWO_31 + 4099  # ragged: 4,099 points past 2^31, not a whole number of tiles


@pytest.fixture(scope="module", autouse=True)
def _extension():
    require_gpu_extension()
    yield
    torch.cuda.empty_cache()  # return the tens of GB to the device for the tests that follow


def _big_coordinates() -> torch.Tensor:
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = torch.rand(BIG, 2, device="cuda", generator=gen)
    return x.mul_(2.0).sub_(1.0)


def test_forward_past_two_to_the_31_points() -> None:
    from fused_hoad._extension import fused_forward_laplacian

    announce(f"forward, batch={BIG} (2^31 + 4099), windows checked against small calls")
    p = packed(0)
    x = _big_coordinates()
    u, lap = fused_forward_laplacian(x, p)
    assert u.shape == lap.shape == (BIG, 1)
    for lo, hi in ((BIG - 4099, BIG), (TWO_31 - 64, TWO_31 + 64), (0, 1000)):
        su, sl = fused_forward_laplacian(x[lo:hi].contiguous(), p)
        assert torch.equal(u[lo:hi], su), f"u differs in [{lo}, {hi})"
        assert torch.equal(lap[lo:hi], sl), f"laplacian differs in [{lo}, {hi})"
    del x, u, lap
    torch.cuda.empty_cache()


def test_backward_past_two_to_the_31_points() -> None:
    from fused_hoad._extension import fused_forward_laplacian_backward

    announce(f"backward, batch={BIG} (2^31 + 4099), three seeded points past 2^31")
    p = packed(0)
    x = _big_coordinates()
    gu = torch.zeros(BIG, device="cuda")
    gl = torch.zeros(BIG, device="cuda")
    idx = torch.tensor([TWO_31 + 5, TWO_31 + 3000, BIG - 1], device="cuda")
    gu[idx] = torch.tensor([0.5, -1.0, 0.25], device="cuda")
    gl[idx] = torch.tensor([1.0, 0.5, -2.0], device="cuda")
    gp, gx = fused_forward_laplacian_backward(x, p, gu, gl)
    assert gp.shape == (12737,) and gx.shape == (BIG, 2)
    sp, sx = fused_forward_laplacian_backward(
        x[idx].contiguous(), p, gu[idx].contiguous(), gl[idx].contiguous()
    )
    for name, lo, hi in BLOCKS:
        assert_scaled_close(gp[lo:hi], sp[lo:hi], 1e-5, name)
    assert_scaled_close(gx[idx], sx, 1e-5, "grad_coordinates at the seeded points")
    assert int(torch.count_nonzero(gx)) <= 6, "grad_coordinates must be zero at unseeded points"
    del x, gu, gl, gx
    torch.cuda.empty_cache()


def test_fused_step_past_two_to_the_31_points() -> None:
    from fused_hoad import DEFAULT_POISSON_MLP, build_mlp
    from fused_hoad._extension import fused_forward_laplacian, fused_forward_laplacian_backward
    from fused_hoad.training import FusedPoissonAdam

    announce(f"fused step, batch={BIG} (2^31 + 4099), random source, lr 0")
    x = _big_coordinates()
    gen = torch.Generator(device="cuda").manual_seed(8)
    f = torch.rand(BIG, device="cuda", generator=gen)
    torch.manual_seed(0)
    model = build_mlp(DEFAULT_POISSON_MLP).cuda()
    trainer = FusedPoissonAdam(model, x, f, lr=0.0)
    p = trainer.parameters.clone()
    loss = float(trainer.step())
    assert torch.equal(trainer.parameters, p), "lr 0 must leave the parameters unchanged"
    _, lap = fused_forward_laplacian(x, p)
    lap = lap.reshape(-1)
    want = 0.0
    for lo in range(0, BIG, 1 << 28):
        r = lap[lo : lo + (1 << 28)].double() - f[lo : lo + (1 << 28)].double()
        want += float((r * r).sum())
    want /= BIG
    assert abs(loss - want) <= 1e-4 * want, f"loss {loss} vs {want}"
    gl = (lap - f) * (2.0 / BIG)
    del lap
    gp, _ = fused_forward_laplacian_backward(x, p, torch.zeros_like(gl), gl)
    for name, lo, hi in BLOCKS:
        assert_scaled_close(trainer.grad[lo:hi], gp[lo:hi], 1e-6, name)
    del x, f, trainer, gl, gp
    torch.cuda.empty_cache()
