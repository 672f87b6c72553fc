"""HIP-graph replay of the PyTorch backends (``*_cudagraph``), as in the reference's
test_backends.py:90-101: a replay must read freshly copied coordinates, not the ones seen at
capture. Each replay is checked against the same backend run eagerly on the same inputs, with
eager work and synchronisations between replays; also across an in-place weight update (the
graph reads the weights at every replay) and a new batch size (a new capture)."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import announce

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible GPU")


@pytest.mark.parametrize("name", ["eager_cudagraph", "forward_laplacian_cudagraph"])
def test_graph_replay_uses_new_coordinates_and_weights(name: str) -> None:
    from fused_hoad import DEFAULT_POISSON_MLP, build_mlp, get_backend

    base = get_backend(name.removesuffix("_cudagraph"))
    run = get_backend(name)
    torch.manual_seed(0)
    model = build_mlp(DEFAULT_POISSON_MLP).to(device="cuda", dtype=torch.float64)
    gen = torch.Generator(device="cuda").manual_seed(1)

    def check(batch: int, what: str) -> None:
        announce(f"{name}: {what}, batch={batch}")
        x = torch.rand(batch, 2, device="cuda", dtype=torch.float64, generator=gen) * 2 - 1
        u, lap = run(model, x)
        u, lap = u.clone(), lap.clone()
        torch.cuda.synchronize()
        eu, el = base(model, x)
        torch.testing.assert_close(u, eu.detach(), atol=1e-12, rtol=1e-10)
        torch.testing.assert_close(lap, el.detach(), atol=1e-10, rtol=1e-8)

    check(96, "capture")
    for i in range(3):
        check(96, f"replay {i}")
    with torch.no_grad():
        model[0].weight.mul_(0.9)
        model[-1].bias.add_(0.25)
    check(96, "replay after an in-place weight update")
    check(40, "new batch size (new capture)")
    check(40, "replay at the new size")
    # the replay returns the graph's own buffers
    x = torch.zeros(40, 2, device="cuda", dtype=torch.float64)
    assert run(model, x)[1].data_ptr() == run(model, x + 0.5)[1].data_ptr()
