"""GPU parity of the saved-layer pair: fhoad_forward_laplacian_saving keeps the hidden layers'
outputs, fhoad_forward_laplacian_backward_saved reads them instead of re-running the forward.

Both are pinned to entry points the other GPU tests pin against the oracle: the saving
forward's u and Laplacian must be bitwise those of the forward, and the saved-layer backward's
parameter and coordinate gradients bitwise those of the backward that re-runs the forward. The
sizes cover every path: the small-batch kernels (which re-run the forward either way), whole
rounds of 64-point tiles, a last 64-point tile whose later waves hold no points (zeros are read
for them), split 16-point tiles past the last whole round, the forward's split rest tiles and
8-wave workgroups, and saturated weights.
"""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import announce, coordinates, knobs, packed, require_gpu_extension, upstream

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _extension():
    return require_gpu_extension()


def _saving_forward(x, p):
    from fused_hoad import _C

    return _C._forward_saving(x, p, 2)


@pytest.mark.parametrize(
    "batch,waves",
    [(1, None), (17, None), (1000, None), (8192, None), (16401, None), (65536, None),
     (65537, None), (70000, None), (81904, None), (262145, None), (65536, "12"), (70000, "12"),
     (70000, "8")],
)
def test_saving_forward_is_bitwise_the_forward(batch: int, waves: str | None) -> None:
    """waves None: each forward with its default workgroup (12 waves plain, 8 saving); else both
    forced to that many waves."""
    announce(f"saving forward vs forward, batch={batch}, waves={waves or 'default'}")
    from fused_hoad import fused_forward_laplacian

    p = packed(0)
    x = coordinates(batch, seed=41)
    with knobs(**({} if waves is None else {"FUSED_HOAD_FWD_WAVES": waves})):
        u, lap = fused_forward_laplacian(x, p, 2)
        su, slap, saved = _saving_forward(x, p)
    torch.cuda.synchronize()
    assert saved.numel() == -(-batch // 16) * 49152
    assert torch.equal(su, u) and torch.equal(slap, lap)


@pytest.mark.parametrize(
    "batch,scale,coordinate_grad",
    [(1, 1.0, True), (1000, 1.0, True), (12288, 1.0, True), (12289, 1.0, True),
     (16384, 1.0, False), (65500, 1.0, True), (65536, 1.0, True), (65536, 3.0, True),
     (70001, 1.0, True), (262144, 1.0, False)],
)
def test_saved_backward_is_bitwise_the_backward(batch: int, scale: float, coordinate_grad: bool) -> None:
    """65,500 points: the last 64-point tile holds 28 points, so its waves 2 and 3 have no
    16-point tile in the saved buffer and read zeros. 70,001: whole rounds plus split tiles,
    which re-run the forward. 12,288 and below: the small-batch kernel."""
    announce(f"saved-layer backward vs backward, batch={batch}, weights x{scale}, coordinate grad={coordinate_grad}")
    from fused_hoad import _C

    p = packed(1, scale)
    x = coordinates(batch, seed=42)
    gu, gl = upstream(batch, seed=42)
    gu, gl = gu.reshape(-1).contiguous(), gl.reshape(-1).contiguous()
    _, _, saved = _saving_forward(x, p)
    want_p, want_x = _C._backward(x, p, gu, gl, coordinate_grad, 6)
    got_p, got_x = _C._backward(x, p, gu, gl, coordinate_grad, 6, saved)
    torch.cuda.synchronize()
    assert torch.equal(got_p, want_p)
    if coordinate_grad:
        assert torch.equal(got_x, want_x)
    else:
        assert got_x is None


def test_saved_backward_with_one_upstream_gradient() -> None:
    """A loss on the Laplacian only: grad_output None (read as zeros by the kernel)."""
    announce("saved-layer backward, Laplacian-only upstream, batch=65536")
    from fused_hoad import _C

    p = packed(2)
    x = coordinates(65536, seed=43)
    _, gl = upstream(65536, seed=43)
    gl = gl.reshape(-1).contiguous()
    _, _, saved = _saving_forward(x, p)
    want_p, want_x = _C._backward(x, p, None, gl, True, 6)
    got_p, got_x = _C._backward(x, p, None, gl, True, 6, saved)
    torch.cuda.synchronize()
    assert torch.equal(got_p, want_p) and torch.equal(got_x, want_x)


def test_saved_layers_must_cover_the_batch() -> None:
    announce("saved-layer backward rejects a buffer that does not cover the batch")
    from fused_hoad import _C

    p = packed(0)
    x = coordinates(1000, seed=44)
    gu, gl = upstream(1000, seed=44)
    _, _, saved = _saving_forward(x[:500], p)
    with pytest.raises(RuntimeError, match="saved layers do not cover the batch"):
        _C._backward(x, p, gu.reshape(-1), gl.reshape(-1), True, 6, saved)


@pytest.mark.parametrize("flatten", [False, True])
@pytest.mark.parametrize("coordinate_grad", [False, True])
def test_saved_mode_gradients_equal_the_cuda_mode(flatten: bool, coordinate_grad: bool) -> None:
    """fused_laplacian(..., backward="saved") through autograd: every parameter's gradient and
    the coordinate gradient bitwise those of backward="cuda", for the packed and the flattened
    autograd paths."""
    announce(f"autograd backward='saved' vs 'cuda', flatten={flatten}, coordinate grad={coordinate_grad}")
    from fused_hoad import DEFAULT_POISSON_MLP, build_mlp, manufactured_source
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.parameters import flatten_poisson_parameters_

    x0 = coordinates(20000, seed=45)
    f = manufactured_source(x0)

    def run(mode: str):
        torch.manual_seed(6)
        model = build_mlp(DEFAULT_POISSON_MLP).cuda()
        if flatten:
            flatten_poisson_parameters_(model)
        x = x0.clone().requires_grad_(coordinate_grad)
        u, lap = fused_laplacian(model, x, backward=mode)
        ((lap - f).pow(2).mean() + 0.1 * u.pow(2).mean()).backward()
        return [q.grad for q in model.parameters()], x.grad

    want, want_x = run("cuda")
    got, got_x = run("saved")
    torch.cuda.synchronize()
    for index, (a, b) in enumerate(zip(got, want, strict=True)):
        assert torch.equal(a, b), f"parameter {index}"
    if coordinate_grad:
        assert torch.equal(got_x, want_x)
