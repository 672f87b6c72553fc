"""The fused kernels inside PyTorch training (autograd.Function, pack cache, Adam, graph
capture), as in the reference's test_fused.py:98-159 and 233-262, plus the large-batch
training config (262,144 points, 100 Adam steps, deterministic gradients)."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import announce, coordinates, require_gpu_extension

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _extension():
    return require_gpu_extension()


def _model(seed: int = 0):
    from fused_hoad import DEFAULT_POISSON_MLP, build_mlp

    torch.manual_seed(seed)
    return build_mlp(DEFAULT_POISSON_MLP).cuda()


def _poisson_loss(u, lap, x):
    from fused_hoad import manufactured_source

    return (lap - manufactured_source(x)).pow(2).mean() + 0.1 * u.pow(2).mean()


@pytest.mark.parametrize(
    "name",
    ["fused_cuda_v0", "fused_cuda_v1", "fused_cuda", "fused_cuda_bwd_v1", "fused_cuda_bwd_v3",
     "fused_cuda_bwd_v5", "fused_cuda_bwd_v4", "fused_cuda_bwd_v2", "fused_cuda_recompute"],
)
def test_fused_gradients_match_forward_laplacian(name: str) -> None:
    announce(f"full-loss gradients through autograd, backend={name}")
    from fused_hoad import forward_laplacian, get_backend

    model = _model()
    x0 = coordinates(4096, seed=1)

    def gradients(run):
        model.zero_grad()
        x = x0.clone().requires_grad_(True)
        _poisson_loss(*run(model, x), x0).backward()
        return [p.grad.clone() for p in model.parameters()] + [x.grad.clone()]

    expected = gradients(forward_laplacian)
    actual = gradients(get_backend(name))
    for got, want in zip(actual, expected, strict=True):
        torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize(
    "loss_kind,coordinate_grad,mode",
    [("lap", False, "cuda"), ("lap", True, "cuda"), ("u_and_lap", True, "cuda"),
     ("u", False, "cuda"), ("lap", True, "recompute")],
)
def test_flattened_model_gradients_equal_the_packed_path(loss_kind: str, coordinate_grad: bool,
                                                         mode: str) -> None:
    """A model flattened with flatten_poisson_parameters_ takes the no-pack autograd path
    (its parameters are the Function's inputs, their gradients views of the packed one, an
    unused output's gradient is read as zero without a zeros tensor, the coordinate gradient is
    skipped unless needed). Its gradients are bitwise those of an unflattened twin, whose
    parameters are packed on every call (by the C++ Function, or by the differentiable
    torch.cat of the recompute mode)."""
    announce(f"flattened vs packed autograd path, loss={loss_kind}, coordinate grad={coordinate_grad}, backward={mode}")
    from fused_hoad import manufactured_source
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.parameters import flatten_poisson_parameters_, flattened_poisson_parameters

    x0 = coordinates(5000, seed=31)
    f = manufactured_source(x0)

    def run(model):
        model.zero_grad(set_to_none=True)
        x = x0.clone().requires_grad_(coordinate_grad)
        u, lap = fused_laplacian(model, x, backward=mode)
        terms = {"lap": (lap - f).pow(2).mean(), "u": u.pow(2).mean()}
        loss = terms["lap"] + terms["u"] if loss_kind == "u_and_lap" else terms[loss_kind]
        loss.backward()
        grads = [p.grad for p in model.parameters()]
        return grads, (x.grad if coordinate_grad else None)

    packed_model = _model(4)
    flat_model = _model(4)
    flatten_poisson_parameters_(flat_model)
    assert flattened_poisson_parameters(flat_model) is not None
    want, want_x = run(packed_model)
    got, got_x = run(flat_model)
    torch.cuda.synchronize()
    for index, (a, b) in enumerate(zip(got, want, strict=True)):
        if b is None:  # a parameter the loss does not reach (b_out for a Laplacian-only loss)
            assert a is None or torch.count_nonzero(a).item() == 0, index
            continue
        assert torch.equal(a, b), f"parameter {index}"
    if coordinate_grad:
        assert torch.equal(got_x, want_x)


@pytest.mark.parametrize("mode", ["cuda", "saved", "recompute"])
def test_in_place_update_before_backward_raises_for_a_flattened_model(mode: str) -> None:
    """A flattened model's parameters are views of the packed buffer the kernels read. An
    optimizer step between the forward and a retain_graph backward changes the buffer without
    changing its version counter; the backward must refuse (PyTorch's in-place-modification
    error, as nn.Linear gives) instead of differentiating at the new weights. The first
    backward, before the step, is unaffected."""
    announce(f"in-place update between forward and backward, flattened model, backward={mode}")
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.parameters import flatten_poisson_parameters_

    model = _model(6)
    flatten_poisson_parameters_(model)
    optimizer = torch.optim.Adam(model.parameters(), lr=1e-3)
    _, lap = fused_laplacian(model, coordinates(512, seed=6), backward=mode)
    loss = lap.pow(2).mean()
    loss.backward(retain_graph=True)
    optimizer.step()
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        loss.backward()


@pytest.mark.parametrize("frozen_layers", [(0, 4), (0, 1, 2, 3, 4)])
@pytest.mark.parametrize("mode", ["cuda", "saved", "recompute"])
def test_flattened_model_with_frozen_layers(mode: str, frozen_layers: tuple[int, ...]) -> None:
    """Frozen layers (requires_grad False) on a flattened model get no gradient, and the
    trainable layers' gradients and the coordinate gradient are bitwise those of an unflattened
    twin frozen the same way (all layers frozen: only the coordinate gradient)."""
    announce(f"flattened model with frozen layers {frozen_layers}, backward={mode}")
    from fused_hoad import manufactured_source
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.parameters import flatten_poisson_parameters_

    x0 = coordinates(3000, seed=32)
    f = manufactured_source(x0)

    def run(flatten: bool):
        model = _model(6)
        if flatten:
            flatten_poisson_parameters_(model)
        for index in frozen_layers:
            model[2 * index].weight.requires_grad_(False)
            model[2 * index].bias.requires_grad_(False)
        x = x0.clone().requires_grad_(True)
        u, lap = fused_laplacian(model, x, backward=mode)
        ((lap - f).pow(2).mean() + 0.1 * u.pow(2).mean()).backward()
        return [p.grad for p in model.parameters()], x.grad

    want, want_x = run(False)
    got, got_x = run(True)
    torch.cuda.synchronize()
    for index, (a, b) in enumerate(zip(got, want, strict=True)):
        if index // 2 in frozen_layers:
            assert a is None and b is None, index
        else:
            assert torch.equal(a, b), f"parameter {index}"
    assert torch.equal(got_x, want_x)


def test_model_laplacian_function_checks_its_parameters() -> None:
    """The C++ autograd Function behind fused_laplacian: the parameters must have the layout's
    shapes and, with a packed buffer given, be its views; without one it packs them itself."""
    announce("C++ autograd Function: parameter checks, packed and unpacked forms")
    from fused_hoad import _C, fused_forward_laplacian, pack_poisson_parameters
    from fused_hoad.parameters import flatten_poisson_parameters_, flattened_poisson_binding

    model = _model(7)
    flatten_poisson_parameters_(model)
    flat, tensors = flattened_poisson_binding(model)
    x = coordinates(100, seed=33)
    with pytest.raises(RuntimeError, match="must have the shape of layout slice 0"):
        _C._model_laplacian(x, flat, 2, 6, False, [tensors[2], *tensors[1:]])
    with pytest.raises(RuntimeError, match="parameter 3 is not the packed buffer's view"):
        _C._model_laplacian(x, flat, 2, 6, False, [*tensors[:3], tensors[3].clone(), *tensors[4:]])
    with pytest.raises(RuntimeError, match="expected the model's 10 parameters"):
        _C._model_laplacian(x, flat, 2, 6, False, tensors[:9])
    u, lap = _C._model_laplacian(x, flat, 2, 6, False, tensors)
    ref_u, ref_lap = fused_forward_laplacian(x, flat, 2)
    twin = _model(7)
    packed_u, packed_lap = _C._model_laplacian(x, None, 2, 6, False, list(twin.parameters()))
    torch.cuda.synchronize()
    assert torch.equal(pack_poisson_parameters(twin), flat)
    assert torch.equal(u, ref_u) and torch.equal(lap, ref_lap)
    assert torch.equal(packed_u, ref_u) and torch.equal(packed_lap, ref_lap)


@pytest.mark.parametrize("mode", ["cuda", "saved", "recompute"])
def test_public_python_function_equals_fused_laplacian(mode: str) -> None:
    """FusedForwardLaplacian, the reference's public autograd Function over a packed buffer,
    called directly on a differentiable pack: the same u, Laplacian and gradients, bitwise, as
    fused_laplacian (whose "cuda" and "saved" modes run the C++ Function)."""
    announce(f"FusedForwardLaplacian.apply vs fused_laplacian, backward={mode}")
    from fused_hoad import manufactured_source, pack_poisson_parameters
    from fused_hoad.backends.fused import FusedForwardLaplacian, fused_laplacian

    x0 = coordinates(2500, seed=34)
    f = manufactured_source(x0)

    def run(direct: bool):
        model = _model(8)
        x = x0.clone().requires_grad_(True)
        if direct:
            u, lap = FusedForwardLaplacian.apply(x, pack_poisson_parameters(model, differentiable=True), 2, mode)
        else:
            u, lap = fused_laplacian(model, x, backward=mode)
        ((lap - f).pow(2).mean() + 0.1 * u.pow(2).mean()).backward()
        return [u.detach(), lap.detach(), x.grad] + [p.grad for p in model.parameters()]

    want, got = run(False), run(True)
    torch.cuda.synchronize()
    for index, (a, b) in enumerate(zip(got, want, strict=True)):
        assert torch.equal(a, b), index


@pytest.mark.parametrize("flatten", [False, True])
@pytest.mark.parametrize("mode", ["cuda", "saved"])
def test_retained_graph_and_two_calls_accumulate(mode: str, flatten: bool) -> None:
    """The C++ autograd Function's saved state and gradient views under accumulation:
    * backward twice through one graph (retain_graph=True) gives each gradient twice its
      single-backward value, bitwise (g + g = 2 g in float32);
    * one loss over two calls on the same model (two Function nodes, each handing the
      parameters views of its own packed gradient) gives the sum of the two calls' gradients,
      taken separately, bitwise (one float32 addition per entry, which commutes)."""
    announce(f"retain_graph twice and two calls in one loss, backward={mode}, flattened={flatten}")
    from fused_hoad import manufactured_source
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.parameters import flatten_poisson_parameters_

    xa, xb = coordinates(1500, seed=35), coordinates(2600, seed=36)
    fa, fb = manufactured_source(xa), manufactured_source(xb)

    def model():
        m = _model(9)
        if flatten:
            flatten_poisson_parameters_(m)
        return m

    def loss(m, x, f):
        u, lap = fused_laplacian(m, x, backward=mode)
        return (lap - f).pow(2).mean() + 0.1 * u.pow(2).mean()

    def grads(m, *extra):
        return [p.grad.clone() for p in m.parameters()] + [t.grad.clone() for t in extra]

    once = model()
    xg = xa.clone().requires_grad_(True)
    loss(once, xg, fa).backward()
    single = grads(once, xg)
    twice = model()
    xg2 = xa.clone().requires_grad_(True)
    value = loss(twice, xg2, fa)
    value.backward(retain_graph=True)
    value.backward()
    doubled = grads(twice, xg2)

    separate = []
    for x, f in ((xa, fa), (xb, fb)):
        m = model()
        loss(m, x, f).backward()
        separate.append(grads(m))
    both = model()
    (loss(both, xa, fa) + loss(both, xb, fb)).backward()
    summed = grads(both)
    torch.cuda.synchronize()
    for index, (a, b) in enumerate(zip(doubled, single, strict=True)):
        assert torch.equal(a, 2 * b), f"retain_graph: gradient {index}"
    for index, (a, b, c) in enumerate(zip(summed, *separate, strict=True)):
        assert torch.equal(a, b + c), f"two calls: gradient {index}"


def test_fused_trains_like_forward_laplacian() -> None:
    announce("50 Adam steps, fused vs forward_laplacian, batch=2048")
    from fused_hoad import forward_laplacian, get_backend

    x = coordinates(2048, seed=2)

    def train(run):
        model = _model()
        opt = torch.optim.Adam(model.parameters(), lr=1e-3)
        losses = []
        for _ in range(50):
            opt.zero_grad()
            loss = _poisson_loss(*run(model, x), x)
            loss.backward()
            opt.step()
            losses.append(loss.item())
        return losses

    fused = train(get_backend("fused_cuda"))
    reference = train(forward_laplacian)
    assert fused[-1] < 0.5 * fused[0]
    torch.testing.assert_close(torch.tensor(fused), torch.tensor(reference), rtol=1e-3, atol=0)


def test_inference_path_stays_out_of_autograd() -> None:
    announce("no_grad fused call")
    from fused_hoad import get_backend

    model = _model()
    with torch.no_grad():
        u, lap = get_backend("fused_cuda")(model, torch.zeros(8, 2, device="cuda"))
    assert not u.requires_grad and not lap.requires_grad


def test_graph_captured_training_step_matches_eager_step() -> None:
    announce("whole-step graph capture vs eager steps, batch=2048")
    from fused_hoad import get_backend
    from fused_hoad.training import cuda_graph_step

    x = coordinates(2048, seed=3)
    run = get_backend("fused_cuda")

    def train(graph: bool):
        model = _model()
        opt = torch.optim.Adam(model.parameters(), lr=1e-3, capturable=graph)

        def loss_fn():
            return _poisson_loss(*run(model, x), x)

        if graph:
            step = cuda_graph_step(loss_fn, opt, warmup=3)
            return [step().item() for _ in range(20)]  # every replay checked, host sync between
        losses = []
        for _ in range(23):
            opt.zero_grad(set_to_none=True)
            loss = loss_fn()
            loss.backward()
            opt.step()
            losses.append(loss.item())
        return losses[3:]

    torch.testing.assert_close(torch.tensor(train(True)), torch.tensor(train(False)), rtol=1e-4, atol=0)


@pytest.mark.parametrize("mode", ["cuda", "saved"])
def test_graph_captured_flattened_step_matches_eager_at_64k(mode: str) -> None:
    """The drop-in step bench.py times as train_step_autograd_graphed_ms (and, with
    backward="saved", as ..._saved_ms): a flattened model at 65,536 points (BASELINE config 3's
    size, where torch's mean reduces over many blocks), captured whole and replayed 10 times
    with a host sync between replays, against the same steps run eagerly: every replay's loss
    (rtol 1e-4) and the weights after."""
    announce(f"whole-step graph capture vs eager, flattened model, batch=65536, backward={mode}")
    from fused_hoad import manufactured_source
    from fused_hoad.backends.fused import fused_laplacian
    from fused_hoad.parameters import flatten_poisson_parameters_
    from fused_hoad.training import cuda_graph_step

    x = coordinates(65536, seed=8)
    f = manufactured_source(x)

    def make():
        model = _model(5)
        flatten_poisson_parameters_(model)
        return model

    def loss_of(model):
        def loss_fn():
            _, lap = fused_laplacian(model, x, backward=mode)
            return (lap - f).pow(2).mean()
        return loss_fn

    graph_model, eager_model = make(), make()
    graph_opt = torch.optim.Adam(graph_model.parameters(), lr=1e-3, capturable=True)
    eager_opt = torch.optim.Adam(eager_model.parameters(), lr=1e-3)
    replay = cuda_graph_step(loss_of(graph_model), graph_opt, warmup=3)
    eager_loss = loss_of(eager_model)
    got, want = [], []
    for k in range(13):
        eager_opt.zero_grad(set_to_none=True)
        loss = eager_loss()
        loss.backward()
        eager_opt.step()
        if k >= 3:
            got.append(replay().item())
            want.append(loss.item())
    torch.testing.assert_close(torch.tensor(got), torch.tensor(want), rtol=1e-4, atol=0)
    for a, b in zip(graph_model.parameters(), eager_model.parameters(), strict=True):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-6)


def _poisson_step_losses(batch: int, steps: int, backward: str):
    from fused_hoad import manufactured_source
    from fused_hoad.backends.fused import fused_laplacian

    model = _model()
    opt = torch.optim.Adam(model.parameters(), lr=1e-3)
    x = coordinates(batch, seed=7)
    f = manufactured_source(x)
    losses, first_grads = [], None
    for step in range(steps):
        opt.zero_grad(set_to_none=True)
        _, lap = fused_laplacian(model, x, backward=backward)
        loss = (lap - f).pow(2).mean()
        loss.backward()
        if step == 0:
            first_grads = [p.grad.clone() for p in model.parameters()]
        opt.step()
        losses.append(loss.item())
    return losses, first_grads


def test_large_batch_training_is_deterministic_and_tracks_recompute() -> None:
    announce("262144 points, 100 Adam steps: determinism and loss curve vs recompute")
    losses_a, grads_a = _poisson_step_losses(262144, 100, "cuda")
    losses_b, grads_b = _poisson_step_losses(262144, 100, "cuda")
    assert losses_a == losses_b
    for a, b in zip(grads_a, grads_b, strict=True):
        assert torch.equal(a, b)
    reference, _ = _poisson_step_losses(262144, 100, "recompute")
    assert losses_a[-1] < losses_a[0]
    torch.testing.assert_close(torch.tensor(losses_a), torch.tensor(reference), rtol=1e-3, atol=0)
