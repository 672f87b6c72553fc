"""A packed parameter buffer that is only 4-byte aligned (a view into a larger tensor, as a
caller's flat optimizer buffer may be) takes the kernels' scalar load paths; the loaded values
are the same, so every result is bitwise equal to the 16-byte-aligned run."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import announce, coordinates, packed, require_gpu_extension, upstream

pytestmark = pytest.mark.gpu


def _misaligned_copy(p: torch.Tensor) -> torch.Tensor:
    big = torch.zeros(p.numel() + 1, device=p.device)
    view = big[1:]
    view.copy_(p)
    assert view.data_ptr() % 16 == 4 and view.is_contiguous()
    return view


@pytest.mark.parametrize("batch", [5000, 40000])
def test_forward_and_backward_with_a_misaligned_parameter_buffer(batch: int) -> None:
    """5000 points run the small-batch forward kernel, 40000 the tiled one."""
    require_gpu_extension()
    announce(f"misaligned parameters: forward + backward vs aligned, batch={batch}")
    from fused_hoad._extension import fused_forward_laplacian, fused_forward_laplacian_backward

    p = packed(0)
    q = _misaligned_copy(p)
    x = coordinates(batch, seed=21)
    gu, gl = upstream(batch, seed=21)
    for a, b in zip(fused_forward_laplacian(x, p), fused_forward_laplacian(x, q)):
        assert torch.equal(a, b)
    for a, b in zip(fused_forward_laplacian_backward(x, p, gu, gl), fused_forward_laplacian_backward(x, q, gu, gl)):
        assert torch.equal(a, b)


def test_fused_step_with_a_misaligned_parameter_buffer() -> None:
    require_gpu_extension()
    announce("misaligned parameters: fused Poisson+Adam step vs aligned, 3 steps, batch=3000")
    from fused_hoad import _C, manufactured_source

    x = coordinates(3000, seed=22)
    f = manufactured_source(x).reshape(-1).contiguous()
    runs = []
    for params in (packed(0), _misaligned_copy(packed(0))):
        m, v, t = torch.zeros(12737, device="cuda"), torch.zeros(12737, device="cuda"), torch.zeros(1, device="cuda")
        losses = [_C.poisson_adam_step(x, f, params, m, v, t, 1e-3, 0.9, 0.999, 1e-8, 0.0) for _ in range(3)]
        runs.append((torch.stack(losses), params.clone(), m.clone(), v.clone()))
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)
