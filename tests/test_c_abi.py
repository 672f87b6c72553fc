"""The C ABI (include/fused_hoad.h) of libfused_hoad_hip.so, called directly through ctypes.

CPU part: the library loads, exports every function the header declares, and rejects bad
arguments before touching a device. GPU part: the raw entry points, driven with device
pointers and the current stream, give bitwise the same results as fused_hoad._C.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fused_hoad.h"
LIBRARY = ROOT / "expanded-gpu-optimization_amd" / "fused_hoad" / "libfused_hoad_hip.so"


def _lib() -> ctypes.CDLL:
    assert LIBRARY.exists(), f"{LIBRARY} is not built (run __graft_entry__.build())"
    lib = ctypes.CDLL(str(LIBRARY))
    lib.fhoad_abi_version.restype = ctypes.c_int
    lib.fhoad_parameter_count.restype = ctypes.c_int64
    lib.fhoad_status_string.restype = ctypes.c_char_p
    lib.fhoad_status_string.argtypes = [ctypes.c_int]
    lib.fhoad_last_error.restype = ctypes.c_char_p
    lib.fhoad_backward_workspace_size.restype = ctypes.c_size_t
    lib.fhoad_backward_workspace_size.argtypes = [ctypes.c_int64]
    vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.fhoad_forward_laplacian.restype = ci
    lib.fhoad_forward_laplacian.argtypes = [vp, vp, vp, vp, i64, ci, vp]
    lib.fhoad_forward_laplacian_backward.restype = ci
    lib.fhoad_forward_laplacian_backward.argtypes = [vp, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, i64, ci, vp]
    d = ctypes.c_double
    lib.fhoad_poisson_adam_step.restype = ci
    lib.fhoad_poisson_adam_step.argtypes = (
        [vp, vp, i64, vp, i64, d] + [vp] * 8 + [ctypes.c_size_t, d, d, d, d, d, vp]
    )
    lib.fhoad_poisson_adam_step_workspace_size.restype = ctypes.c_size_t
    lib.fhoad_poisson_adam_step_workspace_size.argtypes = [i64, i64]
    sz = ctypes.c_size_t
    lib.fhoad_saved_layers_size.restype = sz
    lib.fhoad_saved_layers_size.argtypes = [i64]
    lib.fhoad_forward_laplacian_saving.restype = ci
    lib.fhoad_forward_laplacian_saving.argtypes = [vp, vp, vp, vp, vp, sz, i64, ci, vp]
    lib.fhoad_forward_laplacian_backward_saved.restype = ci
    lib.fhoad_forward_laplacian_backward_saved.argtypes = [vp, vp, vp, sz, vp, vp, vp, vp, vp, sz, i64, ci, vp]
    return lib


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^[a-z_0-9 ]+\*?\s*(fhoad_[a-z_]+)\(", text, flags=re.MULTILINE)))


def test_header_declares_the_entry_points() -> None:
    assert _declared_functions() == [
        "fhoad_abi_version",
        "fhoad_backward_workspace_size",
        "fhoad_check_device",
        "fhoad_forward_laplacian",
        "fhoad_forward_laplacian_backward",
        "fhoad_forward_laplacian_backward_noalloc",
        "fhoad_forward_laplacian_backward_saved",
        "fhoad_forward_laplacian_saving",
        "fhoad_last_error",
        "fhoad_parameter_count",
        "fhoad_poisson_adam_step",
        "fhoad_poisson_adam_step_workspace_size",
        "fhoad_saved_layers_size",
        "fhoad_status_string",
    ]


def test_library_exports_every_declared_function() -> None:
    lib = _lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_constants_and_status_strings() -> None:
    lib = _lib()
    assert lib.fhoad_abi_version() == 1
    assert lib.fhoad_parameter_count() == 12737
    assert lib.fhoad_status_string(0) == b"success"
    assert lib.fhoad_status_string(4) == b"workspace too small"


def _expected_workspace(batch: int, boundary: int = 0) -> int:
    """Either gradient kernel may run (a knob can force either), so the workspace covers the
    larger slot count: 64-point interior tiles or 16-point tiles, plus 16-point boundary
    tiles, one partial row of 12,800 floats per slot, at most 256 slots."""
    row = 12800 * 4
    tiled = min(256, -(-batch // 64) - (-boundary // 16)) * row
    split = min(256, -(-batch // 16) - (-boundary // 16)) * row
    return max(tiled, split)


def test_workspace_size_covers_either_gradient_kernel() -> None:
    lib = _lib()
    assert lib.fhoad_backward_workspace_size(0) == 0
    per_slot = 12800 * 4
    assert lib.fhoad_backward_workspace_size(1) == per_slot
    assert lib.fhoad_backward_workspace_size(65536) == 256 * per_slot
    assert lib.fhoad_backward_workspace_size(1 << 20) == 256 * per_slot
    for batch in (1, 16, 17, 64, 65, 1000, 4096, 12288, 12289, 20000):
        assert lib.fhoad_backward_workspace_size(batch) == _expected_workspace(batch), batch
    assert lib.fhoad_poisson_adam_step_workspace_size(0, 5) == 0
    for batch, boundary in ((64, 0), (65, 1), (1000, 200), (16384, 1024), (12000, 300)):
        assert lib.fhoad_poisson_adam_step_workspace_size(batch, boundary) == _expected_workspace(
            batch, boundary
        ), (batch, boundary)


def test_argument_errors_are_reported_before_any_device_work() -> None:
    lib = _lib()
    assert lib.fhoad_forward_laplacian(None, None, None, None, 4, 7, None) == 1
    assert b"version must be 0 to 5" in lib.fhoad_last_error()
    assert lib.fhoad_forward_laplacian(None, None, None, None, -1, 2, None) == 2
    assert lib.fhoad_forward_laplacian(None, None, None, None, 0, 2, None) == 0
    assert lib.fhoad_forward_laplacian(None, None, None, None, 4, 2, None) == 2
    assert lib.fhoad_forward_laplacian_backward(None, None, None, None, None, None, None, 0, 4, 0, None) == 1
    assert b"backward version must be 1 to 6" in lib.fhoad_last_error()
    assert lib.fhoad_forward_laplacian_backward(None, None, None, None, None, None, None, 0, -3, 6, None) == 2
    step = lib.fhoad_poisson_adam_step
    adam = (1e-3, 0.9, 0.999, 1e-8, 0.0)

    def call(ptr, batch, boundary, count, weight, ws_bytes, *hyper):
        # coordinates, source, batch, boundary, count, weight, 7 state/output pointers, ws
        return step(ptr, ptr, batch, boundary, count, weight, *[ptr] * 5, None, None, ptr,
                    ws_bytes, *hyper, None)

    fake = ctypes.c_void_p(256)  # non-null, never dereferenced: the checks fail first
    assert call(None, 0, None, 0, 100.0, 0, *adam) == 2
    assert b"batch must be positive" in lib.fhoad_last_error()
    assert call(None, 16, None, 0, 100.0, 0, *adam) == 2
    assert b"null device pointer" in lib.fhoad_last_error()
    assert call(fake, 16, None, 5, 100.0, 1 << 30, *adam) == 2  # boundary points missing
    assert call(fake, 16, None, -1, 100.0, 1 << 30, *adam) == 2
    assert call(fake, 16, None, 0, 100.0, 1 << 30, 1e-3, 1.0, 0.999, 1e-8, 0.0) == 2
    assert b"betas" in lib.fhoad_last_error()
    assert call(fake, 16, None, 0, 100.0, 1 << 30, -1e-3, 0.9, 0.999, 1e-8, 0.0) == 2
    assert call(fake, 16, None, 0, -1.0, 1 << 30, *adam) == 2
    assert call(fake, 16, None, 0, 100.0, 10, *adam) == 4
    assert call(fake, 16, fake, 300, 100.0, lib.fhoad_poisson_adam_step_workspace_size(16, 200), *adam) == 4
    # The workspace holds 16-byte vectors: a pointer off that alignment is refused.
    odd = ctypes.c_void_p(260)
    assert step(fake, fake, 16, None, 0, 100.0, *[fake] * 5, None, None, odd, 1 << 30, *adam, None) == 3
    assert b"16-byte aligned" in lib.fhoad_last_error()
    backward = lib.fhoad_forward_laplacian_backward
    assert backward(fake, fake, fake, fake, fake, fake, odd, 1 << 30, 16, 6, None) == 3
    assert b"16-byte aligned" in lib.fhoad_last_error()
    # the saved-layer pair: the buffer is checked (presence, size, alignment) before any launch
    saving = lib.fhoad_forward_laplacian_saving
    need = lib.fhoad_saved_layers_size(16)
    assert saving(fake, fake, fake, fake, None, need, 16, 2, None) == 4
    assert saving(fake, fake, fake, fake, fake, need - 1, 16, 2, None) == 4
    assert b"saved-layer buffer holds" in lib.fhoad_last_error()
    assert saving(fake, fake, fake, fake, odd, need, 16, 2, None) == 3
    assert b"saved-layer buffer must be 16-byte aligned" in lib.fhoad_last_error()
    assert saving(fake, fake, fake, fake, None, 0, 16, 6, None) == 1
    assert saving(None, None, None, None, None, 0, 0, 2, None) == 0
    saved_bwd = lib.fhoad_forward_laplacian_backward_saved
    assert saved_bwd(fake, fake, None, need, fake, fake, fake, fake, fake, 1 << 30, 16, 6, None) == 4
    assert saved_bwd(fake, fake, fake, need - 16, fake, fake, fake, fake, fake, 1 << 30, 16, 6, None) == 4
    assert saved_bwd(fake, fake, odd, need, fake, fake, fake, fake, fake, 1 << 30, 16, 6, None) == 3
    assert saved_bwd(fake, fake, fake, need, fake, fake, fake, fake, fake, 10, 16, 6, None) == 4
    assert b"workspace holds" in lib.fhoad_last_error()
    assert saved_bwd(fake, fake, fake, need, fake, fake, fake, fake, fake, 1 << 30, 16, 0, None) == 1


def test_saved_layers_size() -> None:
    """3,072 f4 (49,152 bytes) per 16-point tile: the three hidden layers' 64 neurons x 4 jet
    components for 16 points, i.e. 3 KB per point, in whole tiles."""
    lib = _lib()
    assert lib.fhoad_saved_layers_size(0) == 0
    assert lib.fhoad_saved_layers_size(-5) == 0
    for batch in (1, 15, 16, 17, 65536, 70001, 1 << 31, 1 << 40):
        assert lib.fhoad_saved_layers_size(batch) == -(-batch // 16) * 49152, batch
    assert lib.fhoad_saved_layers_size(65536) == 65536 * 3 * 64 * 4 * 4
    # a buffer size past size_t saturates (no buffer holds it), as does the largest batch
    size_max = (1 << 64) - 1
    assert lib.fhoad_saved_layers_size(1 << 62) == size_max
    assert lib.fhoad_saved_layers_size((1 << 63) - 1) == size_max


def test_torch_extension_reports_contract_errors_on_cpu() -> None:
    from fused_hoad import _C

    x = torch.zeros(4, 2)
    p = torch.zeros(12737)
    with pytest.raises(RuntimeError, match="version must be 0 to 5"):
        _C.fused_forward_laplacian(x, p, 6)
    with pytest.raises(RuntimeError, match="backward version must be 1 to 6"):
        _C.fused_forward_laplacian_backward(x, p, x[:, 0], x[:, 0], 7)
    with pytest.raises(RuntimeError, match="coordinates must be a CUDA tensor"):
        _C.fused_forward_laplacian(x, p)


@pytest.mark.gpu
def test_raw_entry_points_match_the_torch_extension() -> None:
    from gpu_helpers import announce, coordinates, packed, require_gpu_extension, upstream

    require_gpu_extension()
    announce("C ABI via ctypes vs fused_hoad._C, batch=5000")
    from fused_hoad import _C

    lib = _lib()
    batch = 5000
    p = packed(0)
    x = coordinates(batch, seed=9)
    gu, gl = upstream(batch, seed=9)
    gu, gl = gu.reshape(-1).contiguous(), gl.reshape(-1).contiguous()
    stream = torch.cuda.current_stream().cuda_stream
    u = torch.empty(batch, 1, device="cuda")
    lap = torch.empty(batch, 1, device="cuda")
    status = lib.fhoad_forward_laplacian(x.data_ptr(), p.data_ptr(), u.data_ptr(), lap.data_ptr(), batch, 2, stream)
    assert status == 0, lib.fhoad_last_error()
    eu, el = _C.fused_forward_laplacian(x, p)
    torch.cuda.synchronize()
    assert torch.equal(u, eu) and torch.equal(lap, el)

    ws_bytes = lib.fhoad_backward_workspace_size(batch)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    gp = torch.empty(12737, device="cuda")
    gx = torch.empty(batch, 2, device="cuda")
    status = lib.fhoad_forward_laplacian_backward(
        x.data_ptr(), p.data_ptr(), gu.data_ptr(), gl.data_ptr(), gp.data_ptr(), gx.data_ptr(),
        ws.data_ptr(), ws_bytes, batch, 6, stream)
    assert status == 0, lib.fhoad_last_error()
    ep, ex = _C.fused_forward_laplacian_backward(x, p, gu, gl)
    torch.cuda.synchronize()
    assert torch.equal(gp, ep) and torch.equal(gx, ex)
    # null upstream gradients read as zeros, a null grad_coordinates is not written
    zeros = torch.zeros_like(gu)
    for null_u, null_l in ((True, False), (False, True)):
        gp_null = torch.empty(12737, device="cuda")
        status = lib.fhoad_forward_laplacian_backward(
            x.data_ptr(), p.data_ptr(), None if null_u else gu.data_ptr(),
            None if null_l else gl.data_ptr(), gp_null.data_ptr(), None, ws.data_ptr(), ws_bytes,
            batch, 6, stream)
        assert status == 0, lib.fhoad_last_error()
        ep0, _ = _C.fused_forward_laplacian_backward(x, p, zeros if null_u else gu, zeros if null_l else gl)
        torch.cuda.synchronize()
        assert torch.equal(gp_null, ep0), (null_u, null_l)
    # a workspace one byte short is refused
    status = lib.fhoad_forward_laplacian_backward(
        x.data_ptr(), p.data_ptr(), gu.data_ptr(), gl.data_ptr(), gp.data_ptr(), gx.data_ptr(),
        ws.data_ptr(), ws_bytes - 1, batch, 6, stream)
    assert status == 4


@pytest.mark.gpu
def test_raw_saved_layer_pair_matches_the_pair() -> None:
    """fhoad_forward_laplacian_saving and fhoad_forward_laplacian_backward_saved through ctypes
    at 70,001 points (whole rounds plus split tiles): bitwise the outputs of
    fhoad_forward_laplacian and the gradients of fhoad_forward_laplacian_backward."""
    from gpu_helpers import announce, coordinates, packed, require_gpu_extension, upstream

    require_gpu_extension()
    announce("C ABI saved-layer pair via ctypes vs forward and backward, batch=70001")
    from fused_hoad import _C

    lib = _lib()
    batch = 70001
    p = packed(3)
    x = coordinates(batch, seed=10)
    gu, gl = upstream(batch, seed=10)
    gu, gl = gu.reshape(-1).contiguous(), gl.reshape(-1).contiguous()
    stream = torch.cuda.current_stream().cuda_stream
    saved_bytes = lib.fhoad_saved_layers_size(batch)
    saved = torch.empty(saved_bytes, dtype=torch.uint8, device="cuda")
    u = torch.empty(batch, 1, device="cuda")
    lap = torch.empty(batch, 1, device="cuda")
    status = lib.fhoad_forward_laplacian_saving(x.data_ptr(), p.data_ptr(), u.data_ptr(), lap.data_ptr(),
                                                saved.data_ptr(), saved_bytes, batch, 2, stream)
    assert status == 0, lib.fhoad_last_error()
    ws_bytes = lib.fhoad_backward_workspace_size(batch)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    gp = torch.empty(12737, device="cuda")
    gx = torch.empty(batch, 2, device="cuda")
    status = lib.fhoad_forward_laplacian_backward_saved(
        x.data_ptr(), p.data_ptr(), saved.data_ptr(), saved_bytes, gu.data_ptr(), gl.data_ptr(),
        gp.data_ptr(), gx.data_ptr(), ws.data_ptr(), ws_bytes, batch, 6, stream)
    assert status == 0, lib.fhoad_last_error()
    eu, el = _C.fused_forward_laplacian(x, p)
    ep, ex = _C.fused_forward_laplacian_backward(x, p, gu, gl)
    torch.cuda.synchronize()
    assert torch.equal(u, eu) and torch.equal(lap, el)
    assert torch.equal(gp, ep) and torch.equal(gx, ex)


@pytest.mark.gpu
def test_raw_fused_step_matches_the_torch_extension() -> None:
    from gpu_helpers import announce, coordinates, packed, require_gpu_extension

    require_gpu_extension()
    announce("C ABI fhoad_poisson_adam_step via ctypes vs fused_hoad._C, batch=3000 + 300 boundary")
    from fused_hoad import _C, manufactured_source
    from fused_hoad.training import boundary_points

    lib = _lib()
    batch, nb = 3000, 300
    x = coordinates(batch, seed=13)
    f = manufactured_source(x).reshape(-1).contiguous()
    xb = boundary_points(nb, device="cpu", generator=torch.Generator().manual_seed(13)).cuda()
    stream = torch.cuda.current_stream().cuda_stream

    def state():
        p = packed(0)
        return p, torch.zeros_like(p), torch.zeros_like(p), torch.zeros(1, device="cuda")

    p, m, v, t = state()
    loss = torch.empty((), device="cuda")
    gp = torch.empty(12737, device="cuda")
    gx = torch.empty(batch, 2, device="cuda")
    ws_bytes = lib.fhoad_poisson_adam_step_workspace_size(batch, nb)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    for _ in range(2):
        status = lib.fhoad_poisson_adam_step(
            x.data_ptr(), f.data_ptr(), batch, xb.data_ptr(), nb, 100.0, p.data_ptr(),
            m.data_ptr(), v.data_ptr(), t.data_ptr(), loss.data_ptr(), gp.data_ptr(),
            gx.data_ptr(), ws.data_ptr(), ws_bytes, 1e-3, 0.9, 0.999, 1e-8, 0.0, stream)
        assert status == 0, lib.fhoad_last_error()

    ep, em, ev, et = state()
    egp = torch.empty_like(gp)
    egx = torch.empty_like(gx)
    for _ in range(2):
        eloss = _C.poisson_adam_step(x, f, ep, em, ev, et, 1e-3, 0.9, 0.999, 1e-8, 0.0, egp, egx,
                                     xb, 100.0)
    torch.cuda.synchronize()
    for a, b in ((p, ep), (m, em), (v, ev), (t, et), (loss, eloss), (gp, egp), (gx, egx)):
        assert torch.equal(a, b)
    assert float(t) == 2.0
