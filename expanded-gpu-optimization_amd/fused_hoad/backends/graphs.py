"""Graph replay of a backend, for inference (/root/reference/src/fused_hoad/backends/graphs.py:15-46).

``cuda_graphed(backend)`` captures ``backend(model, coordinates)`` in a HIP graph the first time
it sees a model and an input shape, dtype and device, and afterwards replays the graph: each
call copies its coordinates into the captured input buffer, replays, and returns the captured
output buffers. Like the reference's wrapper:
* it is inference only: a replay records no autograd history;
* the returned tensors are the graph's own buffers, which the next call overwrites (clone them
  to keep a result);
* one capture is kept: another model or shape, or a parameter tensor replaced by a new one,
  replaces it;
* the weights are read at every replay, so in-place weight updates are seen;
* off the GPU it calls the backend directly.
Before the capture the backend runs three times on a side stream (default priority), so lazy
initialisation (library handles, workspaces) happens outside the graph.
"""

from __future__ import annotations

import weakref
from collections.abc import Callable

import torch
from torch import Tensor, nn

Backend = Callable[[nn.Module, Tensor], tuple[Tensor, Tensor]]

_WARMUP_CALLS = 3


def _signature(model: nn.Module, coordinates: Tensor) -> tuple:
    """What a capture depends on besides the model object: the input's shape, dtype and device
    and the storage of every parameter and buffer (the graph holds their addresses)."""
    tensors = [*model.parameters(), *model.buffers()]
    return (tuple(coordinates.shape), coordinates.dtype, coordinates.device,
            tuple(t.data_ptr() for t in tensors))


class _Capture:
    """One captured call: the model it belongs to, the graph, its input and output buffers."""

    def __init__(self, backend: Backend, model: nn.Module, coordinates: Tensor) -> None:
        self.model = weakref.ref(model)
        self.signature = _signature(model, coordinates)
        # The graph reads these storages at every replay: hold them for the graph's lifetime.
        self.tensors = [*model.parameters(), *model.buffers()]
        self.input = coordinates.clone()
        side = torch.cuda.Stream(device=coordinates.device)
        side.wait_stream(torch.cuda.current_stream(coordinates.device))
        with torch.cuda.stream(side):
            for _ in range(_WARMUP_CALLS):
                backend(model, self.input)
        torch.cuda.current_stream(coordinates.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.output = backend(model, self.input)

    def matches(self, model: nn.Module, coordinates: Tensor) -> bool:
        return self.model() is model and self.signature == _signature(model, coordinates)

    def __call__(self, coordinates: Tensor) -> tuple[Tensor, Tensor]:
        self.input.copy_(coordinates)
        self.graph.replay()
        return self.output


def cuda_graphed(backend: Backend) -> Backend:
    """``backend`` with its GPU calls replayed from a captured HIP graph."""
    captured: list[_Capture] = []

    def run(model: nn.Module, coordinates: Tensor) -> tuple[Tensor, Tensor]:
        if coordinates.device.type != "cuda":
            return backend(model, coordinates)
        if not captured or not captured[0].matches(model, coordinates):
            captured.clear()  # release the previous graph's buffers before capturing anew
            captured.append(_Capture(backend, model, coordinates))
        return captured[0](coordinates)

    run.__name__ = f"cuda_graphed_{getattr(backend, '__name__', 'backend')}"
    run.__doc__ = f"HIP-graph replay of {getattr(backend, '__name__', 'a backend')} (inference only)."
    return run
