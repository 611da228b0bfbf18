"""HIP-graph replay of a fused network's forward.

A fused forward is a fixed sequence of kernel launches: routing between
StaticZero / SparseFlow / dense is decided on the device, layers exchange
device tensors, counters are cleared by a kernel (no memset), and nothing
synchronises with the host.  The whole sequence (optionally preceded by the
state reset) is therefore captured once into a HIP graph and replayed, which
removes the host launch latency between the ~40 launches of a forward.

    graphed = catfuse_amd.graph.capture(fused, x_example)     # x: [T, B, ...]
    y = graphed(x)            # copies x into the captured input, replays

The captured input buffer keeps the example's layout: a direct-encoded input
given as a stride-0 view over T (``img.unsqueeze(0).expand(T, ...)``) is
captured as such (the fused stem reads the image once), and a call then
copies only the image.  The returned output is the graph's output tensor,
overwritten by the next replay (clone it to keep it).  A replay does not
update the model's Python-side state objects (StateBuffer.tensor keeps what
the last eager call stored); with reset=True every replay starts from the
initial membrane state, the usual per-batch inference step.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import snn
from .runtime import NHWCSpikes


def _base_of(x: torch.Tensor) -> torch.Tensor:
    """The storage-owning view behind a stride-0 time expansion, else x."""
    if x.dim() >= 1 and x.shape[0] > 1 and x.stride(0) == 0:
        return x[0]
    return x


def _materialize_all(out) -> None:
    """cf_materialize() every NHWC-backed tensor in a (nested) output."""
    stack = [out]
    while stack:
        a = stack.pop()
        if isinstance(a, NHWCSpikes):
            a.cf_materialize()
        elif isinstance(a, (list, tuple)):
            stack.extend(a)
        elif isinstance(a, dict):
            stack.extend(a.values())


class GraphedForward:
    """A captured ``reset_net(model); model(x)`` (or ``model(x)``) sequence."""

    def __init__(self, model: torch.nn.Module, example: torch.Tensor, *, reset: bool = True,
                 warmup: int = 2):
        if not example.is_cuda:
            raise RuntimeError("graph capture needs a GPU input")
        self.model = model
        self.reset = reset
        self.T = example.shape[0]
        self._expanded = example.dim() >= 1 and example.shape[0] > 1 and example.stride(0) == 0
        base = _base_of(example)
        self.static_base = base.detach().clone()
        if self._expanded:
            self.static_in = self.static_base.unsqueeze(0).expand(example.shape)
        else:
            self.static_in = self.static_base
        self.graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=example.device)
        side.wait_stream(torch.cuda.current_stream(example.device))
        with torch.no_grad():
            # warm-up on a side stream: weight packing, one-off input checks
            # and workspace allocation happen here, outside the capture
            with torch.cuda.stream(side):
                for _ in range(max(1, warmup)):
                    self._run()
            torch.cuda.current_stream(example.device).wait_stream(side)
            torch.cuda.synchronize(example.device)
            with torch.cuda.graph(self.graph):
                self.static_out = self._run()
                # a fused layer's output holds its values in its fp16 copy
                # until first read; fill the fp32 form inside the graph so
                # every replay refreshes it (outside, only the first read
                # after capture would)
                _materialize_all(self.static_out)
        torch.cuda.synchronize(example.device)

    def _run(self):
        if self.reset:
            snn.functional.reset_net(self.model)
        return self.model(self.static_in)

    def __call__(self, x: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Copy x (same shape; for a captured stride-0 input, either the
        expanded view or the image itself) into the captured input, replay,
        and return the captured output.  x = None replays on the current
        contents of the input buffer."""
        if x is not None:
            src = _base_of(x) if self._expanded else x
            if src.shape != self.static_base.shape:
                raise ValueError(f"expected input {tuple(self.static_base.shape)} "
                                 f"(or its expansion over T), got {tuple(x.shape)}")
            self.static_base.copy_(src, non_blocking=True)
        self.graph.replay()
        return self.static_out


def capture(model: torch.nn.Module, example: torch.Tensor, *, reset: bool = True,
            warmup: int = 2) -> GraphedForward:
    """Capture ``reset_net(model); model(example)`` (reset=True, the usual
    inference step of a stateful SNN) or ``model(example)`` into a HIP graph."""
    return GraphedForward(model, example, reset=reset, warmup=warmup)
