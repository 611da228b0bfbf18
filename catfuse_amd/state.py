"""StateBuffer: lazily allocated membrane-state container of a fused pattern.

Same contract as catfuse/state.py:26-98: `get(shape, device, dtype)` returns
the cached tensor or allocates zeros on first use / shape / device / dtype
change; `set(v)` stores v detached; `reset()` drops it so the next `get`
starts from zeros (wired to reset_net through CTFPattern.reset).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


class StateBuffer:
    __slots__ = ("_v",)

    def __init__(self):
        self._v: Optional[torch.Tensor] = None

    def get(self, shape: Tuple[int, ...], device, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        shape = torch.Size(shape)
        device = torch.device(device) if not isinstance(device, torch.device) else device
        v = self._v
        if v is None or v.shape != shape or v.device != device or v.dtype != dtype:
            self._v = torch.zeros(shape, device=device, dtype=dtype)
        return self._v

    def peek(self, shape, device, dtype=torch.float32) -> Optional[torch.Tensor]:
        """The stored tensor if it matches, else None (no allocation).  Fused
        kernels treat None as the initial state, which saves a zero fill."""
        v = self._v
        device = torch.device(device) if not isinstance(device, torch.device) else device
        if v is None or v.shape != torch.Size(shape) or v.device != device or v.dtype != dtype:
            return None
        return v

    def set(self, v: torch.Tensor) -> None:
        # a fused launch's lazily filled state (no autograd history) is kept
        # as it is: detach() would fill it now.  Its requires_grad is read
        # with the subclass's torch-function dispatch off (a plain read).
        if hasattr(v, "cf_materialize"):
            with torch._C.DisableTorchFunctionSubclass():
                keep = not v.requires_grad
            if keep:
                self._v = v
                return
        self._v = v.detach()

    def reset(self) -> None:
        self._v = None

    @property
    def is_initialized(self) -> bool:
        return self._v is not None

    @property
    def tensor(self) -> Optional[torch.Tensor]:
        return self._v

    def __repr__(self) -> str:
        if self._v is None:
            return "StateBuffer(uninitialized)"
        return (f"StateBuffer(shape={tuple(self._v.shape)}, device={self._v.device}, "
                f"dtype={self._v.dtype})")
