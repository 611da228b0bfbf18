"""Implementation plug-in point of a Conv->(BN)->LIF operator.

Mirrors catfuse/implementations/base.py:33-483: the frozen `ConvLIFSpec`,
the runtime `ConvLIFParams` (pre-folded BN affine), the analytic `IOCost`
byte ledger, the `Implementation` ABC (forward / analytic_io_cost /
schedule_decomposition / reset_caches), `static_zero_forward`, and the
schedule algebra (`ScheduleTransform`, `ScheduleDecomposition.verify`) with
its TSI/CSR typing rules.  These interfaces are kept identical because
patterns and tests written against the reference consume them.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn


@dataclass(frozen=True)
class ConvLIFSpec:
    in_channels: int
    out_channels: int
    kernel_size: int
    stride: int
    padding: int
    has_conv_bias: bool
    has_bn: bool
    tau: float
    v_threshold: float
    v_reset: Optional[float]
    decay_input: bool = True
    bn_eps: float = 1e-5

    def output_hw(self, h_in: int, w_in: int):
        return ((h_in + 2 * self.padding - self.kernel_size) // self.stride + 1,
                (w_in + 2 * self.padding - self.kernel_size) // self.stride + 1)


class ConvLIFParams:
    """Tensor references: weight [Cout, Cin, k, k], bias [Cout] or None,
    bn_scale / bn_bias [Cout] (folded eval BN: z*bn_scale + bn_bias) or None."""
    __slots__ = ("weight", "bias", "bn_scale", "bn_bias")

    def __init__(self, weight, bias, bn_scale, bn_bias):
        self.weight = weight
        self.bias = bias
        self.bn_scale = bn_scale
        self.bn_bias = bn_bias


@dataclass(frozen=True)
class IOCost:
    """Analytic HBM bytes of one forward, per tensor."""
    x_load: int
    w_load: int
    z_io: int
    v_io: int
    spike_write: int
    schedule: str
    num_blocks: int

    @property
    def intermediate_io(self) -> int:
        return self.z_io + self.v_io

    @property
    def total(self) -> int:
        return self.x_load + self.w_load + self.z_io + self.v_io + self.spike_write

    def as_dict(self) -> dict:
        return {"x_load": self.x_load, "w_load": self.w_load, "z_io": self.z_io,
                "v_io": self.v_io, "spike_write": self.spike_write,
                "intermediate_io": self.intermediate_io, "total": self.total,
                "schedule": self.schedule, "num_blocks": self.num_blocks}


class Implementation(nn.Module, ABC):
    """One member of Impl(sigma): forward(x [T,B,Cin,H,W]) -> spikes
    [T,B,Cout,Ho,Wo], reading/writing the membrane state via StateBuffer."""

    name: str = "<unset>"

    @abstractmethod
    def forward(self, x: torch.Tensor, spec: ConvLIFSpec, params: ConvLIFParams,
                state) -> torch.Tensor:
        ...

    @abstractmethod
    def analytic_io_cost(self, spec: ConvLIFSpec, T: int, B: int, H_in: int, W_in: int,
                         K: int = None, *, dtype_bytes: int = 4) -> IOCost:
        ...

    @abstractmethod
    def schedule_decomposition(self, spec: ConvLIFSpec, T: int,
                               K: int = None) -> "ScheduleDecomposition":
        ...

    def reset_caches(self) -> None:
        pass


def static_zero_forward(spec, params, T, B, H_out, W_out, device, state, lif_sequential_fn):
    """x == 0  =>  Conv(x) = bias, so z = bias*bn_scale + bn_bias (or bn_bias,
    or bias, or 0) broadcast over (T, B, H_out, W_out); the LIF still runs."""
    if spec.has_bn:
        zc = (params.bias * params.bn_scale + params.bn_bias) if spec.has_conv_bias else params.bn_bias
    elif spec.has_conv_bias:
        zc = params.bias
    else:
        zc = torch.zeros(spec.out_channels, dtype=torch.float32, device=device)
    z = zc.float().view(1, 1, -1, 1, 1).expand(T, B, spec.out_channels, H_out, W_out).contiguous()
    v_in = state.get(shape=(B, spec.out_channels, H_out, W_out), device=device,
                     dtype=torch.float32)
    spikes, v_out = lif_sequential_fn(z, v_in, tau=spec.tau, v_threshold=spec.v_threshold,
                                      v_reset=spec.v_reset)
    state.set(v_out)
    return spikes


# ---------------------------------------------------------------------------
# Schedule algebra: TimeBlock / BatchFold / StreamFuse / StateCarry
# ---------------------------------------------------------------------------

TSI_OPS = frozenset({"Conv", "BN", "Linear", "Add", "Pool"})
CSR_OPS = frozenset({"LIF", "PSN"})
TGO_OPS = frozenset({"Attention", "GroupNorm", "LayerNorm"})


def _kind(op):
    return "CSR" if op in CSR_OPS else ("TSI" if op in TSI_OPS else "unknown/TGO")


@dataclass(frozen=True)
class ScheduleTransform:
    primitive: str
    args: tuple

    @classmethod
    def TimeBlock(cls, K: int):
        return cls("TimeBlock", (int(K),))

    @classmethod
    def BatchFold(cls, op: str):
        return cls("BatchFold", (str(op),))

    @classmethod
    def StreamFuse(cls, u: str, v: str):
        return cls("StreamFuse", (str(u), str(v)))

    @classmethod
    def StateCarry(cls, op: str):
        return cls("StateCarry", (str(op),))

    def __str__(self):
        if self.primitive == "TimeBlock":
            return f"TimeBlock(K={self.args[0]})"
        if self.primitive == "StreamFuse":
            return f"StreamFuse({self.args[0]}, {self.args[1]})"
        if self.primitive in ("BatchFold", "StateCarry"):
            return f"{self.primitive}({self.args[0]})"
        return f"{self.primitive}{self.args}"

    def check_typing(self):
        e = []
        p, a = self.primitive, self.args
        if p == "TimeBlock":
            if len(a) != 1:
                e.append(f"TimeBlock takes 1 arg, got {len(a)}")
            elif a[0] < 1:
                e.append(f"TimeBlock(K) requires K >= 1, got {a[0]}")
        elif p == "BatchFold":
            if len(a) != 1:
                e.append(f"BatchFold takes 1 arg, got {len(a)}")
            elif a[0] not in TSI_OPS:
                e.append(f"BatchFold({a[0]}) ILLEGAL — op must be TSI; {a[0]} is {_kind(a[0])}")
        elif p == "StreamFuse":
            if len(a) != 2:
                e.append(f"StreamFuse takes 2 args, got {len(a)}")
            else:
                if a[0] not in TSI_OPS:
                    e.append(f"StreamFuse({a[0]}, {a[1]}) ILLEGAL — u={a[0]} must be TSI")
                if a[1] not in CSR_OPS:
                    e.append(f"StreamFuse({a[0]}, {a[1]}) ILLEGAL — v={a[1]} must be CSR")
        elif p == "StateCarry":
            if len(a) != 1:
                e.append(f"StateCarry takes 1 arg, got {len(a)}")
            elif a[0] not in CSR_OPS:
                e.append(f"StateCarry({a[0]}) ILLEGAL — op must be CSR; {a[0]} is {_kind(a[0])}")
        else:
            e.append(f"Unknown primitive '{p}'")
        return e


@dataclass(frozen=True)
class ScheduleDecomposition:
    """Transforms innermost-first; str() reads outermost-first."""
    transforms: tuple
    form: str
    description: str = ""

    def __str__(self):
        return " ∘ ".join(str(t) for t in reversed(self.transforms))

    def verify(self):
        errors = []
        for i, t in enumerate(self.transforms):
            for e in t.check_typing():
                errors.append(f"transform[{i}] {t}: {e}")
        prims = [t.primitive for t in self.transforms]
        if "TimeBlock" not in prims:
            errors.append("Missing TimeBlock — a chunked schedule is required "
                          "(use TimeBlock(K=T) for the single-block case)")
        fused_csr = {t.args[1] for t in self.transforms
                     if t.primitive == "StreamFuse" and len(t.args) == 2}
        carried = {t.args[0] for t in self.transforms
                   if t.primitive == "StateCarry" and len(t.args) == 1}
        for v in fused_csr - carried:
            errors.append(f"StreamFuse(_, {v}) without StateCarry({v}) — the CSR state of {v} "
                          f"must be carried at block boundaries")
        if self.form not in ("form_1", "form_2", "form_3", "custom"):
            errors.append(f"unknown form '{self.form}'")
        return (len(errors) == 0, errors)
