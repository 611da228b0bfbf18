"""StreamFuse: dense fused Conv -> BN -> LIF with z kept on chip.

The form-2 schedule TimeBlock(K) ∘ StreamFuse(Conv, LIF) ∘ StateCarry(LIF)
for dense inputs: one MFMA conv launch computes all T steps, applies the
folded BN and the LIF in its epilogue with v in registers, and writes only
spikes (and v at the end).  It is the gfx950 realisation of the reference's
dense full-fusion kernel (benchmarks/conv_bn_lif_min.py:56-163) and the
default dense path of the patterns on MI355X.  Results are bit-identical to
DenseKeep (same conv accumulation, same LIF op order).
"""
from __future__ import annotations

import math

from catfuse_amd.implementations._hip_conv import HipConvImplementation
from catfuse_amd.implementations.base import IOCost, ScheduleDecomposition, ScheduleTransform
from catfuse_amd.runtime import ID_ADD_SPIKE


def fused_io_cost(spec, T, B, H_in, W_in, K=None, dtype_bytes=4, label="StreamFuse"):
    """x T·B·HWC_in, w ceil(T/K)·Cout·Cin·k², z 0, v 2·ceil(T/K)·B·HWC_out,
    spikes T·B·HWC_out (catfuse/implementations/sparse_flow.py:330-401)."""
    K = T if K is None else max(1, min(int(K), int(T)))
    nb = math.ceil(T / K)
    H_out, W_out = spec.output_hw(H_in, W_in)
    hwc_in = H_in * W_in * spec.in_channels
    hwc_out = H_out * W_out * spec.out_channels
    kk = spec.kernel_size * spec.kernel_size
    return IOCost(
        x_load=T * B * hwc_in * dtype_bytes,
        w_load=nb * spec.out_channels * spec.in_channels * kk * dtype_bytes,
        z_io=0,
        v_io=2 * nb * B * hwc_out * dtype_bytes,
        spike_write=T * B * hwc_out * dtype_bytes,
        schedule=(f"TimeBlock(K={K})∘StreamFuse(Conv,LIF)∘StateCarry(LIF) "
                  f"— z in registers, v carried at {nb} block boundaries"),
        num_blocks=nb)


def fused_decomposition(T, K, label):
    K = T if K is None else max(1, min(int(K), int(T)))
    return ScheduleDecomposition(
        transforms=(ScheduleTransform.StateCarry("LIF"), ScheduleTransform.StreamFuse("Conv", "LIF"),
                    ScheduleTransform.TimeBlock(K)),
        form="form_2",
        description=(f"{label}: TimeBlock(K={K}) ∘ StreamFuse(Conv, LIF) ∘ StateCarry(LIF); "
                     f"z stays on chip, v carried at {(T + K - 1) // K} block boundaries."))


class StreamFuse(HipConvImplementation):
    name = "StreamFuse"

    def forward(self, x, spec, params, state, identity=None, identity_mode=ID_ADD_SPIKE):
        self.check_input(x, spec)
        _, B, _, H, W = x.shape
        dev = x.device
        Ho, Wo = spec.output_hw(H, W)
        r = self.runner(spec, params, dev)
        v_in = state.peek((B, spec.out_channels, Ho, Wo), dev)
        if self.input_is_analog(x):
            if identity is not None:
                raise NotImplementedError("identity epilogue needs fp16-exact inputs")
            spikes, v_out = r.run_direct(x, v_in, emit_nhwc=True)
        else:
            spikes, v_out = r.run_mfma(x.contiguous(), v_in, identity=identity,
                                       identity_mode=identity_mode, static_zero=True)
        state.set(v_out)
        return spikes

    def forward_with_k(self, x, spec, params, state, K=None):
        T = x.shape[0]
        K = T if K is None else max(1, min(int(K), int(T)))
        if K >= T:
            return self.forward(x, spec, params, state)
        import torch
        return torch.cat([self.forward(x[s:s + K].contiguous(), spec, params, state)
                          for s in range(0, T, K)], dim=0)

    def analytic_io_cost(self, spec, T, B, H_in, W_in, K=None, *, dtype_bytes=4):
        return fused_io_cost(spec, T, B, H_in, W_in, K, dtype_bytes)

    def schedule_decomposition(self, spec, T, K=None):
        return fused_decomposition(T, K, "StreamFuse")

    def __repr__(self):
        return f"StreamFuse(hip, packed={'yes' if self._runner is not None else 'no'})"
