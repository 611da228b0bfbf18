"""DenseKeep: Conv -> BN (z through HBM) then the multi-step LIF.

Realises the reference's form-1 schedule TimeBlock(K=T) ∘ BatchFold(Conv) ∘
StateCarry(LIF) (catfuse/implementations/dense_keep.py:29-251) on gfx950:
the MFMA conv kernel writes z = BN(conv(x)) for all T steps, then
cf_lif_multistep runs the T-step LIF with v in registers.  StaticZero is
decided on the device (nnz == 0 makes the conv kernel skip its K loop, so
z = bias exactly), with no host synchronisation.
"""
from __future__ import annotations

from catfuse_amd.implementations._hip_conv import HipConvImplementation
from catfuse_amd.implementations.base import IOCost, ScheduleDecomposition, ScheduleTransform
from catfuse_amd.runtime import EPI_Z, lif_multistep


class DenseKeep(HipConvImplementation):
    name = "DenseKeep"

    def forward(self, x, spec, params, state):
        self.check_input(x, spec)
        T, B = x.shape[0], x.shape[1]
        Ho, Wo = spec.output_hw(x.shape[3], x.shape[4])
        r = self.runner(spec, params, x.device)
        if self.input_is_analog(x):
            z, _ = r.run_direct(x, epilogue=EPI_Z)
        else:
            z, _ = r.run_mfma(x.contiguous(), epilogue=EPI_Z, static_zero=True)
        v_in = state.peek((B, spec.out_channels, Ho, Wo), x.device)
        spikes, v_out = lif_multistep(z, v_in, tau=spec.tau, v_threshold=spec.v_threshold,
                                      v_reset=spec.v_reset, decay_input=spec.decay_input)
        state.set(v_out)
        return spikes

    def analytic_io_cost(self, spec, T, B, H_in, W_in, K=None, *, dtype_bytes=4):
        """x T·B·HWC_in, w Cout·Cin·k², z 2·T·B·HWC_out (write+read),
        v 2·B·HWC_out, spikes T·B·HWC_out (bytes of dtype_bytes)."""
        H_out, W_out = spec.output_hw(H_in, W_in)
        hwc_in = H_in * W_in * spec.in_channels
        hwc_out = H_out * W_out * spec.out_channels
        kk = spec.kernel_size * spec.kernel_size
        return IOCost(
            x_load=T * B * hwc_in * dtype_bytes,
            w_load=spec.out_channels * spec.in_channels * kk * dtype_bytes,
            z_io=2 * T * B * hwc_out * dtype_bytes,
            v_io=2 * B * hwc_out * dtype_bytes,
            spike_write=T * B * hwc_out * dtype_bytes,
            schedule="TimeBlock(T)∘BatchFold(Conv) — z materialized to HBM",
            num_blocks=1)

    def schedule_decomposition(self, spec, T, K=None):
        return ScheduleDecomposition(
            transforms=(ScheduleTransform.StateCarry("LIF"), ScheduleTransform.BatchFold("Conv"),
                        ScheduleTransform.TimeBlock(T)),
            form="form_1",
            description=f"DenseKeep: TimeBlock(K=T={T}) ∘ BatchFold(Conv) ∘ StateCarry(LIF); "
                        f"z materialized between the MFMA conv and the LIF kernel.")

    def __repr__(self):
        return f"DenseKeep(hip, packed={'yes' if self._runner is not None else 'no'})"
