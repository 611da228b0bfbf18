"""Multi-step LIF launcher (mirrors catfuse/sparseflow/lif_seq_kernel.py:51-90).

`lif_sequential(z, v_init, tau, v_threshold, v_reset)` runs all T steps in
one gfx950 launch (cf_lif_multistep, mode 0) with v held in registers.  The
recurrence follows SpikingJelly's op order v + (z - (v - v_reset)) / tau
rather than the reference's v*DECAY + z*RT + V_RESET*RT reformulation.
"""
from __future__ import annotations

import torch

from catfuse_amd import runtime


def lif_sequential(z: torch.Tensor, v_init: torch.Tensor, tau: float = 2.0,
                   v_threshold: float = 1.0, v_reset: float = 0.0, decay_input: bool = True):
    """z [T, B, C, H, W], v_init [B, C, H, W] -> (spikes [T, ...], v_final)."""
    z = z.float().contiguous()
    v_in = v_init.float().contiguous() if v_init is not None else None
    return runtime.lif_multistep(z, v_in, tau=tau, v_threshold=v_threshold, v_reset=v_reset,
                                 decay_input=decay_input)
