"""SparseFlow: prescan + sparse fused Conv -> BN -> LIF, routed on the device.

Realises TimeBlock(K) ∘ StreamFuse(Conv, LIF) ∘ StateCarry(LIF)
(catfuse/implementations/sparse_flow.py:56-448) on gfx950:

1. cf_pack_input stages x as fp16 NHWC, ORs channel-group activity bits per
   pixel and counts nonzeros (one pass over x);
2. cf_prescan_tiles reduces the bits over each output tile's receptive
   field (group size as the reference's choose_group_size; 8x8 tiles, the
   MI355X profile's sf_tile, where the reference's _select_tile_sizes picks
   8x16 for large maps);
3. cf_compact_tiles orders the tiles on the device, those active at some
   step first (the reference's host-side _build_active_tile_ids,
   catfuse/sparseflow/sparse_conv2d_kernel.py:113-123, without its sync);
4. cf_conv_mfma in rectangular-tile mode reads the nonzero count and
   decides the route itself — nnz == 0: StaticZero (no K loop, z = bias);
   sparsity > threshold: the tiles in the compacted order, skipping every
   32-channel K chunk whose group bits are clear for the tile (and the
   MFMAs of a silent 16-channel half when the groups are 16 channels
   wide); otherwise dense — then applies BN and the LIF in its epilogue.
   No host synchronisation; every route gives bit-identical results
   (skipped chunks contribute exact zeros).

Steps 1-3 and the sparse route run only when the threshold is below 1.  The
MI355X profile's threshold is 1.0: on gfx950 the SparseFlow route beats the
fused dense conv only on channel-group sparse inputs, which the nonzero
count cannot tell from i.i.d. ones (bench.py --workload sf_crossover), so
the layer runs the dense fused conv, with StaticZero decided from the
input's count block.
"""
from __future__ import annotations

import math

import torch

from catfuse_amd.hardware import runtime_profile
from catfuse_amd.implementations._hip_conv import HipConvImplementation
from catfuse_amd.implementations.stream_fuse import fused_decomposition, fused_io_cost
from catfuse_amd.sparseflow.sparse_helpers import _select_tile_sizes, choose_group_size


class SparseFlow(HipConvImplementation):
    name = "SparseFlow"

    def __init__(self, sparsity_threshold: float = None, compact_tiles: bool = True,
                 egd: bool = True):
        """egd: gate the SparseFlow route with the profile's dispatch score
        (tau per kernel size; no gate when the profile's tau is negative; an
        infinite tau refuses SparseFlow for that kernel size outright, so
        its layers run no activity scan or prescan)."""
        super().__init__()
        prof = runtime_profile()
        self.sparsity_threshold = (prof.sf_sparsity_threshold
                                   if sparsity_threshold is None else float(sparsity_threshold))
        self.compact_tiles = bool(compact_tiles)
        self.tile = prof.sf_tile
        self.egd = None
        if egd:
            self.egd = {1: (prof.sf_egd_tau_1x1, prof.sf_egd_r_min),
                        3: (prof.sf_egd_tau_3x3, prof.sf_egd_r_min)}

    def geometry(self, spec, H_in, W_in):
        Ho, Wo = spec.output_hw(H_in, W_in)
        bh, bw = self.tile if self.tile is not None else _select_tile_sizes(Ho, Wo)
        gate = None
        if self.egd is not None:
            gate = self.egd.get(spec.kernel_size, self.egd[3])
            if gate[0] < 0:
                gate = None
        return dict(block_h=bh, block_w=bw, group_size=choose_group_size(spec.in_channels),
                    compact=self.compact_tiles, egd=gate)

    def refused(self, spec) -> bool:
        """Whether the profile refuses SparseFlow for this kernel size."""
        if self.egd is None:
            return False
        return math.isinf(self.egd.get(spec.kernel_size, self.egd[3])[0])

    def route_geometry(self, spec, H_in, W_in):
        """Prescan geometry for the conv, or None when the threshold (>= 1)
        or the profile's refusal for the kernel size can never select the
        SparseFlow route: no activity scan or prescan then, only the
        StaticZero check."""
        if self.sparsity_threshold >= 1.0 or self.refused(spec):
            return None
        return self.geometry(spec, H_in, W_in)

    def forward(self, x, spec, params, state):
        self.check_input(x, spec)
        _, B, _, H, W = x.shape
        dev = x.device
        Ho, Wo = spec.output_hw(H, W)
        r = self.runner(spec, params, dev)
        v_in = state.peek((B, spec.out_channels, Ho, Wo), dev)
        if self.input_is_analog(x):
            spikes, v_out = r.run_direct(x, v_in, emit_nhwc=True)
        else:
            sparse = self.route_geometry(spec, H, W)
            spikes, v_out = r.run_mfma(x.contiguous(), v_in, sparse=sparse,
                                       sparse_threshold=self.sparsity_threshold)
        state.set(v_out)
        return spikes

    def last_route(self) -> int:
        """Route of the most recent forward (0 ZERO, 1 SPARSE, 2 DENSE); reads
        the device counter, so it synchronises."""
        from catfuse_amd import runtime
        r = self._runner
        if r is None or getattr(r, "last_nnz", None) is None:
            return -1
        word = runtime.route_from_nnz(r.last_nnz, r.last_numel, self.sparsity_threshold)
        return int(word.item())

    def last_tiles(self):
        """(tile_class, ag_mask) of the most recent forward (device tensors)."""
        r = self._runner
        return None if r is None else r.last_tiles

    def forward_with_k(self, x, spec, params, state, K=None):
        T = x.shape[0]
        K = T if K is None else max(1, min(int(K), int(T)))
        if K >= T:
            return self.forward(x, spec, params, state)
        return torch.cat([self.forward(x[s:s + K].contiguous(), spec, params, state)
                          for s in range(0, T, K)], dim=0)

    def analytic_io_cost(self, spec, T, B, H_in, W_in, K=None, *, dtype_bytes=4):
        return fused_io_cost(spec, T, B, H_in, W_in, K, dtype_bytes, "SparseFlow")

    def schedule_decomposition(self, spec, T, K=None):
        return fused_decomposition(T, K, "SparseFlow")

    def __repr__(self):
        return (f"SparseFlow(hip, threshold={self.sparsity_threshold}, "
                f"packed={'yes' if self._runner is not None else 'no'})")
