"""SparseFlow prescan on gfx950 (mirrors catfuse/sparseflow/fast_prescan_v2.py
:92-137 and prescan.py:153-306).

Two kernels: cf_pack_input ORs |x| > threshold over each channel group per
pixel (one coalesced pass over x), then cf_prescan_tiles ORs those bits over
each output tile's receptive field with one wave64 per tile.  Results are
bit-identical to the reference's max-pool cascade definition.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from catfuse_amd import runtime
from catfuse_amd.sparseflow.sparse_helpers import TILE_DENSEISH, TILE_SPARSE, TILE_ZERO  # noqa


def fast_spike_prescan_2d_v2(
    x: torch.Tensor,
    H_OUT: int, W_OUT: int,
    kernel_size: int = 3, stride: int = 1, padding: int = 1,
    block_h: int = 8, block_w: int = 16,
    group_size_c: int = 16,
    threshold: float = 1e-6,
    ag_mask_out: Optional[torch.Tensor] = None,
    tile_class_out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [N, C, H, W] fp32 -> (tile_class int32 [N*GH*GW], ag_mask int32 [...])."""
    x = x.float().contiguous()
    N, C, H, W = x.shape
    G = -(-C // group_size_c)
    if G > 32:
        raise ValueError(f"{G} channel groups do not fit a 32-bit mask")
    _, act = runtime.pack_input(x, want_xp=False, group_size=group_size_c, threshold=threshold)
    return runtime.prescan_tiles(act, H, W, H_OUT, W_OUT, kernel_size, stride, padding, block_h,
                                 block_w, G, ag_mask_out, tile_class_out)
