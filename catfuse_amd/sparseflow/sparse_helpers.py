"""Tile classes, group sizing and popcount (mirrors
catfuse/sparseflow/sparse_helpers.py:28-75 and sparse_conv2d_kernel.py:80-84)."""
from __future__ import annotations

import torch

TILE_ZERO = 0
TILE_SPARSE = 1
TILE_DENSEISH = 2
TILE_UNCERTAIN = 3
TILE_ZERO_CANDIDATE = 4


def choose_group_size(k_dim: int) -> int:
    """Channels per prescan group: 16 if k <= 128 else 32, doubled until the
    group count fits one 32-bit mask."""
    gs = 16 if k_dim <= 128 else 32
    while (k_dim + gs - 1) // gs > 32:
        gs *= 2
    return gs


def _select_tile_sizes(H: int, W: int):
    """Output tile (BH, BW): 8x16 when H*W >= 3136, else 8x8."""
    return (8, 16) if H * W >= 3136 else (8, 8)


select_tile_sizes = _select_tile_sizes


def popcount_buf(ag_mask_buf: torch.Tensor, count: int) -> torch.Tensor:
    """Per-entry popcount of an int32 bitmask buffer (device op, no sync)."""
    v = ag_mask_buf[:count].to(torch.int64) & 0xFFFFFFFF
    n = torch.zeros_like(v)
    for _ in range(32):
        n += v & 1
        v >>= 1
    return n.to(torch.int32)
