"""Implementation hierarchy of a Conv->(BN)->LIF operator on gfx950.

Public API (mirrors catfuse/implementations/__init__.py):
    Implementation, ConvLIFSpec, ConvLIFParams, IOCost, ScheduleTransform,
    ScheduleDecomposition, TSI_OPS, CSR_OPS, TGO_OPS, static_zero_forward,
    DenseKeep   — MFMA conv writing z, then the multi-step LIF (form 1),
    SparseFlow  — prescan + sparse fused conv/BN/LIF, device-routed (form 2),
    StreamFuse  — dense fused conv/BN/LIF with z on chip (form 2).
All three produce bit-identical outputs on every input.
"""
from catfuse_amd.implementations.base import (
    CSR_OPS, TGO_OPS, TSI_OPS, ConvLIFParams, ConvLIFSpec, Implementation, IOCost,
    ScheduleDecomposition, ScheduleTransform, static_zero_forward,
)
from catfuse_amd.implementations.dense_keep import DenseKeep
from catfuse_amd.implementations.sparse_flow import SparseFlow
from catfuse_amd.implementations.stream_fuse import StreamFuse

_SPARSEFLOW_AVAILABLE = True

__all__ = ["Implementation", "ConvLIFSpec", "ConvLIFParams", "IOCost", "ScheduleTransform",
           "ScheduleDecomposition", "TSI_OPS", "CSR_OPS", "TGO_OPS", "DenseKeep", "SparseFlow",
           "StreamFuse", "static_zero_forward"]
