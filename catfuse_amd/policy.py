"""Static spatio-temporal policy table (mirrors catfuse/policy.py:28-279).

For each fusible pattern and shape regime: TimeBlock size K, spatial backend
(DenseKeep / SparseFlow / StaticZero), fusion mode and the analytic HBM
ratio of the schedule.  Regime thresholds come from a HardwareProfile
(reference V100 default unless one is passed or detected).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional


class SpatialBackend:
    DENSE_KEEP = "DenseKeep"
    SPARSE_FLOW = "SparseFlow"
    STATIC_ZERO = "StaticZero"


@dataclass
class PolicyRow:
    pattern: str
    shape_regime: str
    K: int
    spatial_backend: str
    fusion_mode: str
    io_ratio: Optional[float] = None

    def __repr__(self):
        return (f"PolicyRow({self.pattern}, {self.shape_regime}, K={self.K}, "
                f"spatial={self.spatial_backend}, fusion={self.fusion_mode}, io={self.io_ratio})")


def io_ratio_partial_fusion(K: int) -> float:
    """(3 + 2/K) / 7: z written and read through HBM, v carried per block."""
    return (3.0 + 2.0 / K) / 7.0


def io_ratio_full_fusion(K: int) -> float:
    """(1 + 2/K) / 5: z stays on chip (StreamFuse), v carried per block."""
    return (1.0 + 2.0 / K) / 5.0


def _profile(hwprof):
    if hwprof is None:
        from catfuse_amd.hardware import DEFAULT
        return DEFAULT
    return hwprof


def optimal_K(T: int, regime: str = "memory_bound", hwprof=None) -> int:
    p = _profile(hwprof)
    if regime == "compute_bound":
        return min(p.default_K_compute_bound, T)
    return min(p.default_K_memory_bound, T)


def classify_shape_regime(C_in: int, C_out: int, H: int, W: int, kernel_size: int = 3,
                          hwprof=None) -> str:
    """1x1 -> memory_bound; C_in >= sf_C and H <= sf_H -> memory_bound;
    C_in <= sf_C/2 -> compute_bound; H >= 2*sf_H -> compute_bound; else
    memory_bound."""
    p = _profile(hwprof)
    sf_C, sf_H = p.sf_threshold_C, p.sf_threshold_H
    if kernel_size == 1:
        return "memory_bound"
    if C_in >= sf_C and H <= sf_H:
        return "memory_bound"
    if C_in <= sf_C // 2:
        return "compute_bound"
    if H >= sf_H * 2:
        return "compute_bound"
    return "memory_bound"


def build_default_policy_table():
    t = {}
    t[("Conv3x3_BN_LIF", "compute_bound")] = PolicyRow(
        "Conv3x3_BN_LIF", "compute_bound", 4, SpatialBackend.DENSE_KEEP, "partial_cudnn",
        io_ratio_partial_fusion(4))
    t[("Conv3x3_BN_LIF", "memory_bound")] = PolicyRow(
        "Conv3x3_BN_LIF", "memory_bound", 8, SpatialBackend.SPARSE_FLOW, "full_triton",
        io_ratio_full_fusion(8))
    t[("Conv1x1_LIF", "memory_bound")] = PolicyRow(
        "Conv1x1_LIF", "memory_bound", 8, SpatialBackend.SPARSE_FLOW, "full_triton",
        io_ratio_full_fusion(8))
    for pat in ("Linear_LIF", "Add_LIF", "Add_BN_LIF", "AvgPool_LIF"):
        t[(pat, "all")] = PolicyRow(pat, "all", 0, SpatialBackend.DENSE_KEEP, "full_triton", None)
    return t


_DEFAULT_TABLE = None


def get_policy(pattern: str, C_in: int = 0, C_out: int = 0, H: int = 0, W: int = 0,
               kernel_size: int = 3, T: int = 16, hwprof=None) -> PolicyRow:
    """Policy row for (pattern, shape); K=0 in the table means K=T."""
    global _DEFAULT_TABLE
    if _DEFAULT_TABLE is None:
        _DEFAULT_TABLE = build_default_policy_table()
    if pattern in ("Linear_LIF", "Add_LIF", "Add_BN_LIF", "AvgPool_LIF"):
        regime = "all"
    else:
        regime = classify_shape_regime(C_in, C_out, H, W, kernel_size, hwprof)
    row = _DEFAULT_TABLE.get((pattern, regime))
    if row is not None:
        if row.K == 0:
            row = PolicyRow(row.pattern, row.shape_regime, T, row.spatial_backend,
                            row.fusion_mode, row.io_ratio)
        return row
    K = min(4, T)
    return PolicyRow(pattern, regime, K, SpatialBackend.DENSE_KEEP, "partial_cudnn",
                     io_ratio_partial_fusion(K))
