"""HardwareProfile: device capabilities and routing thresholds.

Mirrors catfuse/hardware.py:22-179, keyed by the ROCm architecture name
(`gcnArchName`, e.g. "gfx950") instead of the CUDA SM version.  The reference
V100/A100 presets are kept for the static policy table's KATs; the MI355X
profile adds the thresholds the gfx950 kernels use at run time.

Fields (reference): arch_name, sm_version, hbm_bandwidth_gbps, l2_size_mb,
sm_count, sf_threshold_C, sf_threshold_H, default_K_memory_bound,
default_K_compute_bound, notes.
Fields (added): gcn_arch, peak_fp16_tflops, sf_sparsity_threshold (input
sparsity above which STFusionConvBNLIF takes the SparseFlow route),
dense_impl ("StreamFuse": fused Conv->BN->LIF with z on chip; "DenseKeep":
z through HBM as the reference's schedule).
"""
from __future__ import annotations

import os
from dataclasses import dataclass, replace


@dataclass(frozen=True)
class HardwareProfile:
    arch_name: str
    sm_version: tuple
    hbm_bandwidth_gbps: float
    l2_size_mb: float
    sm_count: int
    sf_threshold_C: int
    sf_threshold_H: int
    default_K_memory_bound: int
    default_K_compute_bound: int
    notes: str = ""
    gcn_arch: str = ""
    peak_fp16_tflops: float = 0.0
    sf_sparsity_threshold: float = 0.7
    dense_impl: str = "DenseKeep"

    @property
    def sm_capability(self) -> int:
        return self.sm_version[0] * 10 + self.sm_version[1]


V100_PCIE_32GB = HardwareProfile(
    arch_name="V100 PCIe 32GB", sm_version=(7, 0), hbm_bandwidth_gbps=900.0, l2_size_mb=6.0,
    sm_count=80, sf_threshold_C=256, sf_threshold_H=14, default_K_memory_bound=8,
    default_K_compute_bound=4,
    notes="Reference project default: SF considered at C>=256, H<=14.")

V100_SXM_32GB = replace(V100_PCIE_32GB, arch_name="V100 SXM 32GB")

A100_40GB = HardwareProfile(
    arch_name="A100 40GB", sm_version=(8, 0), hbm_bandwidth_gbps=1555.0, l2_size_mb=40.0,
    sm_count=108, sf_threshold_C=128, sf_threshold_H=28, default_K_memory_bound=8,
    default_K_compute_bound=4, notes="Reference tentative thresholds.")

A100_80GB = replace(A100_40GB, arch_name="A100 80GB", hbm_bandwidth_gbps=2039.0)

# AMD Instinct MI355X (CDNA4, gfx950): 256 CUs in 8 XCDs, 288 GB HBM3E at
# ~8 TB/s, 256 MB Infinity Cache, ~2.5 PFLOP/s dense fp16 MFMA.  The
# SparseFlow route threshold is the measured crossover of the gfx950 kernels
# (catfuse_amd.sparseflow.crossover): at every measured input sparsity of
# config C1 (i.i.d., per-channel and all-channel 8x8 block patterns, rates
# 0.001-0.5) the fused dense conv beat the forced SparseFlow route (scan +
# prescan + chunk skipping), so the threshold is 1.0 (never taken); all-zero
# inputs take StaticZero on every route.  The static regime thresholds keep
# the reference's table shape.
MI355X = HardwareProfile(
    arch_name="AMD Instinct MI355X", sm_version=(9, 5), hbm_bandwidth_gbps=8000.0,
    l2_size_mb=32.0, sm_count=256, sf_threshold_C=256, sf_threshold_H=14,
    default_K_memory_bound=8, default_K_compute_bound=4,
    notes="gfx950; fused StreamFuse conv as the dense path, device-side routing.",
    gcn_arch="gfx950", peak_fp16_tflops=2500.0, sf_sparsity_threshold=1.0,
    dense_impl="StreamFuse")

DEFAULT = V100_PCIE_32GB

_BY_SM = {(7, 0): V100_PCIE_32GB, (8, 0): A100_40GB}
_BY_GCN = {"gfx950": MI355X}


def _env_overrides(p: HardwareProfile) -> HardwareProfile:
    thr = os.environ.get("CATFUSE_SF_SPARSITY_THRESHOLD")
    impl = os.environ.get("CATFUSE_DENSE_IMPL")
    if thr is not None:
        p = replace(p, sf_sparsity_threshold=float(thr))
    if impl is not None:
        p = replace(p, dense_impl=impl)
    return p


def detect_hardware() -> HardwareProfile:
    """Profile of the current GPU: by gcnArchName on ROCm, by SM on CUDA;
    MI355X when the device is gfx950, DEFAULT when unknown or no GPU."""
    try:
        import torch
        if not torch.cuda.is_available():
            return _env_overrides(DEFAULT)
        props = torch.cuda.get_device_properties(torch.cuda.current_device())
        arch = getattr(props, "gcnArchName", "") or ""
        base = arch.split(":")[0]
        if base in _BY_GCN:
            return _env_overrides(_BY_GCN[base])
        key = (props.major, props.minor)
        return _env_overrides(_BY_SM.get(key, DEFAULT))
    except Exception:
        return _env_overrides(DEFAULT)


def runtime_profile() -> HardwareProfile:
    """Profile used by the gfx950 kernels at run time: always the MI355X one
    (the only target of this library), with environment overrides."""
    return _env_overrides(MI355X)


__all__ = ["HardwareProfile", "V100_PCIE_32GB", "V100_SXM_32GB", "A100_40GB", "A100_80GB",
           "MI355X", "DEFAULT", "detect_hardware", "runtime_profile"]
