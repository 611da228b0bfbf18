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
z through HBM as the reference's schedule), sf_tile (output tile of the
SparseFlow prescan and conv; None: the reference's _select_tile_sizes rule),
sf_egd_tau_3x3 / sf_egd_tau_1x1 / sf_egd_r_min (the execution-grounded
dispatch score gate of a SparseFlow launch, scored on the device by
cf_compact_tiles: SparseFlow iff R >= 0.99 or R >= r_min and R * MACs per
tile > tau; tau < 0: no score; tau = inf: SparseFlow refused for that kernel
size, no scan or prescan; the reference's sparseflow/config.py:48-61
DISPATCH_TAU_3X3 / _1X1 / DISPATCH_R_MIN).
"""
from __future__ import annotations

import math
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
    sf_tile: tuple = None
    sf_egd_tau_3x3: float = -1.0
    sf_egd_tau_1x1: float = -1.0
    sf_egd_r_min: float = 0.15

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
# SparseFlow thresholds come from the measured crossover of the gfx950
# kernels (bench.py --workload sf_crossover at 3x3 layers 256ch 14x14,
# 128ch 28x28, 64ch 56x56, 512ch 7x7; T=4, B=32): with i.i.d., per-channel
# 8x8 block and all-channel 8x8 block patterns at rates 0.001-0.5 the fused
# dense conv beats the forced SparseFlow route (activity scan + tile
# prescan + tile compaction + chunk skipping) at every sparsity; with dead
# 16-channel groups per image, or activity confined to a quarter of the
# image, SparseFlow wins at 82-99% input sparsity depending on the shape.
# The nonzero count does not tell these apart at equal sparsity, so the
# density threshold is 1.0: SparseFlow is never taken by default
# (CATFUSE_SF_SPARSITY_THRESHOLD enables it).  When enabled, the launch is
# gated on the device by the dispatch score over its tile masks: across the
# 140 measured rows the fraction R of (tile, group) pairs silent at every
# step separates wins from losses best with R_min = 0.4 (7 rows
# misclassified, each within 4% of break-even), while S = R * MACs-per-tile
# against any single tau misclassifies 24, so the 3x3 gate is R >= 0.4 with
# tau = 0 (the reference's V100 values, sparseflow/config.py:48-61, are
# tau_3x3 = 1e5 and R_min = 0.15).  1x1 layers (bench.py --workload
# sf_crossover --xo-kernel 1: the SEW downsamples 64->128 at 56x56, 128->256
# at 28x28, 256->512 at 14x14, stride 2, and a stride-1 256->256 pointwise
# conv at 14x14; same patterns, rates 0.001-0.5, 140 rows): forced SparseFlow
# takes 1.42-2.11x the dense route's time in every row (one tap leaves little
# MFMA work to skip, against the same activity scan, prescan and compaction),
# so the MI355X profile refuses SparseFlow for 1x1 convs (tau_1x1 = inf: no
# scan, no prescan; the reference's V100 tau_1x1 is 1e4, config.py:51-54).
# All-zero inputs take StaticZero on every route.  SparseFlow tiles are 8x8
# at every size: the 8x16 tile of the reference's rule (>= 3136 output
# pixels) needs the kernel's full register file (one workgroup per CU).  The
# static regime thresholds keep the reference's table shape.
MI355X = HardwareProfile(
    arch_name="AMD Instinct MI355X", sm_version=(9, 5), hbm_bandwidth_gbps=8000.0,
    l2_size_mb=32.0, sm_count=256, sf_threshold_C=256, sf_threshold_H=14,
    default_K_memory_bound=8, default_K_compute_bound=4,
    notes="gfx950; fused StreamFuse conv as the dense path, device-side routing.",
    gcn_arch="gfx950", peak_fp16_tflops=2500.0, sf_sparsity_threshold=1.0,
    dense_impl="StreamFuse", sf_tile=(8, 8), sf_egd_tau_3x3=0.0, sf_egd_tau_1x1=math.inf,
    sf_egd_r_min=0.4)

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
