"""SparseFlow thresholds (mirrors catfuse/sparseflow/config.py:15-72).

The numeric values below are the reference's own.  The MI355X routing
thresholds that decide StaticZero / SparseFlow / DenseKeep at run time live
in catfuse_amd.hardware (HardwareProfile.sf_sparsity_threshold) and can be
overridden with the environment variable CATFUSE_SF_SPARSITY_THRESHOLD.
"""
from __future__ import annotations

import os

# Prescan activation threshold: a channel group is active in a tile iff some
# |x| > PRESCAN_ACTIVITY_EPS inside the tile's receptive field.
PRESCAN_ACTIVITY_EPS = 1e-6
NUMERIC_EPS = 1e-6

STATICZERO_EPS_BY_SPIKE_MODE = {
    "normalized_bernoulli": 1e-7,
    "raw_bernoulli": 1e-8,
    "raw_repeat": 1e-8,
}
STATICZERO_EPS_DEFAULT = 1e-6


def staticzero_eps_for_mode(spike_mode: str) -> float:
    return float(STATICZERO_EPS_BY_SPIKE_MODE.get(str(spike_mode), STATICZERO_EPS_DEFAULT))


SPARSE_DENSE_RATIO_THRESHOLD = 0.85
ENABLE_RUNTIME_FALLBACK_POLICY = False

# Execution-grounded dispatch (EGD) score thresholds of the reference
# (V100-calibrated; consumed only by the standalone SparseFlow framework).
DISPATCH_TAU_3X3 = 100_000
DISPATCH_TAU_1X1 = 200_000
DISPATCH_TAU_LINEAR = 800_000
DISPATCH_TAU_ATTN_LINEAR = 900_000
DISPATCH_TAU_ATTN_MATMUL = 1_200_000
DISPATCH_R_MIN = 0.15
DISPATCH_R_MARGIN = 0.0
DISPATCH_TAU_MARGIN = 0.0
DISPATCH_MIN_CONFIDENCE = 0.60

# Runtime route of STFusionConvBNLIF: SparseFlow iff input sparsity exceeds
# this value (reference: 0.7 at st_fusion_conv_bn_lif.py:516-524).
RUNTIME_SPARSITY_THRESHOLD = float(os.environ.get("CATFUSE_SF_SPARSITY_THRESHOLD", "0.7"))
