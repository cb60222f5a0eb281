"""Shared configuration constants.

Same names and values as the reference's Utils/config.py so callers that
import them keep working (Utils/config.py:15,38,43,50-61).
"""

from __future__ import annotations

# Prescan activity threshold: an element is active iff f16(|x|) > f16(eps).
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


# Dense-fallback ratio of the (disabled) runtime policy.
SPARSE_DENSE_RATIO_THRESHOLD = 0.85

# The reference ships its runtime EMA policy switched off; the same default
# here means a SparseConv2d always takes the sparse kernels on device tensors.
ENABLE_RUNTIME_FALLBACK_POLICY = False

DISPATCH_TAU_3X3 = 100_000
DISPATCH_TAU_1X1 = 200_000
DISPATCH_TAU_LINEAR = 800_000
DISPATCH_TAU_ATTN_LINEAR = 900_000
DISPATCH_TAU_ATTN_MATMUL = 1_200_000
DISPATCH_R_MIN = 0.15
DISPATCH_R_MARGIN = 0.0
DISPATCH_TAU_MARGIN = 0.0
DISPATCH_MIN_CONFIDENCE = 0.60

REPORT_ENERGY_PROXY_DEFAULT = False
BENCH_VERSION = "sparseflow-amd-0.1"
