"""SparseBMM / SparseMatmul: functional spike-sparse matmul modules
(drop-in for Ops/sparse_bmm.py:22-131 and Ops/sparse_matmul.py:22-190).
Device tensors run the library kernels (Kernels.bmm / Kernels.matmul);
host tensors run torch.bmm / torch.mm in f32 as the reference does."""

from __future__ import annotations

from typing import Any, Dict

import torch
import torch.nn as nn

from ..Kernels.bmm import sparse_bmm_forward
from ..Kernels.matmul import sparse_matmul_forward
from ._runtime import OpReporting


def _tile_diag(ts) -> Dict[str, Any]:
    out: Dict[str, Any] = {"tile_stats": ts}
    if isinstance(ts, dict):
        total, zero = ts.get("total_tiles", -1), ts.get("zero_tiles", -1)
        if total and total > 0:
            out["total_tile_count"] = int(total)
            if zero is not None and zero >= 0:
                out["tile_zero_count"] = int(zero)
                out["tile_zero_ratio"] = float(zero) / float(total)
    return out


class _SparseMM(OpReporting, nn.Module):
    def __init__(self, threshold: float = 1e-6, fallback_ratio: float = 0.85, return_ms: bool = False,
                 profile_runtime: bool = False):
        super().__init__()
        self.threshold = float(threshold)
        self.fallback_ratio = float(fallback_ratio)
        self.return_ms = bool(return_ms)
        self._init_reporting("sparse_kernel", self.diag_path, self.score_family, profile_runtime=profile_runtime)

    def _bmm(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        self._last_diag = {}
        self.fallback_reason = ""
        if not a.is_cuda:
            self.fallback_reason = "host_tensor"
            self.diag_source = "missing"
            return torch.bmm(a.float(), b.float())
        want = self.collect_diag and not self._inference_mode
        res = sparse_bmm_forward(a, b, threshold=self.threshold, return_ms=self.return_ms,
                                 return_avg_active_ratio=want, return_tile_stats=want,
                                 fallback_ratio=self.fallback_ratio)
        self._last_sparse_ms = float(res[1])
        if want:
            self._last_diag = _tile_diag(res[3])
            self._last_diag["avg_active_ratio"] = res[2]
            self._last_diag["active_group_ratio"] = float(res[2])
            self.diag_source = "measured"
        return res[0]

    def extra_repr(self):
        return f"threshold={self.threshold}, fallback_ratio={self.fallback_ratio}, return_ms={self.return_ms}"


class SparseBMM(_SparseMM):
    """C[b] = A[b] @ B[b] with A [B, M, K] spike-sparse."""

    diag_path = score_family = "bmm"

    def forward(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        if a.ndim != 3 or b.ndim != 3:
            raise ValueError("SparseBMM expects [B, M, K] @ [B, K, N]")
        return self._bmm(a, b)


class SparseMatmul(_SparseMM):
    """C = A @ B with A [M, K] or [*, M, K] spike-sparse; B [K, N] or
    [*, K, N] (batched B takes the batched-matmul path)."""

    diag_path = score_family = "matmul"

    def forward(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        if a.ndim > 2:
            lead = a.shape[:-2]
            M, K = a.shape[-2], a.shape[-1]
            N = b.shape[-1]
            if b.ndim > 2:
                out = self._bmm(a.reshape(-1, M, K), b.reshape(-1, K, N))
                return out.reshape(*lead, M, N)
            return self._mm(a.reshape(-1, K), b).reshape(*lead, M, N)
        return self._mm(a, b)

    def _mm(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        self._last_diag = {}
        self.fallback_reason = ""
        if not a.is_cuda:
            self.fallback_reason = "host_tensor"
            self.diag_source = "missing"
            return torch.mm(a.float(), b.float())
        want = self.collect_diag and not self._inference_mode
        res = sparse_matmul_forward(a, b, threshold=self.threshold, return_ms=self.return_ms,
                                    return_avg_active_ratio=want, return_tile_stats=want,
                                    fallback_ratio=self.fallback_ratio)
        self._last_sparse_ms = float(res[1])
        if want:
            self._last_diag = _tile_diag(res[3])
            self._last_diag["avg_active_ratio"] = res[2]
            self._last_diag["active_group_ratio"] = float(res[2])
        return res[0]
