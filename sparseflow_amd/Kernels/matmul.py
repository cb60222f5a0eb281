"""Sparse matmul C = A @ B with A [M, K] spike-sparse (drop-in for
Kernels/matmul.py:152).  A two-operand matmul is the sparse linear with
B as its [K, N] weight^T, so it runs the row-bitmap linear kernels
(sf_linear_*) when N % 4 == 0, else the sparse batched matmul at batch 1;
host tensors run torch.mm, as the reference does (Kernels/matmul.py:181-183)."""

from __future__ import annotations

import torch

from .. import _lib
from ..Utils.config import PRESCAN_ACTIVITY_EPS, SPARSE_DENSE_RATIO_THRESHOLD
from .bmm import sparse_bmm_forward
from .linear import sparse_linear_forward

FALLBACK_RATIO = SPARSE_DENSE_RATIO_THRESHOLD


def sparse_matmul_forward(a: torch.Tensor, b: torch.Tensor, threshold: float = PRESCAN_ACTIVITY_EPS,
                          ag_mask_buf: torch.Tensor = None, tile_class_buf: torch.Tensor = None,
                          return_ms: bool = False, return_avg_active_ratio: bool = False,
                          return_tile_stats: bool = False, fallback_ratio: float = FALLBACK_RATIO):
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError(f"Expected 2D inputs, got {tuple(a.shape)}, {tuple(b.shape)}")
    M, K = a.shape
    K2, N = b.shape
    if K != K2:
        raise ValueError(f"K mismatch: {K} vs {K2}")
    if not a.is_cuda:
        c = torch.mm(a.float(), b.float())
        ret = (c, 0.0)
        if return_avg_active_ratio:
            ret = ret + (1.0,)
        if return_tile_stats:
            ret = ret + (None,)
        return ret
    if N % 4 == 0:
        # weight = b^T as a [N, K] view; its transpose b is the weight^T the kernel reads.
        wt = b.detach().float().contiguous()
        res = sparse_linear_forward(a, wt.t(), None, threshold=threshold, w_t=wt, ag_mask_buf=ag_mask_buf,
                                    tile_class_buf=tile_class_buf, return_ms=return_ms,
                                    return_avg_active_ratio=return_avg_active_ratio,
                                    return_tile_stats=return_tile_stats)
        return res
    res = sparse_bmm_forward(a.unsqueeze(0), b.unsqueeze(0), threshold=threshold, return_ms=return_ms,
                             return_avg_active_ratio=return_avg_active_ratio, return_tile_stats=return_tile_stats)
    return (res[0][0],) + tuple(res[1:])
