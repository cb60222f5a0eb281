"""Dense convolution reference (test infrastructure only).

The reference checks its sparse kernels against torch's dense conv
(Benchmark/ops/conv.py:147-148) and falls back to F.conv2d itself
(Ops/sparse_conv2d.py:819-834).  The oracle runs that same library routine
on the CPU, in float64 for parity checks and in float32 for the CPU
baseline timing.
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from .prescan import active_elements


def masked_input(x: torch.Tensor, threshold: float) -> torch.Tensor:
    """x with every element whose fp16(|x|) <= fp16(threshold) set to 0:
    the spike-sparse operand the sparse kernels actually contract."""
    keep = torch.from_numpy(active_elements(x.detach().cpu().float().numpy(), threshold))
    return x.detach().cpu() * keep.to(x.dtype)


def conv2d_ref(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor], stride: int, padding: int,
               dtype=torch.float64) -> torch.Tensor:
    """F.conv2d on CPU tensors in `dtype` (float64 by default)."""
    xb = x.detach().cpu().to(dtype)
    wb = w.detach().cpu().to(dtype)
    bb = None if b is None else b.detach().cpu().to(dtype)
    return F.conv2d(xb, wb, bb, stride=stride, padding=padding)


def sparse_conv2d_ref(x, w, b, stride: int, padding: int, threshold: float = 1e-6, dtype=torch.float64):
    return conv2d_ref(masked_input(x, threshold), w, b, stride, padding, dtype)


def conv2d_at(x: np.ndarray, w: np.ndarray, b, stride: int, padding: int, n: int, co: int, oh: int, ow: int) -> float:
    """One output element by direct summation in float64 (size independent)."""
    C = x.shape[1]
    k = w.shape[-1]
    acc = 0.0 if b is None else float(b[co])
    for ci in range(C):
        for kh in range(k):
            ih = oh * stride - padding + kh
            if ih < 0 or ih >= x.shape[2]:
                continue
            for kw in range(k):
                iw = ow * stride - padding + kw
                if iw < 0 or iw >= x.shape[3]:
                    continue
                acc += float(x[n, ci, ih, iw]) * float(w[co, ci, kh, kw])
    return acc
