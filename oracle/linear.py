"""CPU references for the sparse Linear and batched-matmul kernels
(test infrastructure only).

Reference algorithms:
  linear  y = x @ W^T + b on the spike-sparse x (Kernels/linear.py:460-778;
          its own dense fallback is F.linear, :502-530).  Elements with
          fp16(|x|) <= fp16(thr) count as zero (the activity test of the
          reference's prescan, :129-133,186-191,252-256).
  bmm     C[b] = A[b] @ B[b] with the same activity test on A
          (Kernels/bmm.py:66-184; dense fallback torch.bmm, :221-223).
  metadata (ag_mask, tile_class) over BLOCK_M-row tiles and column groups:
          bit g = any active element of the tile's rows in group g; class
          0 none / 2 all groups / 1 otherwise.  The reference computes it in
          three passes for linear (coarse representative-channel classify,
          zero-candidate refine, exact refine, Kernels/linear.py:110-357),
          which all end in this exact per-group OR, and in one pass for bmm
          (Kernels/bmm.py:66-109).
This build's row bitmap is restated alongside: bits[r, w] bit j =
fp16|x[r, 32w + j]| > fp16(thr); ceil(k/32) words per row, rounded up to a
multiple of 4 beyond two words (padding words zero).
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from .prescan import active_elements


def linear_words_per_row(k: int) -> int:
    w = -(-k // 32)
    return w if w <= 2 else -(-w // 4) * 4


def row_bitmap(x2d: np.ndarray, threshold: float) -> np.ndarray:
    """uint32 [m, words] row bitmap of x [m, k]."""
    m, k = x2d.shape
    words = linear_words_per_row(k)
    act = np.zeros((m, words * 32), dtype=np.uint64)
    act[:, :k] = active_elements(x2d, threshold)
    shifts = np.arange(32, dtype=np.uint64)
    return (act.reshape(m, words, 32) << shifts).sum(axis=-1).astype(np.uint32)


def row_chunk_nonbinary(x2d: np.ndarray, chunk: int = 16) -> np.ndarray:
    """bool per chunk of `chunk` rows: any value outside {0, 1}."""
    m = x2d.shape[0]
    nb = ((x2d != 0) & (x2d != 1)).any(axis=1)
    out = np.zeros(-(-m // chunk), dtype=bool)
    for i in range(out.size):
        out[i] = nb[i * chunk:(i + 1) * chunk].any()
    return out


def masked(x: torch.Tensor, threshold: float) -> torch.Tensor:
    keep = torch.from_numpy(active_elements(x.detach().cpu().float().numpy(), threshold))
    return x.detach().cpu() * keep.to(x.dtype)


def linear_ref(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor], threshold: float = 1e-6,
               dtype=torch.float64) -> torch.Tensor:
    xm = masked(x, threshold).to(dtype)
    return F.linear(xm, w.detach().cpu().to(dtype), None if b is None else b.detach().cpu().to(dtype))


def bmm_ref(a: torch.Tensor, b: torch.Tensor, threshold: float = 1e-6, dtype=torch.float64) -> torch.Tensor:
    return torch.bmm(masked(a, threshold).to(dtype), b.detach().cpu().to(dtype))


def tile_group_metadata(active: np.ndarray, block_m: int, group_size: int):
    """Loop form: (ag_mask int32 [tiles], tile_class int32 [tiles])."""
    rows, cols = active.shape
    ng = -(-cols // group_size)
    nt = -(-rows // block_m)
    masks = np.zeros(nt, dtype=np.int64)
    classes = np.zeros(nt, dtype=np.int32)
    for t in range(nt):
        m = 0
        for g in range(ng):
            blk = active[t * block_m:(t + 1) * block_m, g * group_size:(g + 1) * group_size]
            if blk.any():
                m |= 1 << g
        masks[t] = m
        cnt = bin(m).count("1")
        classes[t] = 0 if cnt == 0 else (2 if cnt == ng else 1)
    masks = np.where(masks >= (1 << 31), masks - (1 << 32), masks).astype(np.int32)
    return masks, classes
