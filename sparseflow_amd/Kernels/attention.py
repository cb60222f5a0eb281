"""Sparse attention stages (drop-in for Kernels/attention.py): Q @ K^T and
attn @ V through the sparse batched matmul, heads folded into the batch
(Kernels/attention.py:27-121).  K^T is passed as a strided view; the
batched-matmul kernel reads it in place."""

from __future__ import annotations

import math

import torch

from ..Utils.config import PRESCAN_ACTIVITY_EPS
from .bmm import sparse_bmm_forward


def sparse_qk_forward(q: torch.Tensor, k: torch.Tensor, scale: float = None, threshold: float = PRESCAN_ACTIVITY_EPS,
                      return_ms: bool = False, return_tile_stats: bool = False):
    """q, k [B, heads, seq, head_dim] -> (q @ k^T * scale [B, heads, seq, seq], ms) [+ (tile_stats,)]."""
    B, H, S, D = q.shape
    if k.shape != q.shape:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} differ")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q_flat = q.reshape(B * H, S, D)
    k_t = k.reshape(B * H, S, D).transpose(1, 2)
    res = sparse_bmm_forward(q_flat, k_t, threshold=threshold, return_ms=return_ms, return_tile_stats=return_tile_stats)
    attn = (res[0] * scale).reshape(B, H, S, S)
    out = (attn, res[1])
    if return_tile_stats:
        out = out + (res[2] if len(res) > 2 else None,)
    return out


def sparse_attn_v_forward(attn: torch.Tensor, v: torch.Tensor, threshold: float = PRESCAN_ACTIVITY_EPS,
                          return_ms: bool = False, return_tile_stats: bool = False):
    """attn [B, heads, sq, sk] @ v [B, heads, sk, head_dim] -> (out, ms) [+ (tile_stats,)]."""
    B, H, SQ, SK = attn.shape
    if v.shape[0] != B or v.shape[1] != H or v.shape[2] != SK:
        raise ValueError(f"attn {tuple(attn.shape)} and v {tuple(v.shape)} do not chain")
    D = v.shape[3]
    res = sparse_bmm_forward(attn.reshape(B * H, SQ, SK), v.reshape(B * H, SK, D), threshold=threshold,
                             return_ms=return_ms, return_tile_stats=return_tile_stats)
    out = (res[0].reshape(B, H, SQ, D), res[1])
    if return_tile_stats:
        out = out + (res[2] if len(res) > 2 else None,)
    return out
