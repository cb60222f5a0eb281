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
    res = sparse_bmm_forward(q_flat, k_t, threshold=threshold, return_ms=return_ms, return_tile_stats=return_tile_stats,
                             alpha=scale)
    attn = res[0].reshape(B, H, S, S)
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


def sparse_spike_attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float = None,
                                   threshold: float = PRESCAN_ACTIVITY_EPS, token_major: bool = False,
                                   out: torch.Tensor = None):
    """(q @ k^T * scale) @ v in one pass per (frame, head), without the
    seq x seq scores (sf_spike_attention; softmax-free attention only).

    token_major=False: q, k, v [B, heads, seq, head_dim] -> y of that shape.
    token_major=True:  q, k, v [B, seq, heads, head_dim] (the projections'
    [B, seq, dim] output viewed per head) -> y [B, seq, heads, head_dim].
    Returns None when the kernel does not take the shape (head_dim not in
    {16, 32, 64} or k, v do not fit in LDS): the caller runs the two stages."""
    from .. import _lib

    if not q.is_cuda or q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return None
    if token_major:
        B, S, H, D = q.shape
        qv, kv, vv = q, k, v
    else:
        B, H, S, D = q.shape
        qv, kv, vv = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if not _lib.spike_attention_supported(S, D):
        return None
    if k.dtype != q.dtype or v.dtype != q.dtype or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must share shape and dtype")
    if qv.stride(3) != 1 or kv.stride() != qv.stride() or vv.stride() != qv.stride():
        qv, kv, vv = (t.contiguous() for t in (qv, kv, vv))
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    yv = out if token_major else out.transpose(1, 2)
    _lib.spike_attention(qv, kv, vv, scale, threshold, yv)
    return out
