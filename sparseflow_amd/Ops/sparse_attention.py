"""SparseAttention: parameter-free Q @ K^T and attn @ V for spiking
transformers (drop-in for Ops/sparse_attention.py:29-157).  Device tensors
run the sparse batched-matmul kernel (heads folded into the batch, K^T read
in place); host tensors run torch.matmul in f32 as the reference does."""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from ..Kernels.attention import sparse_attn_v_forward, sparse_qk_forward, sparse_spike_attention_forward
from ._runtime import OpReporting


class SparseAttention(OpReporting, nn.Module):
    def __init__(self, num_heads: int = 8, head_dim: int = 64, threshold: float = 1e-6, return_ms: bool = False):
        super().__init__()
        self.num_heads = int(num_heads)
        self.head_dim = int(head_dim)
        self.scale = 1.0 / math.sqrt(head_dim)
        self.threshold = float(threshold)
        self.return_ms = bool(return_ms)
        self._init_reporting("sparse_kernel", "attention", "attn_matmul", profile_runtime=False)

    def qk(self, q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
        """[B, heads, seq, head_dim] x2 -> attention logits [B, heads, seq, seq] (scaled)."""
        self.fallback_reason = ""
        if not q.is_cuda:
            self.fallback_reason = "host_tensor"
            self.diag_source = "missing"
            return self._dense_qk(q, k)
        want = self.collect_diag and not self._inference_mode
        res = sparse_qk_forward(q, k, scale=self.scale, threshold=self.threshold, return_ms=self.return_ms,
                                return_tile_stats=want)
        self._last_sparse_ms = float(res[1])
        if want and len(res) > 2:
            self._last_diag["qk_stats"] = res[2]
            self.diag_source = "measured"
        return res[0]

    def av(self, attn: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """attn [B, heads, sq, sk] @ v [B, heads, sk, head_dim]."""
        if not attn.is_cuda:
            self.fallback_reason = "host_tensor"
            self.diag_source = "missing"
            return self._dense_av(attn, v)
        want = self.collect_diag and not self._inference_mode
        res = sparse_attn_v_forward(attn, v, threshold=self.threshold, return_ms=self.return_ms,
                                    return_tile_stats=want)
        self._last_sparse_ms += float(res[1])
        if want and len(res) > 2:
            self._last_diag["av_stats"] = res[2]
        return res[0]

    def qkv(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """av(qk(q, k), v) in one fused pass where the kernel takes the shape
        (no seq x seq scores); [B, heads, seq, head_dim] in and out."""
        if q.is_cuda:
            y = sparse_spike_attention_forward(q, k, v, self.scale, self.threshold)
            if y is not None:
                return y
        return self.av(self.qk(q, k), v)

    def _dense_qk(self, q, k):
        return torch.matmul(q.float(), k.float().transpose(-2, -1)) * self.scale

    def _dense_av(self, attn, v):
        return torch.matmul(attn.float(), v.float())

    def extra_repr(self):
        return (f"num_heads={self.num_heads}, head_dim={self.head_dim}, scale={self.scale:.4f}, "
                f"threshold={self.threshold}")
