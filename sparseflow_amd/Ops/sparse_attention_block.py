"""SparseAttentionBlock: a spiking self-attention block rebuilt around the
sparse attention matmuls (drop-in for Ops/sparse_attention_block.py:35-315).

Takes the dense block's q/k/v/proj Linear layers, their BatchNorm1d and
neuron layers, and runs one of the reference's variants on [T, B, N, C]:
  attention_qkav   (q @ k^T) * scale @ v          (on the GPU one fused pass per
                                                  frame and head computing
                                                  q @ (k^T v) * scale, the
                                                  same product without the
                                                  seq x seq scores; else
                                                  SparseAttention qk / av)
  attention_linear q @ (k^T @ v / N)              (two SparseMatmul)
  attention_qkmix  q @ (k^T v / N) + v @ (q^T k / N)
"""

from __future__ import annotations

from typing import Any, Dict

import torch
import torch.nn as nn

from ..Kernels.attention import sparse_spike_attention_forward
from .sparse_attention import SparseAttention
from .sparse_bmm import SparseMatmul
from .sparse_linear import SparseLinear


def _attr(module: nn.Module, name: str, default):
    return getattr(module, name, default)


class SparseAttentionBlock(nn.Module):
    def __init__(self, dense_attn: nn.Module, variant: str, threshold: float = 1e-6, return_ms: bool = False,
                 profile_runtime: bool = False):
        super().__init__()
        v = str(variant)
        v = {"attention_proj_linear": "attention_linear", "attention_matmul": "attention_qkav"}.get(v, v)
        if v not in ("attention_qkav", "attention_linear", "attention_qkmix"):
            raise ValueError(f"Unsupported attention variant: {variant}")
        self.variant = v
        self.threshold = float(threshold)
        self.return_ms = bool(return_ms)
        # The projections run as SparseLinear too (their inputs are spike
        # maps or sums of a few); the reference keeps them dense.
        for name in ("q", "k", "v", "proj"):
            lin = getattr(dense_attn, name)
            if isinstance(lin, nn.Linear):
                lin = SparseLinear.from_dense(lin, threshold=self.threshold, return_ms=self.return_ms)
            setattr(self, name, lin)
        self.q_bn = _attr(dense_attn, "q_bn", nn.Identity())
        self.k_bn = _attr(dense_attn, "k_bn", nn.Identity())
        self.v_bn = _attr(dense_attn, "v_bn", nn.Identity())
        self.proj_bn = _attr(dense_attn, "proj_bn", nn.Identity())
        self.q_lif = _attr(dense_attn, "q_lif", nn.Identity())
        self.k_lif = _attr(dense_attn, "k_lif", nn.Identity())
        self.v_lif = _attr(dense_attn, "v_lif", nn.Identity())
        self.attn_lif = _attr(dense_attn, "attn_lif", nn.Identity())
        self.proj_lif = _attr(dense_attn, "proj_lif", nn.Identity())
        self.dim = int(_attr(dense_attn, "dim", self.q.out_features))
        self.num_heads = int(_attr(dense_attn, "num_heads", 1))
        self.head_dim = int(_attr(dense_attn, "head_dim", max(1, self.dim // max(1, self.num_heads))))
        self._sparse_attn = SparseAttention(self.num_heads, self.head_dim, self.threshold, self.return_ms)
        n_mm = {"attention_qkav": 0, "attention_linear": 2, "attention_qkmix": 4}[v]
        self._mms = nn.ModuleList(SparseMatmul(self.threshold, 0.85, self.return_ms, profile_runtime)
                                  for _ in range(n_mm))
        self.collect_diag = False
        self.profile_runtime = bool(profile_runtime)
        self._inference_mode = False
        self._last_sparse_ms = 0.0
        self._last_diag: Dict[str, Any] = {}
        self.backend_family = "sparse_kernel"
        self.diag_path = "attention_block"
        self.fallback_reason = ""
        self.meta_source = "measured"
        self.diag_source = "measured"
        self.support_status = "supported"
        self.score_family = "attn_linear" if v == "attention_linear" else "attn_matmul"

    @classmethod
    def from_dense(cls, dense_attn: nn.Module, variant: str, threshold: float = 1e-6, return_ms: bool = False,
                   profile_runtime: bool = False) -> "SparseAttentionBlock":
        return cls(dense_attn, variant, threshold, return_ms, profile_runtime)

    def set_inference_mode(self, enabled: bool):
        self._inference_mode = bool(enabled)
        if enabled:
            self.collect_diag = False
            self.profile_runtime = False
        self._sync_inner()

    def _sync_inner(self):
        for m in [self._sparse_attn, *self._mms]:
            m.collect_diag = self.collect_diag
            m.return_ms = self.return_ms
            m.profile_runtime = self.profile_runtime
            m.set_inference_mode(self._inference_mode)

    def _linear_bn_lif(self, x, linear, bn, lif):
        t, b, n, c = x.shape
        y = linear(x.flatten(0, 1))
        y = bn(y.transpose(-1, -2)).transpose(-1, -2).reshape(t, b, n, -1).contiguous()
        return lif(y)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        t, b, n, c = x.shape
        self._sync_inner()
        self._last_diag = {}
        self.diag_path = self.variant
        q = self._linear_bn_lif(x, self.q, self.q_bn, self.q_lif)
        k = self._linear_bn_lif(x, self.k, self.k_bn, self.k_lif)
        v = self._linear_bn_lif(x, self.v, self.v_bn, self.v_lif)
        y = None
        if self.variant == "attention_qkav" and q.is_cuda:
            # One pass per (frame, head) over the token-major projections:
            # no head permutes, no seq x seq scores.
            tok = (t * b, n, self.num_heads, self.head_dim)
            y = sparse_spike_attention_forward(q.reshape(tok), k.reshape(tok), v.reshape(tok),
                                               self._sparse_attn.scale, self.threshold, token_major=True)
        if y is not None:
            self._last_sparse_ms = 0.0
            self.diag_source = "missing"
            y = self.attn_lif(y.reshape(t, b, n, c))
            y2 = self.proj(y.flatten(0, 1))
            y2 = self.proj_bn(y2.transpose(-1, -2)).transpose(-1, -2).reshape(t, b, n, c).contiguous()
            return self.proj_lif(y2)
        heads = lambda z: z.reshape(t, b, n, self.num_heads, self.head_dim).permute(0, 1, 3, 2, 4).contiguous()  # noqa: E731
        q, k, v = heads(q), heads(k), heads(v)
        if self.variant == "attention_qkav":
            shp = (t * b, self.num_heads, n, self.head_dim)
            attn = self._sparse_attn.qk(q.reshape(shp), k.reshape(shp))
            y = self._sparse_attn.av(attn, v.reshape(shp)).reshape(t, b, self.num_heads, n, self.head_dim)
            self._last_sparse_ms = float(self._sparse_attn._last_sparse_ms)
            self._last_diag = dict(self._sparse_attn._last_diag.get("qk_stats") or {})
        else:
            nf = float(max(1, n))
            kv = self._mms[0](k.transpose(-2, -1).contiguous(), v) / nf
            y = self._mms[1](q, kv)
            if self.variant == "attention_qkmix":
                qk = self._mms[2](q.transpose(-2, -1).contiguous(), k) / nf
                y = y + self._mms[3](v, qk)
            self._last_sparse_ms = sum(float(m._last_sparse_ms) for m in self._mms)
            self._last_diag = dict(self._mms[0]._last_diag)
        self.diag_source = "measured" if self._last_diag else "missing"
        y = y.to(x.dtype).transpose(2, 3).reshape(t, b, n, c).contiguous()
        y = self.attn_lif(y)
        y2 = self.proj(y.flatten(0, 1))
        y2 = self.proj_bn(y2.transpose(-1, -2)).transpose(-1, -2).reshape(t, b, n, c).contiguous()
        return self.proj_lif(y2)

    def extra_repr(self) -> str:
        return (f"variant={self.variant}, dim={self.dim}, num_heads={self.num_heads}, head_dim={self.head_dim}, "
                f"threshold={self.threshold}")
