"""StaticZeroLinear: the exact-zero Linear backend (drop-in for
Ops/static_zero_linear.py).

A layer that dispatch found to receive only all-zero input computes
y = x @ W^T + b = b, so this module never reads the input values: it returns
the bias repeated over the input's leading dimensions (zeros without a bias)
in the input's dtype.  Inputs of rank < 2 are refused, as in the reference.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ._runtime import bias_rows


class StaticZeroLinear(nn.Module):
    backend_family = "exact_zero"
    diag_path = "staticzero_linear"

    def __init__(self, out_features: int, bias: Optional[torch.Tensor] = None):
        super().__init__()
        self.out_features = int(out_features)
        self.register_buffer("bias_buf", None if bias is None else bias.detach().float().clone())
        self.fallback_reason = ""
        self.calls = 0

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "StaticZeroLinear":
        return cls(linear.out_features, linear.bias).to(linear.weight.device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() < 2:
            raise ValueError(f"StaticZeroLinear takes [..., in_features] input of rank >= 2, not {tuple(x.shape)}")
        self.calls += 1
        return bias_rows(self.bias_buf, tuple(x.shape[:-1]), self.out_features, (), x.dtype, x.device)

    def get_diag(self) -> dict:
        return dict(backend_family=self.backend_family, diag_path=self.diag_path,
                    zero_reason="static_zero_input_linear", out_features=self.out_features,
                    has_bias=self.bias_buf is not None, forward_count=self.calls)

    def extra_repr(self) -> str:
        return f"out_features={self.out_features}, bias={'yes' if self.bias_buf is not None else 'no'}, exact_zero"
