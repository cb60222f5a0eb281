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

from ._runtime import ExactZeroOp


class StaticZeroLinear(ExactZeroOp, nn.Module):
    def __init__(self, out_features: int, bias: Optional[torch.Tensor] = None):
        super().__init__()
        self.out_features = int(out_features)
        self._init_exact_zero(bias, "static_zero_input_linear", "staticzero_linear")
        self.fallback_reason = ""

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "StaticZeroLinear":
        return cls(linear.out_features, linear.bias).to(linear.weight.device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() < 2:
            raise ValueError(f"StaticZeroLinear takes [..., in_features] input of rank >= 2, not {tuple(x.shape)}")
        return self._zero_output(tuple(x.shape[:-1]), self.out_features, (), x)

    def get_diag(self) -> dict:
        return self._zero_diag(out_features=self.out_features)

    def extra_repr(self) -> str:
        return f"out_features={self.out_features}, bias={'yes' if self.bias_buf is not None else 'no'}, exact_zero"
