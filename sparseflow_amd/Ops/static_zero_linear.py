"""StaticZeroLinear: exact-zero Linear backend (drop-in for
Ops/static_zero_linear.py).  For an all-zero input a Linear is
y = bias (or 0), so the output is the bias broadcast over the input's
leading dimensions, with no read of the input values."""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch
import torch.nn as nn


class StaticZeroLinear(nn.Module):
    def __init__(self, out_features: int, bias: Optional[torch.Tensor] = None):
        super().__init__()
        self.out_features = int(out_features)
        if bias is not None:
            self.register_buffer("bias_buf", bias.detach().float().clone())
        else:
            self.bias_buf = None
        self._forward_count = 0
        self.backend_family = "exact_zero"
        self.diag_path = "staticzero_linear"
        self.fallback_reason = ""

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "StaticZeroLinear":
        return cls(out_features=linear.out_features, bias=linear.bias).to(linear.weight.device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() < 2:
            raise ValueError(f"StaticZeroLinear expects dim>=2 input, got {x.dim()}D")
        self._forward_count += 1
        shape = (*x.shape[:-1], self.out_features)
        if self.bias_buf is None:
            return torch.zeros(shape, dtype=x.dtype, device=x.device)
        return self.bias_buf.to(device=x.device, dtype=x.dtype).expand(shape).clone()

    def get_diag(self) -> Dict[str, Any]:
        return {"backend_family": self.backend_family, "zero_reason": "static_zero_input_linear",
                "diag_path": self.diag_path, "has_bias": self.bias_buf is not None,
                "out_features": self.out_features, "forward_count": self._forward_count}

    def extra_repr(self) -> str:
        return f"out_features={self.out_features}, has_bias={self.bias_buf is not None}"
