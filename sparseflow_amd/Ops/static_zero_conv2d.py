"""Exact-zero convolution backend (drop-in for Ops/static_zero_conv2d.py).

For an all-zero input a convolution is y[n, c, h, w] = bias[c] (or 0).  The
module materialises that from a cached [1, C, H, W] template, with the same
4-D/5-D handling and diagnostics contract as the reference
(Ops/static_zero_conv2d.py:31-238).
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

ZERO_BACKEND_FAMILY = "exact_zero"


def _pair(v):
    return (int(v), int(v)) if isinstance(v, int) else tuple(int(t) for t in v)


class StaticZeroConv2d(nn.Module):
    def __init__(self, out_channels: int, kernel_size, stride=1, padding=0, dilation=1, bias=None,
                 zero_reason: str = "static_zero_input"):
        super().__init__()
        self.out_channels = int(out_channels)
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        if bias is not None:
            self.register_buffer("bias_buf", bias.detach().float().clone())
        else:
            self.bias_buf = None
        self.zero_reason = zero_reason
        self.backend_family = ZERO_BACKEND_FAMILY
        self.diag_path = "staticzero"
        self.fallback_reason = "exact_zero_shortcut"
        self._forward_count = 0
        self.collect_diag = False
        self.profile_runtime = False
        self._last_diag: Dict[str, Any] = {}
        self._last_sparse_ms = 0.0
        self._template_cache: Dict[Tuple, torch.Tensor] = {}

    @classmethod
    def from_conv(cls, conv: nn.Conv2d, zero_reason: str = "static_zero_input"):
        return cls(conv.out_channels, conv.kernel_size, conv.stride, conv.padding, conv.dilation,
                   bias=conv.bias, zero_reason=zero_reason).to(conv.weight.device)

    def _output_hw(self, H: int, W: int) -> Tuple[int, int]:
        (kh, kw), (sh, sw), (ph, pw), (dh, dw) = self.kernel_size, self.stride, self.padding, self.dilation
        return (H + 2 * ph - dh * (kh - 1) - 1) // sh + 1, (W + 2 * pw - dw * (kw - 1) - 1) // sw + 1

    def _get_template(self, device, dtype, H_out: int, W_out: int) -> torch.Tensor:
        key = (str(device), str(dtype), H_out, W_out,
               None if self.bias_buf is None else (self.bias_buf.data_ptr(), self.bias_buf._version))
        tpl = self._template_cache.get(key)
        if tpl is None:
            tpl = make_zero_conv_output(1, self.out_channels, H_out, W_out, self.bias_buf, device, dtype)
            self._template_cache[key] = tpl
        return tpl

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        self._forward_count += 1
        if x.dim() == 4:
            lead = (int(x.shape[0]),)
        elif x.dim() == 5:
            lead = (int(x.shape[0]), int(x.shape[1]))
        else:
            raise ValueError(f"Expected 4D or 5D input, got {x.dim()}D")
        H_out, W_out = self._output_hw(int(x.shape[-2]), int(x.shape[-1]))
        tpl = self._get_template(x.device, x.dtype, H_out, W_out)
        frames = 1
        for v in lead:
            frames *= v
        # A private copy, so in-place consumers (out += identity) are safe.
        y = tpl.expand(frames, -1, -1, -1).clone().reshape(*lead, self.out_channels, H_out, W_out)
        if self.collect_diag:
            self._last_diag = self.get_diag()
        return y

    def get_diag(self) -> Dict[str, Any]:
        return {
            "backend_family": self.backend_family,
            "zero_reason": self.zero_reason,
            "diag_path": self.diag_path,
            "fallback_reason": self.fallback_reason,
            "has_bias": self.bias_buf is not None,
            "out_channels": self.out_channels,
            "forward_count": self._forward_count,
            "template_cache_size": len(self._template_cache),
            "sparse_path_executed": False,
            "sparse_total_ms": 0.0,
        }

    def extra_repr(self) -> str:
        return (f"out_channels={self.out_channels}, kernel_size={self.kernel_size}, stride={self.stride}, "
                f"padding={self.padding}, has_bias={self.bias_buf is not None}, backend={self.backend_family}, "
                f"reason={self.zero_reason}")


def make_zero_conv_output(batch_size: int, out_channels: int, H_out: int, W_out: int,
                          bias: Optional[torch.Tensor], device, dtype=torch.float32) -> torch.Tensor:
    """[batch, C, H_out, W_out] holding bias[c] (or zeros), write-safe."""
    if bias is None:
        return torch.zeros(batch_size, out_channels, H_out, W_out, dtype=dtype, device=device)
    b = bias.detach().to(device=device, dtype=dtype)
    return b.view(1, -1, 1, 1).expand(batch_size, out_channels, H_out, W_out).clone()


def make_synthetic_zero_diag(layer_name: str = "", source: str = "staticzero",
                             total_group_count: float = -1.0, total_tile_count: float = -1.0) -> Dict[str, Any]:
    """Diagnostics record for any exact-zero path (same keys as SparseConv2d)."""
    zt = int(total_tile_count) if total_tile_count >= 0 else -1
    return {
        "active_group_ratio": 0.0, "tile_zero_ratio": 1.0,
        "total_group_count": total_group_count, "nonzero_group_count": 0.0,
        "tile_zero_count": total_tile_count, "total_tile_count": total_tile_count,
        "effective_k_ratio": 0.0, "sparse_compute_ms": -1.0, "sparse_total_ms": -1.0,
        "zero_tiles": zt, "sparse_tiles": 0, "denseish_tiles": 0,
        "stage1_zero_tiles": zt, "stage2_tiles": 0, "prescan_mode": "skipped_zero",
        "_synthetic": True, "_diag_path": source,
        "backend_family": ZERO_BACKEND_FAMILY, "zero_reason": source,
        "layer_name": layer_name,
    }
