"""StaticZeroConv2d: the exact-zero Conv2d backend.

Drop-in for the reference's Ops/static_zero_conv2d.py:31-238.  What is kept
from there is the interface: the class name, constructor arguments,
`from_conv`, 4-D / 5-D input, the `get_diag` key names and the two module
functions `make_zero_conv_output` and `make_synthetic_zero_diag`.

When dispatch has shown a layer's input to be exactly zero, every output
element is bias[c] (0 without a bias) whatever the weights.  The module
therefore keeps only what that output depends on -- C_out, the geometry that
fixes H_out x W_out, the bias -- and returns `_runtime.bias_rows`, the same
tensor SparseConv2d's own zero path and StaticZeroLinear return.  Each call
gets a fresh tensor, so callers may add into it in place (a bottleneck's
`out += identity`).  No per-shape template is cached: the broadcast bias
costs one fill kernel per call, the same as copying a cached template.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from ._runtime import ExactZeroOp, bias_rows

ZERO_BACKEND_FAMILY = ExactZeroOp.backend_family


def _as_pair(v) -> Tuple[int, int]:
    return (int(v), int(v)) if isinstance(v, int) else tuple(int(t) for t in v)


def _conv_out_len(n: int, k: int, s: int, p: int, d: int) -> int:
    """Output length of one spatial axis (the F.conv2d formula)."""
    return (n + 2 * p - d * (k - 1) - 1) // s + 1


class StaticZeroConv2d(ExactZeroOp, nn.Module):
    """A Conv2d whose input is known to be all zero: y = bias broadcast."""

    def __init__(self, out_channels: int, kernel_size, stride=1, padding=0, dilation=1,
                 bias: Optional[torch.Tensor] = None, zero_reason: str = "static_zero_input"):
        super().__init__()
        self.out_channels = int(out_channels)
        self.kernel_size = _as_pair(kernel_size)
        self.stride = _as_pair(stride)
        self.padding = _as_pair(padding)
        self.dilation = _as_pair(dilation)
        self._init_exact_zero(bias, zero_reason, "staticzero")

    @classmethod
    def from_conv(cls, conv: nn.Conv2d, zero_reason: str = "static_zero_input") -> "StaticZeroConv2d":
        mod = cls(conv.out_channels, conv.kernel_size, conv.stride, conv.padding, conv.dilation,
                  bias=conv.bias, zero_reason=zero_reason)
        return mod.to(conv.weight.device)

    def output_hw(self, h_in: int, w_in: int) -> Tuple[int, int]:
        geo = zip(self.kernel_size, self.stride, self.padding, self.dilation)
        return tuple(_conv_out_len(n, *g) for n, g in zip((h_in, w_in), geo))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() not in (4, 5):
            raise ValueError(f"Expected 4D or 5D input, got {x.dim()}D")
        lead = tuple(x.shape[:-3])  # (N,) or (T, N)
        return self._zero_output(lead, self.out_channels, self.output_hw(x.shape[-2], x.shape[-1]), x)

    def get_diag(self) -> Dict[str, Any]:
        # template_cache_size stays in the record for readers of the schema;
        # this module caches no template.
        return self._zero_diag(out_channels=self.out_channels, template_cache_size=0)

    def extra_repr(self) -> str:
        return (f"out_channels={self.out_channels}, kernel_size={self.kernel_size}, stride={self.stride}, "
                f"padding={self.padding}, bias={'yes' if self.bias_buf is not None else 'no'}, "
                f"{self.backend_family} ({self.zero_reason})")


def make_zero_conv_output(batch_size: int, out_channels: int, H_out: int, W_out: int,
                          bias: Optional[torch.Tensor], device, dtype=torch.float32) -> torch.Tensor:
    """[batch_size, out_channels, H_out, W_out], bias[c] everywhere (zeros
    without a bias): the conv output of an all-zero batch."""
    return bias_rows(bias, (int(batch_size),), int(out_channels), (int(H_out), int(W_out)), dtype, device)


def make_synthetic_zero_diag(layer_name: str = "", source: str = "staticzero",
                             total_group_count: float = -1.0, total_tile_count: float = -1.0) -> Dict[str, Any]:
    """The SparseConv2d diagnostics record of a layer that ran no sparse
    work because its input was exactly zero: nothing active, every tile
    zero, no kernel time (-1 = not measured).  Counts that are unknown stay
    -1."""
    tiles = float(total_tile_count)
    zero_tiles = int(tiles) if tiles >= 0 else -1
    record: Dict[str, Any] = {
        # activity: none
        "active_group_ratio": 0.0, "effective_k_ratio": 0.0, "nonzero_group_count": 0.0,
        "total_group_count": total_group_count,
        # tiles: all of them zero, none sent to Stage 2
        "total_tile_count": total_tile_count, "tile_zero_count": total_tile_count, "tile_zero_ratio": 1.0,
        "zero_tiles": zero_tiles, "stage1_zero_tiles": zero_tiles,
        "sparse_tiles": 0, "denseish_tiles": 0, "stage2_tiles": 0,
        # timing: no kernel ran
        "sparse_compute_ms": -1.0, "sparse_total_ms": -1.0,
        "prescan_mode": "skipped_zero",
    }
    record.update(_synthetic=True, _diag_path=source, backend_family=ZERO_BACKEND_FAMILY, zero_reason=source,
                  layer_name=layer_name)
    return record
