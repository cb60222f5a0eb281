"""FusedSparseConvLIF: stateful conv + LIF module
(drop-in for Ops/sparse_fused_conv_lif.py).

Differences from the reference module, by design:
  * 5-D input [T, B, C, H, W] runs all T steps in one HIP launch (the
    reference loops in Python and launches per step,
    Ops/sparse_fused_conv_lif.py:191-197); the membrane never leaves the
    chip between steps.
  * No spikingjelly dependency: the membrane is a plain attribute `v`
    cleared by `reset()` (spikingjelly's MemoryModule protocol), so
    functional.reset_net works on it.
  * No runtime dense/sparse EMA switch: the fused kernel is always used on
    device tensors.

Host tensors follow the reference's torch fallback
(Ops/sparse_fused_conv_lif.py:271-293).
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _lib
from ..Kernels.fused_conv_lif import _torch_lif_step, sparse_fused_conv_lif_multistep
from ._runtime import OpReporting


def _pair(v):
    return (int(v), int(v)) if isinstance(v, int) else tuple(int(t) for t in v)


class FusedSparseConvLIF(OpReporting, nn.Module):
    def __init__(
        self,
        in_channels,
        out_channels,
        kernel_size,
        stride=1,
        padding=0,
        dilation=1,
        groups=1,
        bias=True,
        tau: float = 2.0,
        v_threshold: float = 1.0,
        v_reset: Optional[float] = 0.0,
        detach_reset: bool = False,
        decay_input: bool = True,
        backend: str = "torch",
        threshold: float = 1e-6,
        block_size=None,
        return_ms: bool = False,
    ):
        super().__init__()
        self.in_channels = int(in_channels)
        self.out_channels = int(out_channels)
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        self.groups = int(groups)
        self.tau = float(tau)
        self.v_threshold = float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.detach_reset = bool(detach_reset)
        self.decay_input = bool(decay_input)
        self.backend = backend
        self.threshold = float(threshold)
        self.block_size = block_size
        self.return_ms = bool(return_ms)

        self.weight = nn.Parameter(torch.empty(self.out_channels, self.in_channels // self.groups, *self.kernel_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(self.out_channels))
        else:
            self.register_parameter("bias", None)
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            bound = 1 / math.sqrt(self.in_channels * self.kernel_size[0] * self.kernel_size[1])
            nn.init.uniform_(self.bias, -bound, bound)

        self.v: Optional[torch.Tensor] = None
        self._w_tap = None
        self._w_tap_key = None
        self._workspace = None
        self._init_reporting("fused_sparse", "fused_conv_lif_hip", "conv", profile_runtime=False)

    # spikingjelly MemoryModule protocol
    def reset(self):
        self.v = None

    @classmethod
    def from_conv_and_lif(cls, conv: nn.Conv2d, lif_node, block_size=None, threshold: float = 1e-6,
                          return_ms: bool = False):
        mod = cls(
            in_channels=conv.in_channels, out_channels=conv.out_channels, kernel_size=conv.kernel_size,
            stride=conv.stride, padding=conv.padding, dilation=conv.dilation, groups=conv.groups,
            bias=conv.bias is not None,
            tau=float(getattr(lif_node, "tau", 2.0)),
            v_threshold=float(getattr(lif_node, "v_threshold", 1.0)),
            v_reset=getattr(lif_node, "v_reset", 0.0),
            detach_reset=bool(getattr(lif_node, "detach_reset", False)),
            decay_input=bool(getattr(lif_node, "decay_input", True)),
            backend=str(getattr(lif_node, "backend", "torch")),
            threshold=threshold, block_size=block_size, return_ms=return_ms,
        )
        with torch.no_grad():
            mod.weight.copy_(conv.weight)
            if conv.bias is not None:
                mod.bias.copy_(conv.bias)
        return mod.to(conv.weight.device)

    def _conv_output_hw(self, h: int, w: int):
        (kh, kw), (sh, sw), (ph, pw), (dh, dw) = self.kernel_size, self.stride, self.padding, self.dilation
        return ((h + 2 * ph - dh * (kh - 1) - 1) // sh) + 1, ((w + 2 * pw - dw * (kw - 1) - 1) // sw) + 1

    def _supports_fused(self, x) -> bool:
        pattern = (self.kernel_size, self.stride, self.padding)
        return (
            x.is_cuda and self.groups == 1 and self.dilation == (1, 1)
            and pattern in (((3, 3), (1, 1), (1, 1)), ((1, 1), (1, 1), (0, 0)))
        )

    def _get_w_tap(self):
        key = (self.weight._version, self.weight.data_ptr(), self.weight.device)
        if self._w_tap is None or self._w_tap_key != key:
            self._w_tap = _lib.tap_major_weight(self.weight)
            self._w_tap_key = key
        return self._w_tap

    def forward(self, x):
        if x.dim() == 5:
            return self._forward_multistep(x)
        if x.dim() == 4:
            return self._forward_multistep(x.unsqueeze(0))[0]
        raise ValueError(f"Expected 4D or 5D input, got {x.dim()}D")

    def _forward_multistep(self, x):
        T, B, C, H, W = (int(v) for v in x.shape)
        out_h, out_w = self._conv_output_hw(H, W)
        state_shape = (B, self.out_channels, out_h, out_w)
        if self.v is None or tuple(self.v.shape) != state_shape or self.v.device != x.device:
            v_init = None  # V_0 = 0 (Ops/sparse_fused_conv_lif.py:202-203)
        else:
            v_init = self.v
        if not self._supports_fused(x):
            self.fallback_reason = "module_dense_path"
            v = torch.zeros(state_shape, dtype=torch.float32, device=x.device) if v_init is None else v_init
            outs = []
            for t in range(T):
                conv = F.conv2d(x[t], self.weight, self.bias, self.stride, self.padding, self.dilation,
                                self.groups).float()
                s, v = _torch_lif_step(conv, v, self.tau, self.v_threshold, self.v_reset, self.decay_input)
                outs.append(s.to(x.dtype))
            self.v = v
            self._last_sparse_ms = 0.0
            return torch.stack(outs, 0)
        if self._workspace is None or self._workspace.device != x.device:
            self._workspace = None
        spikes, v_out, ms = sparse_fused_conv_lif_multistep(
            x, self.weight, self.bias, tau=self.tau, v_threshold=self.v_threshold, v_reset=self.v_reset,
            decay_input=self.decay_input, kernel_size=self.kernel_size[0], threshold=self.threshold,
            v_init=v_init, w_tap=self._get_w_tap(), workspace=self._workspace, return_ms=self.return_ms)
        self.v = v_out
        self._last_sparse_ms = float(ms)
        return spikes

    def extra_repr(self):
        bs = self.block_size if self.block_size is not None else "auto"
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, stride={self.stride}, "
                f"padding={self.padding}, tau={self.tau}, v_threshold={self.v_threshold}, "
                f"v_reset={self.v_reset}, block_size={bs}, fused=True, backend=hip_t_loop")


class SparseConv1x1LIF(nn.Module):
    """A 1x1 stride-1 SparseConv2d followed by its multi-step LIFNode (and an
    optional residual added before the neuron), run as one fused kernel on
    device tensors (Kernels.fused_conv_lif.sparse_conv1x1_lif_multistep).
    Holds the two original modules: host tensors, shapes the kernel does
    not take, and inputs for which the pair is faster (see runs_fused) run
    them one after the other.  The membrane is the LIFNode's `v` (so
    reset_net clears it)."""

    def __init__(self, conv: nn.Module, lif: nn.Module):
        super().__init__()
        self.conv = conv
        self.lif = lif

    @staticmethod
    def eligible(conv: nn.Module, lif: nn.Module) -> bool:
        from ..neuron import LIFNode
        from .sparse_conv2d import SparseConv2d

        return (isinstance(conv, SparseConv2d) and isinstance(lif, LIFNode) and conv.kernel_size == (1, 1)
                and conv.stride == (1, 1) and conv.padding == (0, 0) and conv.groups == 1
                and conv.out_channels % 4 == 0 and lif.step_mode == "m")

    def runs_fused(self, x: torch.Tensor) -> bool:
        """The fused kernel runs for [T, N, C, H, W] device tensors of a
        supported dtype where it is the faster form
        (Kernels.fused_conv_lif.conv1x1_lif_prefers_fused: resident weights,
        or streamed ones with enough samples to fill the GPU), unless a
        dispatch decision put the conv on the dense path.  Otherwise conv and
        neuron run one after the other.  (The two forms agree up to rounding:
        the fused kernel adds the weights into the decayed membrane, the pair
        adds the finished current, so spikes can differ at threshold ties.)"""
        from ..Kernels.fused_conv_lif import CONV1X1_LIF_RESIDENT_CIN, _cus, conv1x1_lif_prefers_fused

        if not (x.dim() == 5 and x.is_cuda and x.dtype in (torch.float32, torch.float16, torch.bfloat16)
                and getattr(self.conv, "backend_mode", "sparse") != "dense"):
            return False
        _, n, c, h, w = (int(v) for v in x.shape)
        if c <= CONV1X1_LIF_RESIDENT_CIN:  # resident weights: no device query needed
            return True
        return conv1x1_lif_prefers_fused(c, self.conv.out_channels, n, h, w, _cus(x.device))

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        from ..Kernels.fused_conv_lif import sparse_conv1x1_lif_multistep

        if not self.runs_fused(x):
            T, N = x.shape[0], x.shape[1]
            y = self.conv(x.flatten(0, 1))
            y = y.reshape(T, N, *y.shape[1:])
            return self.lif(y, residual) if residual is not None else self.lif(y)
        lif = self.lif
        N = int(x.shape[1])
        state = (N, self.conv.out_channels, int(x.shape[3]), int(x.shape[4]))
        # The neuron's membrane carries over only at the same shape and device;
        # otherwise it starts afresh, as LIFNode itself does on a new shape.
        v0 = lif.v if (lif.v is not None and tuple(lif.v.shape) == state and lif.v.device == x.device) else None
        if v0 is None and lif.v_reset is not None and float(lif.v_reset) != 0.0:
            # A fresh LIFNode starts at v_reset (hard reset), not 0.
            v0 = torch.full(state, float(lif.v_reset), dtype=torch.float32, device=x.device)
        spikes, lif.v = sparse_conv1x1_lif_multistep(
            x, self.conv.weight, self.conv.bias, tau=lif.tau, v_threshold=lif.v_threshold, v_reset=lif.v_reset,
            decay_input=lif.decay_input, residual=residual, threshold=self.conv.threshold, v_init=v0,
            w_tap=self.conv._get_w_tap(), map_requests=getattr(lif, "map_requests", None))
        return spikes
