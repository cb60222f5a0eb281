"""Spike sources without spikingjelly.

spikingjelly (the reference's neuron library, pinned at 0.0.0.0.14 in
Benchmark/snn118_config.yml:72) is not installed here.  `LIFNode` and
`IFNode` restate the LIF/IF dynamics the reference relies on
(Core/registry.py:22-29, Ops/sparse_fused_conv_lif.py:283-292) so spiking
models can be built, analysed and optimised.  They are registered as spike
sources by Core.registry.SpikeOpRegistry.default().

Multi-step mode takes [T, B, ...] input and loops over T; single-step mode
takes one step and keeps the membrane in `self.v` until `reset()`.

On ROCm tensors `LIFNode` runs the library's multi-step LIF kernel
(`sf_lif_multistep`: one pass over the T steps with the membrane in
registers, the same arithmetic as the torch path below, bit for bit); the
torch path is the CPU implementation and the checker.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .Kernels.spike_map import LayoutRequests


class BaseNode(nn.Module):
    def __init__(self, v_threshold: float = 1.0, v_reset: Optional[float] = 0.0, detach_reset: bool = False,
                 step_mode: str = "s", backend: str = "torch"):
        super().__init__()
        self.v_threshold = float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.detach_reset = bool(detach_reset)
        if step_mode not in ("s", "m"):
            raise ValueError("step_mode must be 's' or 'm'")
        self.step_mode = step_mode
        self.backend = backend
        self.v: Optional[torch.Tensor] = None

    def reset(self):
        self.v = None

    def _v0(self, like: torch.Tensor) -> torch.Tensor:
        fill = 0.0 if self.v_reset is None else self.v_reset
        return torch.full_like(like, fill, dtype=torch.float32)

    def neuronal_charge(self, x: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError

    def single_step_forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.v is None or self.v.shape != x.shape or self.v.device != x.device:
            self.v = self._v0(x)
        h = self.neuronal_charge(x.float(), self.v)
        spike = (h >= self.v_threshold).to(h.dtype)
        if self.v_reset is None:
            self.v = h - spike * self.v_threshold
        else:
            self.v = torch.where(spike.bool(), torch.full_like(h, self.v_reset), h)
        return spike.to(x.dtype)

    def multi_step_forward(self, x_seq: torch.Tensor) -> torch.Tensor:
        return torch.stack([self.single_step_forward(x_seq[t]) for t in range(x_seq.shape[0])], 0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.multi_step_forward(x) if self.step_mode == "m" else self.single_step_forward(x)

    def extra_repr(self):
        return f"v_threshold={self.v_threshold}, v_reset={self.v_reset}, step_mode={self.step_mode}"


class LIFNode(BaseNode):
    """H = V + (X - (V - V_reset)) / tau  (decay_input=True)
    H = V - (V - V_reset) / tau + X      (decay_input=False); V_reset=0 in
    the decay when soft reset is used."""

    def __init__(self, tau: float = 2.0, decay_input: bool = True, v_threshold: float = 1.0,
                 v_reset: Optional[float] = 0.0, detach_reset: bool = False, step_mode: str = "s",
                 backend: str = "torch"):
        super().__init__(v_threshold, v_reset, detach_reset, step_mode, backend)
        self.tau = float(tau)
        self.decay_input = bool(decay_input)
        self.emit_spike_map = True
        # The layouts this neuron's spike-map consumers read fastest.
        self.map_requests = LayoutRequests()

    def neuronal_charge(self, x, v):
        vr = 0.0 if self.v_reset is None else self.v_reset
        if self.decay_input:
            return v + (x - (v - vr)) / self.tau
        return v - (v - vr) / self.tau + x

    def _hip_steps(self, x_seq: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        from . import _lib
        from .Kernels import spike_map

        lif = _lib.LifParams(self.tau, self.v_threshold, 0.0 if self.v_reset is None else self.v_reset,
                             0 if self.v_reset is None else 1, 1 if self.decay_input else 0)
        v0 = self.v if (self.v is not None and self.v.shape == x_seq.shape[1:] and self.v.device == x_seq.device
                        and self.v.dtype == torch.float32) else None
        # [T, N, C, H, W] spikes also leave as a spike map for the next
        # sparse convolution (skips its prescan).
        want_map = self.emit_spike_map and x_seq.dim() == 5
        layout = self.map_requests.layout
        spikes, self.v, smap = _lib.lif_multistep(x_seq, int(x_seq.shape[0]), lif, v_init=v0, x2=residual,
                                                  spike_map=want_map, map_layout=layout)
        if smap is not None:
            T, N, C, H, W = (int(v) for v in x_seq.shape)
            spike_map.attach(spikes, T * N, C, H, W, smap[0], smap[1], layout, self.map_requests)
        return spikes

    def single_step_forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda:
            return self._hip_steps(x.unsqueeze(0))[0]
        return super().single_step_forward(x)

    def multi_step_forward(self, x_seq: torch.Tensor) -> torch.Tensor:
        if x_seq.is_cuda:
            return self._hip_steps(x_seq)
        return super().multi_step_forward(x_seq)

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """LIF(x), or LIF(x + residual): the sum feeds the neuron directly (on
        the GPU in the same pass; bit-identical to adding first)."""
        if residual is not None:
            if x.is_cuda:
                if self.step_mode == "m":
                    return self._hip_steps(x, residual)
                return self._hip_steps(x.unsqueeze(0), residual.unsqueeze(0))[0]
            x = x + residual
        return super().forward(x)

    def extra_repr(self):
        return f"tau={self.tau}, decay_input={self.decay_input}, " + super().extra_repr()


class IFNode(BaseNode):
    """H = V + X."""

    def neuronal_charge(self, x, v):
        return v + x


def reset_net(net: nn.Module) -> None:
    """Clear the state of every stateful module (spikingjelly's
    functional.reset_net)."""
    for m in net.modules():
        fn = getattr(m, "reset", None)
        if callable(fn):
            fn()
