"""Spike-source / target-op registry (drop-in for Core/registry.py).

Default spike sources are this package's LIFNode / IFNode plus, when
spikingjelly is importable, its LIFNode / IFNode / ParametricLIFNode
(Core/registry.py:15-34).  Users register further spike types with
`register`.
"""

from __future__ import annotations

from typing import Tuple, Type

import torch.nn as nn

from .. import neuron as _neuron

_DEFAULT_SPIKE_OPS = None


def _get_default_spike_ops():
    global _DEFAULT_SPIKE_OPS
    if _DEFAULT_SPIKE_OPS is None:
        ops = [_neuron.LIFNode, _neuron.IFNode]
        try:
            from spikingjelly.activation_based import neuron as sj_neuron  # optional dependency

            ops.extend([sj_neuron.LIFNode, sj_neuron.IFNode, sj_neuron.ParametricLIFNode])
        except ImportError:
            pass
        _DEFAULT_SPIKE_OPS = tuple(ops)
    return _DEFAULT_SPIKE_OPS


class SpikeOpRegistry:
    """Spike-op types plus replaceable target families (Conv1d/2d/3d,
    Linear); only Conv2d targets are replaced by this build."""

    def __init__(self):
        self._spike_op_types: list = []
        self._target_op_types: list = [nn.Conv1d, nn.Conv2d, nn.Conv3d, nn.Linear]

    def register(self, op_type: Type[nn.Module]):
        if op_type not in self._spike_op_types:
            self._spike_op_types.append(op_type)
        return self

    def register_many(self, op_types):
        for t in op_types:
            self.register(t)
        return self

    def register_target(self, op_type: Type[nn.Module]):
        if op_type not in self._target_op_types:
            self._target_op_types.append(op_type)
        return self

    def is_spike_op(self, module: nn.Module) -> bool:
        return bool(self._spike_op_types) and isinstance(module, tuple(self._spike_op_types))

    def is_target_conv1d(self, module: nn.Module) -> bool:
        return isinstance(module, nn.Conv1d)

    def is_target_conv2d(self, module: nn.Module) -> bool:
        return isinstance(module, nn.Conv2d)

    def is_target_conv3d(self, module: nn.Module) -> bool:
        return isinstance(module, nn.Conv3d)

    def is_target_linear(self, module: nn.Module) -> bool:
        return isinstance(module, nn.Linear)

    def is_target_depthwise_conv2d(self, module: nn.Module) -> bool:
        return (isinstance(module, nn.Conv2d) and module.groups == module.in_channels
                and module.out_channels == module.in_channels)

    @property
    def spike_op_types(self) -> Tuple:
        return tuple(self._spike_op_types)

    @property
    def target_op_types(self) -> Tuple:
        return tuple(self._target_op_types)

    @classmethod
    def default(cls) -> "SpikeOpRegistry":
        return cls().register_many(_get_default_spike_ops())
