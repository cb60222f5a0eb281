"""Max pooling that takes spike inputs from their spike map.

`SpikeMaxPool2d` is an `nn.MaxPool2d` (same arguments, state and results)
for the max pooling after a spiking network's stem neuron (the reference's
spiking ResNets pool the stem's dense spikes with nn.MaxPool2d,
Models/spiking_resnet.py there).  When its input is a spike tensor for which
a neuron layer handed over a spike map (`Kernels.spike_map`), the pooled
spikes are built from the map alone (`sf_spike_maxpool2d`: the max of 0 / 1
values is the OR of the window's bitmap words) and hand their own map to the
next sparse convolution, which then needs no prescan.  Any other input takes
torch's max pooling.
"""

from __future__ import annotations

import torch
import torch.nn as nn


class SpikeMaxPool2d(nn.MaxPool2d):
    def _spike_path(self, x: torch.Tensor):
        from .. import _lib
        from ..Kernels import spike_map

        if not (x.dim() == 4 and x.is_cuda and x.dtype in (torch.float32, torch.float16, torch.bfloat16)):
            return None
        k, s, p = self.kernel_size, self.stride, self.padding
        if not (isinstance(k, int) and isinstance(s, int) and isinstance(p, int)):
            return None
        if self.dilation != 1 or self.ceil_mode or self.return_indices or x.shape[1] > 256:
            return None
        if not spike_map.recorded(x):
            return None
        # The pooling kernel reads pixel-major words.
        handed = spike_map.lookup(x, 0.0, want=spike_map.PIXEL_MAJOR, consumer=("spike_maxpool", id(self)))
        if handed is None:
            return None
        n, c, h, w = (int(v) for v in x.shape)
        y, (bits, flags) = _lib.spike_maxpool2d(handed[0], n, c, h, w, k, s, p, x.dtype, x.device)
        spike_map.attach(y, n, c, int(y.shape[2]), int(y.shape[3]), bits, flags)
        return y

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self._spike_path(x)
        return y if y is not None else super().forward(x)
