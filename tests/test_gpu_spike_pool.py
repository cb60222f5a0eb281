"""Spike max pooling from a handed spike map (sf_spike_maxpool2d through
Ops.spike_pool.SpikeMaxPool2d) against torch's max pooling of the same dense
spikes: bit-exact, and the output's own map equals the oracle's bitmap of
the pooled spikes."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import prescan as opre
from sparseflow_amd.Kernels import spike_map
from tests.gpu_helpers import DEV, announce, bits_numpy, native_loaded

pytestmark = pytest.mark.gpu

CASES = [
    # (T, N, C, H, W, k, stride, padding, dtype)
    (2, 2, 64, 16, 16, 3, 2, 1, torch.float32),   # the ResNet stem's pooling
    (2, 3, 40, 7, 9, 3, 2, 1, torch.float32),     # ragged channels and frame
    (1, 2, 200, 10, 6, 2, 2, 0, torch.float32),   # 8 words per pixel
    (2, 2, 32, 9, 11, 3, 1, 1, torch.float16),
    (3, 1, 96, 13, 13, 3, 2, 1, torch.bfloat16),
]


@pytest.mark.parametrize("case", CASES)
def test_spike_maxpool_matches_torch(case):
    from sparseflow_amd.neuron import LIFNode
    from sparseflow_amd.Ops.spike_pool import SpikeMaxPool2d

    T, N, C, H, W, k, s, p, dtype = case
    announce(f"spike maxpool {case}")
    g = torch.Generator().manual_seed(C * 7 + H)
    cur = (torch.randn(T, N, C, H, W, generator=g) * 1.5 + 0.6).to(DEV, dtype)
    spike_map.clear()
    spk = LIFNode(step_mode="m")(cur)
    x = spk.flatten(0, 1)
    assert spike_map.lookup(x, 0.0) is not None  # the neuron handed a map
    y = SpikeMaxPool2d(k, s, p)(x)
    torch.cuda.synchronize()
    want = F.max_pool2d(x.float(), k, s, p).to(dtype)
    assert y.dtype == dtype and y.shape == want.shape
    assert torch.equal(y, want)
    assert 0.0 < float(y.float().mean()) < 1.0
    handed = spike_map.lookup(y, 0.0)  # only the spike-map path attaches one
    assert handed is not None
    n, c, ho, wo = (int(v) for v in y.shape)
    cwp = opre.words_per_pixel(c)
    assert np.array_equal(bits_numpy(handed[0], n, ho * wo, cwp), opre.bitmap(y.float().cpu().numpy(), 1e-6))
    assert int(handed[1].abs().sum()) == 0
    assert native_loaded()


def test_spike_maxpool_without_map_is_torch():
    from sparseflow_amd.Ops.spike_pool import SpikeMaxPool2d

    x = (torch.rand(2, 8, 9, 9, generator=torch.Generator().manual_seed(3)) > 0.7).float().to(DEV)
    spike_map.clear()
    y = SpikeMaxPool2d(3, 2, 1)(x)
    assert torch.equal(y, F.max_pool2d(x, 3, 2, 1))
    assert spike_map.lookup(y, 0.0) is None
