"""Matrix-core Stage 2 (k_conv_mfma, chosen by sf_conv2d_sparse for 3x3
layers whose whole reduction C_in * 9 is at most 32) against the float64 dense-conv
oracle on the prescan-masked input: fp32 within 1e-4 abs + 1e-4 rel.

Covers the config-5 patch-embed stem (3 -> 384 on dense N(0,1) frames),
ragged channel and pixel counts, stride 2, binary spikes, and
values under the activity threshold (which must count as zero, as on every
other path); the timing registry shows the matrix-core kernel ran."""

import pytest
import torch

from oracle import conv as oconv
from sparseflow_amd import _lib
from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward
from tests.gpu_helpers import DEV, announce, close, native_loaded, spikes

pytestmark = pytest.mark.gpu

CASES = [
    # (N, C_in, H, W, C_out, k, s, input)
    (16, 3, 32, 32, 384, 3, 1, "normal"),     # config-5 stem shape (fewer frames)
    (3, 3, 17, 13, 40, 3, 1, "normal"),       # C_out < 64, h*w not a multiple of 4
    (2, 2, 9, 11, 70, 3, 2, "normal"),        # stride 2, two channel groups, ragged
    (4, 1, 7, 5, 64, 3, 1, "spikes"),
    (2, 3, 12, 10, 100, 3, 1, "spikes"),      # binary spikes
    (4, 3, 20, 20, 128, 3, 2, "normal"),      # 3x3 stride 2, stem-like
    (5, 3, 32, 32, 96, 3, 1, "tiny"),         # values below the threshold count as zero
]


def _input(shape, kind, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "spikes":
        return spikes(shape, 0.2, seed=seed)
    x = torch.randn(shape, generator=g)
    if kind == "tiny":  # a third of the values under the 1e-6 activity threshold
        x = torch.where(torch.rand(shape, generator=g) < 0.33, x * 1e-7, x)
    return x


@pytest.mark.parametrize("case", CASES)
def test_mfma_conv_matches_dense(case):
    N, C, H, W, Co, k, s, kind = case
    p = (k - 1) // 2
    announce(f"conv mfma {case}")
    x = _input((N, C, H, W), kind, seed=N + C + Co)
    g = torch.Generator().manual_seed(Co)
    w = torch.randn(Co, C, k, k, generator=g) * (2.0 / (C * k * k)) ** 0.5
    b = torch.randn(Co, generator=g) * 0.1
    _lib.timing_reset()
    _lib.timing_enable(True)
    y, ms, meta = sparse_conv2d_forward(x.to(DEV), w.to(DEV), b.to(DEV), kernel_size=k, stride=s, padding=p,
                                        return_backend_meta=True)
    torch.cuda.synchronize()
    stats = _lib.timing_collect()
    _lib.timing_enable(False)
    assert meta["backend"] == "sparse_hip"
    assert stats["conv_mfma"][0] == 1, stats
    ref = oconv.sparse_conv2d_ref(x, w, b, s, p)
    ok, err, excess = close(y, ref, atol=1e-4, rtol=1e-4)
    assert ok, f"max err {err:.3e} (excess {excess:.3e})"
    if kind == "tiny":
        # Against the unmasked input the result must differ: the masked
        # elements really were dropped.
        assert not torch.allclose(y.double().cpu(), oconv.conv2d_ref(x, w, b, s, p), atol=1e-9, rtol=0)
    # Repeat: bit-identical.
    y2 = sparse_conv2d_forward(x.to(DEV), w.to(DEV), b.to(DEV), kernel_size=k, stride=s, padding=p)[0]
    assert torch.equal(y, y2)
    assert native_loaded()
