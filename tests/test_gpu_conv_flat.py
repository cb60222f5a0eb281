"""Flat-tile Stage 2 for 1x1 stride-1 convolutions (any C_in, C_out % 4 == 0).

Same bar as the gather kernel: fp32 within 1e-4 abs + 1e-4 rel of float64
F.conv2d on the spike-masked input, fp16/bf16 within 1e-2, bit-identical
repeats.  Every case also checks which Stage-2 kernel produced the result:
weights resident for C_in <= 512, streamed through two LDS buffers beyond;
float4 stores when h*w % 4 == 0, element stores otherwise.
"""

import pytest
import torch

from oracle import conv as oconv
from sparseflow_amd import _lib
from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward
from tests.gpu_helpers import DEV, announce, close, native_loaded, spikes

pytestmark = pytest.mark.gpu

FP32_TOL = dict(atol=1e-4, rtol=1e-4)


def _weights(c_out, c_in, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(c_out, c_in, 1, 1, generator=g) * (2.0 / c_in) ** 0.5


def _run(x, w, b, **kw):
    """sparse_conv2d_forward with kernel timing on; returns (y, kernels)."""
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        y = sparse_conv2d_forward(x, w, b, kernel_size=1, stride=1, padding=0, **kw)[0]
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return y, {k: c for k, (c, _) in stats.items() if c > 0}


CASES = [
    # (N, C_in, H, W, C_out)
    (4, 256, 56, 56, 64),    # BASELINE config 2 layer shape (8 words, one chunk)
    (2, 64, 56, 56, 256),    # ResNet50 layer1 conv3 shape (2 words, four groups)
    (2, 512, 28, 28, 128),   # two chunks, resident
    (2, 1024, 14, 14, 256),  # four chunks, streamed
    (2, 2048, 7, 7, 512),    # eight chunks, 49-pixel planes: element stores
    (3, 1, 5, 7, 4),         # one channel, 35-pixel planes
    (2, 33, 9, 9, 12),       # two words, second nearly empty; ragged group
    (2, 300, 10, 10, 68),    # last chunk partially filled, ragged second group
    (17, 128, 8, 8, 64),     # one tile per frame, passes past the end
    (1, 96, 3, 100, 20),     # last tile of the frame 44 pixels
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("density", [0.0, 0.01, 0.3])
def test_flat_fp32_matches_dense(case, density):
    N, C, H, W, Co = case
    announce(f"flat {case} p={density}")
    x = spikes((N, C, H, W), density, seed=N * 7 + C)
    w = _weights(Co, C, seed=C + Co)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(3)) * 0.1
    y, kernels = _run(x.to(DEV), w.to(DEV), b.to(DEV))
    assert "conv_flat" in kernels and "conv_gather" not in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, 1, 0), **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert native_loaded()


def test_flat_dense_input():
    # 90% density: most words hold many spikes.
    x = spikes((2, 256, 16, 16), 0.9, seed=21)
    w = _weights(64, 256, seed=22)
    announce("flat dense")
    y, kernels = _run(x.to(DEV), w.to(DEV), None)
    assert "conv_flat" in kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 1, 0), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_flat_all_ones_input():
    x = torch.ones(2, 1024, 6, 8)
    w = _weights(64, 1024, seed=9)
    announce("flat all-ones")
    y, kernels = _run(x.to(DEV), w.to(DEV), None)
    assert "conv_flat" in kernels
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, None, 1, 0), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_flat_value_path_only_where_flagged():
    g = torch.Generator().manual_seed(4)
    x = spikes((3, 256, 32, 32), 0.05, seed=6)
    x[1, :, 10:12] = x[1, :, 10:12] * torch.randn(256, 2, 32, generator=g)
    x[2, 5, 31, 31] = -2.5
    x[0, 0, 0, 0] = 3e-7       # below the activity threshold: dropped
    w = _weights(64, 256, seed=10)
    announce("flat value path")
    y, kernels = _run(x.to(DEV), w.to(DEV), None)
    assert "conv_flat" in kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 1, 0), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_flat_half_activations(dtype):
    x = spikes((4, 256, 14, 14), 0.05, seed=11)
    x[0, :, 3] = x[0, :, 3] * 0.5   # a value-path chunk in reduced precision
    w = _weights(128, 256, seed=12)
    b = torch.linspace(-0.5, 0.5, 128)
    announce(f"flat {dtype}")
    xr = x.to(dtype).float()
    y, kernels = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV))
    assert "conv_flat" in kernels and y.dtype == dtype
    ok, err, _ = close(y, oconv.conv2d_ref(xr, w, b, 1, 0), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"
    y32, _ = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), output_dtype=torch.float32)
    assert y32.dtype == torch.float32
    ok, err, _ = close(y32, oconv.conv2d_ref(xr, w, b, 1, 0), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_flat_deterministic_bitwise():
    x = spikes((32, 256, 28, 28), 0.02, seed=13).to(DEV)
    w = _weights(64, 256, seed=14).to(DEV)
    announce("flat determinism")
    y1, _ = _run(x, w, None)
    y2, _ = _run(x, w, None)
    assert torch.equal(y1, y2)


def test_flat_and_gather_agree():
    # C_out = 6 is not a multiple of 4, so the same input goes through the
    # gather kernel; its channels match the flat kernel's first six.
    x = spikes((4, 128, 12, 20), 0.03, seed=15)
    w = _weights(8, 128, seed=16)
    announce("flat vs gather")
    y_flat, k1 = _run(x.to(DEV), w.to(DEV), None)
    y_gather, k2 = _run(x.to(DEV), w[:6].contiguous().to(DEV), None)
    assert "conv_flat" in k1 and "conv_gather" in k2
    assert torch.allclose(y_flat[:, :6], y_gather, atol=1e-5, rtol=1e-5)


def _random_flat_cases(n, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(n):
        N = int(torch.randint(1, 9, (1,), generator=g))
        C = int(torch.randint(1, 1100, (1,), generator=g))
        Co = 4 * int(torch.randint(1, 80, (1,), generator=g))
        H = int(torch.randint(1, 30, (1,), generator=g))
        W = int(torch.randint(1, 40, (1,), generator=g))
        dens = [0.005, 0.05, 0.3][int(torch.randint(0, 3, (1,), generator=g))]
        out.append((N, C, H, W, Co, dens))
    return out


@pytest.mark.parametrize("case", _random_flat_cases(30, 5150))
def test_flat_random_shapes(case):
    # Random geometry through the 1x1 pixel-tile kernel: resident and
    # streamed chunks, ragged words and channel groups, planes from one
    # pixel, workgroups of one to sixteen wavefronts (sized so that every
    # CU makes the same number of passes).
    N, C, H, W, Co, dens = case
    announce(f"flat random {case}")
    x = spikes((N, C, H, W), dens, seed=C + H * W)
    w = _weights(Co, C, seed=Co + N)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(C)) * 0.1
    y, kernels = _run(x.to(DEV), w.to(DEV), b.to(DEV))
    assert "conv_flat" in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, 1, 0), **FP32_TOL)
    assert ok, f"max abs err {err}"
