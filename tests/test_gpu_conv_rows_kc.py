"""Row-tile scatter Stage 2, K-chunked variant (3x3 stride 1, frame width 28 or 14, any C_in).

Same bar as the gather kernel: fp32 within 1e-4 abs + 1e-4 rel of float64
F.conv2d on the spike-masked input, fp16/bf16 within 1e-2, bit-identical
repeats.  Every case also checks that the K-chunked row kernel produced the
result: weights resident for C_in <= 64, streamed through two LDS buffers
otherwise.
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
    return torch.randn(c_out, c_in, 3, 3, generator=g) * (2.0 / (c_in * 9)) ** 0.5


def _run(x, w, b, **kw):
    """sparse_conv2d_forward with kernel timing on; returns (y, kernels)."""
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        y = sparse_conv2d_forward(x, w, b, kernel_size=3, stride=1, padding=1, **kw)[0]
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return y, {k: c for k, (c, _) in stats.items() if c > 0}


CASES = [
    # (N, C_in, H, W, C_out)
    (4, 128, 28, 28, 128),  # ResNet50 layer2 conv2 shape (4 chunks, streamed)
    (4, 256, 14, 14, 256),  # ResNet50 layer3 conv2 shape (8 chunks)
    (3, 64, 28, 28, 64),    # two chunks: resident, no barriers
    (2, 4, 27, 28, 4),      # four channels, odd height (last tile one row)
    (2, 64, 13, 14, 64),    # odd plane size (13*14 % 4 != 0): goes to the pixel-tile kernel
    (5, 96, 10, 14, 100),   # three chunks, last tile two rows, ragged group
    (2, 33, 2, 14, 64),     # two-row frames: one tile per frame
    (1, 300, 14, 14, 64),   # last chunk partially filled
    (17, 128, 14, 14, 192), # passes whose last tiles are past the end
    (4, 160, 28, 28, 128),  # C_in > 128: the row-band kernel at 28x28
    (3, 192, 10, 14, 100),  # C_in > 128, last tile two rows, ragged group
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("density", [0.0, 0.01, 0.3])
def test_rows_kc_fp32_matches_dense(case, density):
    N, C, H, W, Co = case
    announce(f"rows_kc {case} p={density}")
    x = spikes((N, C, H, W), density, seed=N * 5 + C)
    w = _weights(Co, C, seed=C + Co)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(3)) * 0.1
    y, kernels = _run(x.to(DEV), w.to(DEV), b.to(DEV))
    # The pixel-tile kernel takes odd planes and C_in <= 128 (its weights then
    # stay resident in LDS); the K-chunked row kernel the rest.
    expect = "conv_px3" if (H * W) % 4 or C <= 128 else "conv_rows_kc"
    # prescan_pack + one conv kernel (+ the dense-tile kernel after the row
    # kernel, which leaves at once when nothing was queued)
    extra = {"conv_dense_mfma"} if expect == "conv_rows_kc" else set()
    assert expect in kernels and set(kernels) - {"prescan_pack", expect} <= extra, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert native_loaded()


def test_rows_kc_all_ones_input():
    x = torch.ones(2, 160, 6, 14)
    w = _weights(64, 160, seed=9)
    announce("rows_kc all-ones")
    y, kernels = _run(x.to(DEV), w.to(DEV), None)
    assert "conv_rows_kc" in kernels
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, None, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_rows_kc_value_path_only_where_flagged():
    g = torch.Generator().manual_seed(4)
    x = spikes((3, 160, 28, 28), 0.03, seed=6)
    x[1, :, 10:12] = x[1, :, 10:12] * torch.randn(160, 2, 28, generator=g)
    x[2, 100, 27, 27] = -2.5
    x[0, 0, 0, 0] = 3e-7
    w = _weights(128, 160, seed=10)
    announce("rows_kc value path")
    y, kernels = _run(x.to(DEV), w.to(DEV), None)
    assert "conv_rows_kc" in kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rows_kc_half_activations(dtype):
    x = spikes((4, 160, 14, 14), 0.05, seed=11)
    w = _weights(128, 160, seed=12)
    b = torch.linspace(-0.5, 0.5, 128)
    announce(f"rows_kc {dtype}")
    y, kernels = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV))
    assert "conv_rows_kc" in kernels and y.dtype == dtype
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, b, 1, 1), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"
    y32, _ = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), output_dtype=torch.float32)
    assert y32.dtype == torch.float32
    ok, err, _ = close(y32, oconv.conv2d_ref(x, w, b, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_rows_kc_deterministic_bitwise():
    x = spikes((32, 160, 28, 28), 0.02, seed=13).to(DEV)
    w = _weights(128, 160, seed=14).to(DEV)
    announce("rows_kc determinism")
    y1, _ = _run(x, w, None)
    y2, _ = _run(x, w, None)
    assert torch.equal(y1, y2)
