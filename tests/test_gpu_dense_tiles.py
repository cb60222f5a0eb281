"""Dense-tile branch of the streamed pixel-tile kernel and of the row kernel
(C_in > 128).

Wave-tiles whose first chunk is dense are queued by k_conv_px3s (and the
64-pixel tiles covering a heavy row tile by k_conv_rows_kc) and computed
on the matrix cores (k_conv_dense_mfma: implicit GEMM, spikes exact in bf16,
W split into bf16 hi + lo, f32 accumulation).  Bar: fp32 within 1e-4 abs +
1e-4 rel of float64 F.conv2d, fp16/bf16 outputs within 1e-2; the kernel
pair is deterministic (repeats are bit-identical) and leaves its queue
clear (a following call without dense tiles runs no matrix-core work and is
still exact); inputs whose tiles are all dense, tiles that span frames,
partial channel groups and chunks, value-path (non-binary) tiles, which are
never deferred, and more dense tiles than the queue holds (the rest are
walked) are covered.  Inputs mix bursts of dense frames (a time step where
most neurons fire) with sparse ones, as a live spiking network does.
"""

import pytest
import torch

from oracle import conv as oconv
from sparseflow_amd import _lib
from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward
from tests.gpu_helpers import DEV, announce, close, native_loaded

pytestmark = pytest.mark.gpu

FP32_TOL = dict(atol=1e-4, rtol=1e-4)


def _weights(c_out, c_in, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(c_out, c_in, 3, 3, generator=g) * (2.0 / (c_in * 9)) ** 0.5


def _bursty(shape, dense_frames, p_dense=0.12, p_sparse=0.005, seed=0):
    """Binary spikes: the listed frames at p_dense, the rest at p_sparse."""
    g = torch.Generator().manual_seed(seed)
    n = shape[0]
    p = torch.full((n, 1, 1, 1), p_sparse)
    p[list(dense_frames)] = p_dense
    return (torch.rand(shape, generator=g) < p).float()


def _run(x, w, b, stride, **kw):
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        y = sparse_conv2d_forward(x, w, b, kernel_size=3, stride=stride, padding=1, **kw)[0]
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return y, {k: c for k, (c, _) in stats.items() if c > 0}


CASES = [
    # (N, C_in, H, W, C_out, stride, dense frames)
    (24, 256, 28, 28, 256, 2, range(8, 16)),       # layer3.0 conv2 shape, a burst of 8 frames
    (24, 512, 14, 14, 512, 2, range(16, 24)),      # layer4.0 conv2 (49-pixel planes: tiles span frames)
    (12, 200, 15, 13, 100, 1, (1, 5, 6, 7, 11)),   # partial last chunk, partial last group
    (6, 160, 9, 31, 68, 2, (0, 1, 2, 3, 4, 5)),    # every frame dense
]


@pytest.mark.parametrize("case", CASES)
def test_dense_tiles_match_dense_conv(case):
    N, C, H, W, Co, s, dense = case
    announce(f"dense tiles {case[:6]}")
    x = _bursty((N, C, H, W), dense, seed=C + H)
    w = _weights(Co, C, seed=Co)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(2)) * 0.1
    xd = x.to(DEV)
    y, kernels = _run(xd, w.to(DEV), b.to(DEV), s)
    assert "conv_px3" in kernels and "conv_dense_mfma" in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, s, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"
    y2, _ = _run(xd, w.to(DEV), b.to(DEV), s)
    assert torch.equal(y, y2)  # deterministic, and the queue was clear again
    assert native_loaded()


ROW_CASES = [
    # (N, C_in, H, W, C_out, dense frames): the row kernel's 14- and 28-wide
    # planes (C_in > 128, stride 1); 14 x 14 planes put 64-pixel tiles across
    # frame boundaries.
    (16, 256, 14, 14, 256, range(4, 8)),
    (8, 192, 28, 28, 128, (2, 3, 6)),
]


@pytest.mark.parametrize("case", ROW_CASES)
def test_row_kernel_dense_tiles_match_dense_conv(case):
    # The row kernel queues its heavy tiles' 64-pixel tiles for the matrix
    # cores instead of walking them.
    N, C, H, W, Co, dense = case
    announce(f"row-kernel dense tiles {case[:5]}")
    x = _bursty((N, C, H, W), dense, seed=5 + W)
    w = _weights(Co, C, seed=6)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(3)) * 0.1
    xd = x.to(DEV)
    y, kernels = _run(xd, w.to(DEV), b.to(DEV), 1)
    assert "conv_rows_kc" in kernels and "conv_dense_mfma" in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"
    y2, _ = _run(xd, w.to(DEV), b.to(DEV), 1)
    assert torch.equal(y, y2)  # deterministic, and the queue was clear again


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_row_kernel_dense_tiles_half_precision(dtype):
    # Half-precision spikes and output through the row kernel's runs.
    N, C, H, W, Co = 8, 192, 14, 14, 128
    announce(f"row-kernel dense tiles {dtype}")
    x = _bursty((N, C, H, W), (2, 3), seed=41)
    w = _weights(Co, C, seed=42)
    b = torch.linspace(-0.3, 0.3, Co)
    y, kernels = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), 1)
    assert y.dtype == dtype and "conv_rows_kc" in kernels and "conv_dense_mfma" in kernels, kernels
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, b, 1, 1), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"
    y32, _ = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), 1, output_dtype=torch.float32)
    ok, err, _ = close(y32, oconv.conv2d_ref(x, w, b, 1, 1), **FP32_TOL)
    assert ok, f"f32 output: max abs err {err}"


def test_row_kernel_keeps_tiles_next_to_value_frames():
    # Every frame dense, frame 3 non-binary: the 64-pixel tiles reaching into
    # frame 3 (14 x 14 planes: tiles span frames) must not be deferred, since
    # the matrix-core kernel takes its input as spikes.
    N, C, H, W, Co = 8, 256, 14, 14, 64
    announce("row-kernel dense tiles beside a value frame")
    x = _bursty((N, C, H, W), range(N), seed=21)
    g = torch.Generator().manual_seed(22)
    x[3] = x[3] * torch.randn(C, H, W, generator=g)
    w = _weights(Co, C, seed=23)
    y, kernels = _run(x.to(DEV), w.to(DEV), None, 1)
    assert "conv_rows_kc" in kernels and "conv_dense_mfma" in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_row_kernel_more_dense_tiles_than_the_queue_holds():
    # 1400 dense 14 x 14 frames = 4288 64-pixel tiles in one group: the row
    # kernel queues what fits (4096) and walks the rest.  (Four output
    # channels keep the float64 reference quick.)
    N, C, H, W, Co = 1400, 160, 14, 14, 4
    announce("row-kernel queue overflow")
    x = _bursty((N, C, H, W), range(N), seed=31)
    w = _weights(Co, C, seed=32)
    y, kernels = _run(x.to(DEV), w.to(DEV), None, 1)
    assert "conv_rows_kc" in kernels and "conv_dense_mfma" in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_row_kernel_small_frames_walk_dense_tiles():
    # Frames of 4 x 14 = 56 pixels: a 64-pixel tile would reach past both
    # neighbouring frames, so the branch keeps such tiles on the walk.
    N, C, H, W, Co = 24, 192, 4, 14, 64
    announce("row-kernel dense tiles, frames under 64 pixels")
    x = _bursty((N, C, H, W), range(N), seed=33)
    w = _weights(Co, C, seed=34)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(35)) * 0.1
    y, kernels = _run(x.to(DEV), w.to(DEV), b.to(DEV), 1)
    assert "conv_rows_kc" in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def _run1(x, w, b, **kw):
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


def _weights1(c_out, c_in, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(c_out, c_in, 1, 1, generator=g) * (2.0 / c_in) ** 0.5


FLAT_CASES = [
    # (N, C_in, H, W, C_out, dense frames): the streamed 1x1 walk (C_in > 256)
    (16, 1024, 14, 14, 256, range(4, 8)),   # the live network's layer3.x conv1 shape
    (8, 512, 28, 28, 128, (2, 5)),          # layer2.x conv1
    (6, 600, 9, 11, 100, (1, 2, 3)),        # 19 of 32 words, partial last stage, partial group, 99-pixel planes
]


@pytest.mark.parametrize("case", FLAT_CASES)
def test_flat_dense_tiles_match_dense_conv(case):
    # The 1x1 walk queues its heavy tiles' runs for the matrix cores (the
    # dense kernel's 1x1 form: nine bitmap words per stage).
    N, C, H, W, Co, dense = case
    announce(f"1x1 dense tiles {case[:5]}")
    x = _bursty((N, C, H, W), dense, seed=51 + C)
    w = _weights1(Co, C, seed=52)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(53)) * 0.1
    xd = x.to(DEV)
    y, kernels = _run1(xd, w.to(DEV), b.to(DEV))
    assert "conv_flat" in kernels and "conv_dense_mfma" in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, 1, 0), **FP32_TOL)
    assert ok, f"max abs err {err}"
    y2, _ = _run1(xd, w.to(DEV), b.to(DEV))
    assert torch.equal(y, y2)


def test_flat_dense_tiles_half_precision_and_value_frames():
    N, C, H, W, Co = 8, 768, 14, 14, 128
    announce("1x1 dense tiles f16, a non-binary frame")
    x = _bursty((N, C, H, W), range(N), seed=54)
    g = torch.Generator().manual_seed(55)
    x[5] = x[5] * torch.randn(C, H, W, generator=g)   # multiplied on the walk, never deferred
    w = _weights1(Co, C, seed=56)
    y, kernels = _run1(x.to(DEV), w.to(DEV), None)
    assert "conv_flat" in kernels and "conv_dense_mfma" in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 1, 0), **FP32_TOL)
    assert ok, f"max abs err {err}"
    xh = x.clone()
    xh[5] = (xh[5] != 0).float()                       # all binary again, as f16 spikes
    y16, _ = _run1(xh.to(DEV, torch.float16), w.to(DEV), None)
    assert y16.dtype == torch.float16
    ok, err, _ = close(y16, oconv.conv2d_ref(xh, w, None, 1, 0), atol=1e-2, rtol=1e-2)
    assert ok, f"f16: max abs err {err}"


def test_queue_is_clear_after_a_dense_call():
    N, C, H, W, Co = 16, 256, 28, 28, 128
    announce("dense then sparse")
    w = _weights(Co, C, seed=7).to(DEV)
    xd = _bursty((N, C, H, W), range(N), seed=8)          # all dense
    xs = _bursty((N, C, H, W), (), seed=9)                # all sparse
    yd, kd = _run(xd.to(DEV), w, None, 2)
    ys, ks = _run(xs.to(DEV), w, None, 2)
    assert "conv_dense_mfma" in kd
    ok, err, _ = close(ys, oconv.sparse_conv2d_ref(xs, w.cpu(), None, 2, 1), **FP32_TOL)
    assert ok, f"sparse call after a dense one: max abs err {err}"
    ok, err, _ = close(yd, oconv.sparse_conv2d_ref(xd, w.cpu(), None, 2, 1), **FP32_TOL)
    assert ok, f"dense call: max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dense_tiles_half_precision(dtype):
    N, C, H, W, Co = 8, 192, 14, 14, 128
    announce(f"dense tiles {dtype}")
    x = _bursty((N, C, H, W), (2, 3, 4), seed=10)
    w = _weights(Co, C, seed=11)
    b = torch.linspace(-0.3, 0.3, Co)
    y, kernels = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), 2)
    assert y.dtype == dtype and "conv_dense_mfma" in kernels
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, b, 2, 1), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"
    y32, _ = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), 2, output_dtype=torch.float32)
    ok, err, _ = close(y32, oconv.conv2d_ref(x, w, b, 2, 1), **FP32_TOL)
    assert ok, f"f32 output: max abs err {err}"


def test_value_path_tiles_are_walked_not_deferred():
    N, C, H, W, Co = 8, 256, 14, 14, 64
    announce("dense value tiles")
    x = _bursty((N, C, H, W), range(N), seed=12)
    g = torch.Generator().manual_seed(13)
    x[3] = x[3] * torch.randn(C, H, W, generator=g)   # a non-binary frame: multiplied, never deferred
    w = _weights(Co, C, seed=14)
    y, kernels = _run(x.to(DEV), w.to(DEV), None, 2)
    assert "conv_dense_mfma" in kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 2, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_more_dense_tiles_than_the_queue_holds():
    # 84 frames of 56 x 56 outputs = 4116 wave-tiles in one group, all dense:
    # 4096 go to the queue, the rest are walked.  (Four output channels keep
    # the float64 reference quick.)
    N, C, H, W, Co = 84, 160, 56, 56, 4
    announce("queue overflow")
    x = _bursty((N, C, H, W), range(N), p_dense=0.06, seed=15)
    w = _weights(Co, C, seed=16)
    y, kernels = _run(x.to(DEV), w.to(DEV), None, 1)
    assert "conv_dense_mfma" in kernels
    ref = oconv.sparse_conv2d_ref(x, w, None, 1, 1)
    ok, err, _ = close(y, ref, **FP32_TOL)
    assert ok, f"max abs err {err}"
