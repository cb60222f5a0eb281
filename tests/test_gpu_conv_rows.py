"""Row-band Stage 2 (3x3 stride 1, C_in <= 64, frame width 32), in its two
input forms: from the bitmap (k_pack, then k_conv_band -- the path of a
handed spike map) and from x (k_conv_rows_fused, the prescan fused in --
the path of sf_conv2d_forward).

Same bar as the gather kernel: fp32 within 1e-4 abs + 1e-4 rel of float64
F.conv2d on the spike-masked input, fp16/bf16 within 1e-2, bit-identical
repeats.  Both kernels sum every output in the same order, so they must
agree bit for bit.  Every case also checks which kernels produced the result.
"""

import pytest
import torch

from oracle import conv as oconv
from sparseflow_amd import _lib
from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward
from sparseflow_amd.Utils.config import PRESCAN_ACTIVITY_EPS
from tests.gpu_helpers import DEV, announce, close, native_loaded, spikes

pytestmark = pytest.mark.gpu

FP32_TOL = dict(atol=1e-4, rtol=1e-4)


def _weights(c_out, c_in, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(c_out, c_in, 3, 3, generator=g) * (2.0 / (c_in * 9)) ** 0.5


def _timed(fn):
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        y = fn()
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return y, {k: c for k, (c, _) in stats.items() if c > 0}


def _run(x, w, b, threshold=PRESCAN_ACTIVITY_EPS, **kw):
    """sparse_conv2d_forward (the fused kernel here); returns (y, kernels)."""
    return _timed(lambda: sparse_conv2d_forward(x, w, b, kernel_size=3, stride=1, padding=1,
                                                threshold=threshold, **kw)[0])


def _run_two_stage(x, w, b, out_dtype=None, threshold=PRESCAN_ACTIVITY_EPS):
    """k_pack, then the conv on the bitmap; returns (y, kernels)."""
    N, C, H, W = x.shape
    Co = w.shape[0]
    out_dtype = x.dtype if out_dtype is None else out_dtype

    def go():
        desc = _lib.conv_desc(N, C, H, W, Co, H, W, 3, 1, 1, _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype))
        bits, flags = _lib.prescan_pack(x, threshold)
        y = torch.empty(N, Co, H, W, dtype=out_dtype, device=x.device)
        return _lib.conv2d_sparse(desc, bits, flags, x, _lib.tap_major_weight(w), b, y)
    return _timed(go)


def _both(x, w, b, **kw):
    """Both paths on the same input; they agree bit for bit.  Returns y."""
    y, kernels = _run(x, w, b, **kw)
    assert set(kernels) == {"conv_rows_fused"}, kernels
    y2, k2 = _run_two_stage(x, w, b, out_dtype=kw.get("output_dtype"), threshold=kw.get("threshold", PRESCAN_ACTIVITY_EPS))
    assert set(k2) == {"prescan_pack", "conv_rows"}, k2
    assert y.dtype == y2.dtype and torch.equal(y, y2), (y - y2).abs().max().item()
    return y


CASES = [
    # (N, C_in, H, W, C_out)
    (8, 64, 32, 32, 64),    # BASELINE config 1 shape
    (4, 64, 57, 32, 64),    # tall frames
    (2, 4, 5, 32, 3),       # four input channels (one nearly empty word), few rows
    (3, 17, 1, 32, 10),     # single row: no input row above or below
    (2, 32, 2, 32, 64),     # one 32-bit word per pixel
    (2, 33, 7, 32, 65),     # two words, second nearly empty; C_out one past a group
    (2, 48, 9, 32, 200),    # several output-channel groups, ragged last group
    (1, 64, 32, 32, 128),   # two full groups
    (3, 20, 6, 32, 30),     # C_out % 4 != 0: weights staged through registers
    (70, 64, 30, 32, 64),   # more row blocks than CUs (the kernel loops), last block half full
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("density", [0.0, 0.01, 0.3])
def test_rows_fp32_matches_dense(case, density):
    N, C, H, W, Co = case
    announce(f"rows {case} p={density}")
    x = spikes((N, C, H, W), density, seed=N * 5 + C)
    w = _weights(Co, C, seed=C + Co)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(3)) * 0.1
    y = _both(x.to(DEV), w.to(DEV), b.to(DEV))
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert native_loaded()


@pytest.mark.parametrize("width", [32])
def test_rows_all_ones_input(width):
    # Every tap active: the scalar walk visits all 64 channel bits of every
    # input position.
    x = torch.ones(2, 64, 6, width)
    w = _weights(64, 64, seed=9)
    announce(f"rows all-ones w{width}")
    y = _both(x.to(DEV), w.to(DEV), None)
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, None, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("width", [32])
def test_rows_value_path_only_where_flagged(width):
    # Non-binary values in a few rows of one frame: those tiles take the
    # multiply path, the rest stay on the add path.
    g = torch.Generator().manual_seed(4)
    x = spikes((3, 64, 20, width), 0.05, seed=6)
    x[1, :, 10:12] = x[1, :, 10:12] * torch.randn(64, 2, width, generator=g)
    x[2, 5, 19, width - 1] = -2.5
    x[0, 0, 0, 0] = 3e-7       # below the activity threshold: dropped
    w = _weights(64, 64, seed=10)
    announce(f"rows value path w{width}")
    y = _both(x.to(DEV), w.to(DEV), None)
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rows_half_activations(dtype):
    x = spikes((4, 64, 8, 32), 0.05, seed=11)
    w = _weights(64, 64, seed=12)
    b = torch.linspace(-0.5, 0.5, 64)
    announce(f"rows {dtype}")
    y = _both(x.to(DEV, dtype), w.to(DEV), b.to(DEV))
    assert y.dtype == dtype
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, b, 1, 1), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"
    y32 = _both(x.to(DEV, dtype), w.to(DEV), b.to(DEV), output_dtype=torch.float32)
    assert y32.dtype == torch.float32
    ok, err, _ = close(y32, oconv.conv2d_ref(x, w, b, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_rows_deterministic_bitwise():
    x = spikes((32, 64, 32, 32), 0.02, seed=13).to(DEV)
    w = _weights(64, 64, seed=14).to(DEV)
    announce("rows determinism")
    y1, _ = _run(x, w, None)
    y2, _ = _run(x, w, None)
    assert torch.equal(y1, y2)
    y3, _ = _run_two_stage(x, w, None)
    y4, _ = _run_two_stage(x, w, None)
    assert torch.equal(y3, y4) and torch.equal(y1, y3)


def test_rows_and_pixel_kernel_agree():
    # The row kernel (W=32) and the pixel-tile kernel (same data with one
    # padding column, W=33, which the row kernel does not take) agree on the
    # shared columns to fp32 rounding.
    x = spikes((4, 64, 12, 32), 0.03, seed=15)
    w = _weights(64, 64, seed=16)
    announce("rows vs px3")
    y_rows = _both(x.to(DEV), w.to(DEV), None)
    xp = torch.nn.functional.pad(x, (0, 1))
    y_px, k2 = _run(xp.to(DEV), w.to(DEV), None)
    assert "conv_px3" in k2
    # Column 31 of the padded run sees the zero column 32 as its right
    # neighbour, exactly like the unpadded frame edge.
    assert torch.allclose(y_rows, y_px[..., :32], atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("threshold", [0.0, 0.5, 2.0, float("inf"), float("nan")])
def test_rows_fused_activity_threshold(threshold):
    # The fused kernel applies the prescan's activity rule (f16(|x|) >
    # f16(threshold)) itself: values at or below the cutoff drop out, as with
    # the separate prescan; NaN and +inf thresholds leave nothing active.
    g = torch.Generator().manual_seed(21)
    x = spikes((4, 64, 8, 32), 0.05, seed=22) * torch.randn(4, 64, 8, 32, generator=g) * 2
    w = _weights(64, 64, seed=23)
    announce(f"rows fused threshold {threshold}")
    y = _both(x.to(DEV), w.to(DEV), None, threshold=threshold)
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, 1, 1, threshold=threshold), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_rows_fused_nan_input_only_masks_its_element():
    # A NaN activation is inactive under |x| >= cutoff (the comparison is
    # false) and sends its row block down the value path; every other
    # element, in its channel and elsewhere, still counts.
    x = spikes((2, 64, 8, 32), 0.05, seed=24)
    x[0, 3, 2, 5] = float("nan")
    w = _weights(64, 64, seed=25)
    announce("rows fused NaN input")
    y = _both(x.to(DEV), w.to(DEV), None)
    ref = oconv.conv2d_ref(torch.nan_to_num(x, nan=0.0), w, None, 1, 1)
    ok, err, _ = close(y, ref, **FP32_TOL)
    assert ok, f"max abs err {err}"
