"""Pixel-tile Stage 2 for 3x3 convolutions (stride 1 or 2, padding 1, C_out % 4 == 0).

Same bar as the gather kernel: fp32 within 1e-4 abs + 1e-4 rel of float64
F.conv2d on the spike-masked input, fp16/bf16 within 1e-2, bit-identical
repeats.  Every case also checks which Stage-2 kernel produced the result:
weights resident for C_in <= 64, streamed in 32-channel chunks through two
LDS buffers beyond.
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


def _band(C, W, s):
    """Stride-1 layers with C_in <= 64 on 32-wide frames take the row-band
    kernel (x input: prescan fused in), covered by its own tests."""
    return s == 1 and C <= 64 and W == 32


def _expect(C, W, s):
    return "conv_rows_fused" if _band(C, W, s) else "conv_px3"


def _run(x, w, b, stride, **kw):
    """sparse_conv2d_forward with kernel timing on; returns (y, kernels)."""
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
    # (N, C_in, H, W, C_out, stride)
    (4, 64, 56, 56, 64, 1),     # ResNet50 layer1 conv2 shape (resident weights)
    (8, 64, 30, 30, 64, 1),     # config-1-like, width 30
    (4, 128, 27, 27, 128, 1),   # layer2-like (four chunks, streamed)
    (3, 256, 13, 13, 256, 1),   # layer3-like (eight chunks)
    (2, 512, 7, 7, 128, 1),     # layer4 conv2 (16 chunks, 49-pixel planes)
    (2, 128, 56, 56, 128, 2),   # layer2.0 conv2, stride 2
    (2, 256, 28, 28, 64, 2),    # layer3.0 conv2, stride 2
    (2, 512, 14, 14, 64, 2),    # layer4.0 conv2, stride 2
    (2, 64, 15, 13, 8, 2),      # odd input, stride 2
    (2, 4, 5, 7, 4, 1),         # four channels (one nearly empty word)
    (3, 17, 1, 56, 12, 1),      # single row
    (2, 33, 7, 9, 68, 1),       # two words, second nearly empty; ragged second group
    (1, 300, 6, 10, 100, 1),    # last chunk partially filled
    (17, 96, 8, 8, 64, 1),      # one tile per frame, passes past the end
    (2, 48, 3, 100, 20, 1),     # tiles spanning rows
    (2, 72, 9, 11, 40, 1),      # 32-channel slices: second super-chunk of one sparse word, ragged group
    (3, 100, 10, 10, 36, 2),    # 32-channel slices, stride 2, last word partial
    (2, 65, 17, 5, 96, 1),      # one channel past a super-chunk
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("density", [0.0, 0.01, 0.3])
def test_px3_fp32_matches_dense(case, density):
    N, C, H, W, Co, s = case
    announce(f"px3 {case} p={density}")
    x = spikes((N, C, H, W), density, seed=N * 11 + C + s)
    w = _weights(Co, C, seed=C + Co)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(3)) * 0.1
    y, kernels = _run(x.to(DEV), w.to(DEV), b.to(DEV), s)
    assert _expect(C, W, s) in kernels and "conv_gather" not in kernels, kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, b, s, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert native_loaded()


@pytest.mark.parametrize("case", [(200, 128, 28, 28, 128, 1), (256, 96, 56, 56, 128, 2), (160, 64, 56, 56, 64, 1)])
def test_px3_resident_slices_over_passes(case):
    # The resident pixel-tile walk (C_in <= 64: 64-channel slices; 64 < C_in
    # <= 128: 32-channel slices, two 64-channel super-chunks).  Enough tiles for
    # every workgroup to make at least two passes, with non-binary frames
    # (the value path reads x at the walked super-chunk's channels) in the
    # first and in the last tiles.  Frames are independent, so a spread of
    # them is checked against the float64 reference, and every frame against
    # the device's own f32 convolution (a tile left out or taken twice would
    # show there).
    N, C, H, W, Co, s = case
    announce(f"px3 passes {case}")
    x = spikes((N, C, H, W), 0.01, seed=C + N)
    g = torch.Generator().manual_seed(N)
    x[0, :, 3:5] = x[0, :, 3:5] * torch.randn(C, 2, W, generator=g)
    x[N - 1, :, H - 2:] = x[N - 1, :, H - 2:] * torch.randn(C, 2, W, generator=g)
    w = _weights(Co, C, seed=Co + 5)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(9)) * 0.1
    y, kernels = _run(x.to(DEV), w.to(DEV), b.to(DEV), s)
    assert "conv_px3" in kernels, kernels
    Ho, Wo = (H + 2 - 3) // s + 1, (W + 2 - 3) // s + 1
    waves = (-(-Ho * Wo // 64)) * N * (-(-Co // 64))  # wave-tiles of 64 channels: a lower bound
    assert waves > 16 * torch.cuda.get_device_properties(0).multi_processor_count
    frames = [0, 1, N // 3, (2 * N) // 3, N - 2, N - 1]
    ok, err, _ = close(y[frames], oconv.sparse_conv2d_ref(x[frames], w, b, s, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"
    with torch.no_grad():
        yd = torch.nn.functional.conv2d(x.to(DEV), w.to(DEV), b.to(DEV), stride=s, padding=1)
    assert torch.allclose(y, yd, atol=1e-4, rtol=1e-4), float((y - yd).abs().max())
    y2, _ = _run(x.to(DEV), w.to(DEV), b.to(DEV), s)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("stride", [1, 2])
def test_px3_dense_input(stride):
    x = spikes((2, 96, 12, 12), 0.9, seed=21)
    w = _weights(64, 96, seed=22)
    announce(f"px3 dense s{stride}")
    y, kernels = _run(x.to(DEV), w.to(DEV), None, stride)
    assert "conv_px3" in kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, stride, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_px3_all_ones_input():
    x = torch.ones(2, 64, 6, 56)
    w = _weights(64, 64, seed=9)
    announce("px3 all-ones")
    y, kernels = _run(x.to(DEV), w.to(DEV), None, 1)
    assert "conv_px3" in kernels
    ok, err, _ = close(y, oconv.conv2d_ref(x, w, None, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("stride", [1, 2])
def test_px3_value_path_only_where_flagged(stride):
    g = torch.Generator().manual_seed(4)
    x = spikes((3, 96, 32, 32), 0.05, seed=6)
    x[1, :, 10:12] = x[1, :, 10:12] * torch.randn(96, 2, 32, generator=g)
    x[2, 5, 31, 31] = -2.5
    x[0, 0, 0, 0] = 3e-7       # below the activity threshold: dropped
    w = _weights(64, 96, seed=10)
    announce(f"px3 value path s{stride}")
    y, kernels = _run(x.to(DEV), w.to(DEV), None, stride)
    assert "conv_px3" in kernels
    ok, err, _ = close(y, oconv.sparse_conv2d_ref(x, w, None, stride, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_px3_half_activations(dtype):
    x = spikes((4, 128, 13, 13), 0.05, seed=11)
    x[0, :, 3] = x[0, :, 3] * 0.5   # a value-path chunk in reduced precision
    w = _weights(128, 128, seed=12)
    b = torch.linspace(-0.5, 0.5, 128)
    announce(f"px3 {dtype}")
    xr = x.to(dtype).float()
    y, kernels = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), 1)
    assert "conv_px3" in kernels and y.dtype == dtype
    ok, err, _ = close(y, oconv.conv2d_ref(xr, w, b, 1, 1), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"
    y32, _ = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), 1, output_dtype=torch.float32)
    assert y32.dtype == torch.float32
    ok, err, _ = close(y32, oconv.conv2d_ref(xr, w, b, 1, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


def test_px3_deterministic_bitwise():
    x = spikes((16, 64, 56, 56), 0.02, seed=13).to(DEV)
    w = _weights(64, 64, seed=14).to(DEV)
    announce("px3 determinism")
    y1, _ = _run(x, w, None, 1)
    y2, _ = _run(x, w, None, 1)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("stride", [1, 2])
def test_px3_and_gather_agree(stride):
    # C_out = 6 is not a multiple of 4, so the same input goes through the
    # gather kernel; its channels match the pixel kernel's first six.
    x = spikes((4, 80, 12, 20), 0.03, seed=15)
    w = _weights(8, 80, seed=16)
    announce(f"px3 vs gather s{stride}")
    y_px, k1 = _run(x.to(DEV), w.to(DEV), None, stride)
    y_gather, k2 = _run(x.to(DEV), w[:6].contiguous().to(DEV), None, stride)
    assert "conv_px3" in k1 and "conv_gather" in k2
    assert torch.allclose(y_px[:, :6], y_gather, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("case", [
    (4, 256, 14, 14, 64, 2),    # streamed chunks, 8 words per pixel
    (3, 512, 7, 9, 128, 1),     # 16 words per pixel, ragged plane
    (3, 96, 12, 10, 40, 1),     # 32-channel slices, second super-chunk of one word
    (2, 64, 9, 13, 64, 2),      # resident 64-channel walk, two words
    (2, 300, 5, 6, 36, 1),      # last word partial, ragged channel group
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_px3_word_planes_equal_pixel_words(case, dtype):
    # sf_conv2d_forward prescans into word planes for the pixel-tile kernels;
    # sf_prescan_pack + sf_conv2d_sparse hand them the [hw][cwp] words.  Same
    # kernel, same walk order: the outputs agree bit for bit, and with the
    # float64 reference.
    N, C, H, W, Co, s = case
    announce(f"px3 word planes {case} {dtype}")
    x = spikes((N, C, H, W), 0.05, seed=N + C + Co).to(dtype)
    x[0, :, 1, 1:3] = x[0, :, 1, 1:3] * 0.5  # one non-binary tile: the value path
    w = _weights(Co, C, seed=C * 3 + Co)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(8)) * 0.1
    xd, wt, bd = x.to(DEV), _lib.tap_major_weight(w.to(DEV)), b.to(DEV)
    Ho, Wo = (H + 2 - 3) // s + 1, (W + 2 - 3) // s + 1
    code = _lib.dtype_code(dtype)
    desc = _lib.conv_desc(N, C, H, W, Co, Ho, Wo, 3, s, 1, code, _lib.dtype_code(torch.float32))
    ws = torch.empty(max(_lib.conv2d_workspace_size(desc), 1), dtype=torch.uint8, device=DEV)
    y_planes = torch.empty((N, Co, Ho, Wo), dtype=torch.float32, device=DEV)
    _lib.conv2d_forward(desc, xd, wt, bd, 0.0, ws, y_planes)
    bits, flags = _lib.prescan_pack(xd, 0.0)
    y_words = torch.empty_like(y_planes)
    _lib.conv2d_sparse(desc, bits, flags, xd, wt, bd, y_words)
    torch.cuda.synchronize()
    assert torch.equal(y_planes, y_words)
    ok, err, _ = close(y_planes, oconv.sparse_conv2d_ref(x.float(), w, b, s, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", [(3, 256, 9, 9, 64, 2), (5, 160, 7, 7, 100, 1)])
def test_px3_streamed_half_output(case, dtype):
    # C_in > 128: streamed chunks over tiles of the flattened (frame, pixel)
    # axis (a tile spans up to three 25- or 49-pixel planes), half output.
    N, C, H, W, Co, s = case
    x = spikes((N, C, H, W), 0.05, seed=C + N)
    x[1, :, 2] = x[1, :, 2] * 0.75  # a non-binary row inside a frame-spanning tile
    w = _weights(Co, C, seed=C + 1)
    b = torch.linspace(-0.3, 0.3, Co)
    announce(f"px3 streamed {case} {dtype}")
    xr = x.to(dtype).float()
    y, kernels = _run(x.to(DEV, dtype), w.to(DEV), b.to(DEV), s)
    assert "conv_px3" in kernels and y.dtype == dtype
    ok, err, _ = close(y, oconv.conv2d_ref(xr, w, b, s, 1), atol=1e-2, rtol=1e-2)
    assert ok, f"max abs err {err}"


def _random_cases(n, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(n):
        c_in = int(torch.randint(1, 600, (1,), generator=g))
        c_out = 4 * int(torch.randint(1, 50, (1,), generator=g))
        h = int(torch.randint(1, 24, (1,), generator=g))
        w = int(torch.randint(1, 40, (1,), generator=g))
        frames = int(torch.randint(1, 9, (1,), generator=g))
        s = 1 + int(torch.randint(0, 2, (1,), generator=g))
        dens = [0.003, 0.03, 0.2][int(torch.randint(0, 3, (1,), generator=g))]
        out.append((frames, c_in, h, w, c_out, s, dens))
    return out


@pytest.mark.parametrize("case", _random_cases(40, 2026))
def test_px3_random_shapes(case):
    # Random geometry across every pixel-tile variant (resident 64- and
    # 32-channel slices, streamed chunks over flattened tiles, ragged words,
    # planes smaller than a tile): the forward (word planes) against the
    # float64 reference, and bit for bit against the two-stage path with the
    # [hw][cwp] words.
    N, C, H, W, Co, s, dens = case
    announce(f"px3 random {case}")
    x = spikes((N, C, H, W), dens, seed=C * 7 + H)
    w = _weights(Co, C, seed=Co + W)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(C)) * 0.1
    xd, wt, bd = x.to(DEV), _lib.tap_major_weight(w.to(DEV)), b.to(DEV)
    Ho, Wo = (H + 2 - 3) // s + 1, (W + 2 - 3) // s + 1
    desc = _lib.conv_desc(N, C, H, W, Co, Ho, Wo, 3, s, 1, _lib.dtype_code(torch.float32),
                          _lib.dtype_code(torch.float32))
    ws = torch.empty(max(_lib.conv2d_workspace_size(desc), 1), dtype=torch.uint8, device=DEV)
    y1 = torch.empty((N, Co, Ho, Wo), dtype=torch.float32, device=DEV)
    _lib.conv2d_forward(desc, xd, wt, bd, 0.0, ws, y1)
    bits, flags = _lib.prescan_pack(xd, 0.0)
    y2 = torch.empty_like(y1)
    _lib.conv2d_sparse(desc, bits, flags, xd, wt, bd, y2)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    ok, err, _ = close(y1, oconv.sparse_conv2d_ref(x, w, b, s, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"
