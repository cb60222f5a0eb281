"""Spike maps as word planes ([frame][word][pixel]) next to the prescan's
pixel-major words ([frame][pixel][word]).

Bar: a conv over a handed map in either layout equals the conv that
prescans x itself, bit for bit (same kernels, same words), and both lie
within 1e-4 of float64 F.conv2d; a neuron layer's planar map is the
transpose of its pixel-major map, which equals the oracle bitmap of its
spikes; a LIFNode -> SparseConv2d pair switches to planes after the first
forward (the conv notes the layout its kernel reads) without changing a
bit of the output.  Shapes whose Stage-2 kernel reads pixel-major words
refuse planes (UnsupportedError), and the module then falls back to the
prescan path.
"""

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import prescan as opre
from sparseflow_amd import _lib
from sparseflow_amd.Kernels import spike_map
from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward
from sparseflow_amd.Kernels.fused_conv_lif import sparse_conv1x1_lif_multistep
from sparseflow_amd.neuron import LIFNode
from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d
from tests.gpu_helpers import DEV, announce, bits_numpy, close, native_loaded, spikes

pytestmark = pytest.mark.gpu

FP32_TOL = dict(atol=1e-4, rtol=1e-4)
PM, PL = _lib.SF_BITMAP_PIXEL_MAJOR, _lib.SF_BITMAP_PLANES


def _weights(c_out, c_in, k=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(c_out, c_in, k, k, generator=g) * (2.0 / (c_in * k * k)) ** 0.5


def _planes(bits, n, hw, cwp):
    """Pixel-major words -> word planes (a transpose of each frame)."""
    return bits[: n * hw * cwp].view(n, hw, cwp).permute(0, 2, 1).contiguous().view(-1)


def _kernels(fn):
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        out = fn()
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return out, {k for k, (c, _) in stats.items() if c > 0}


CASES = [
    # (N, C_in, H, W, C_out, stride, Stage-2 kernel)
    (6, 64, 56, 56, 64, 1, "conv_px3"),        # layer1 conv2 (resident, 64-channel walk)
    (6, 128, 28, 28, 128, 1, "conv_px3"),      # layer2 conv2 (32-channel slices, two super-chunks)
    (3, 128, 56, 56, 128, 2, "conv_px3"),      # layer2.0 conv2, stride 2
    (8, 256, 14, 14, 256, 1, "conv_rows_kc"),  # layer3 conv2 (K-chunked row kernel)
    (5, 256, 28, 28, 256, 2, "conv_px3"),      # layer3.0 conv2 (streamed chunks, flattened tiles)
    (9, 512, 14, 14, 512, 2, "conv_px3"),      # layer4.0 conv2
    (4, 96, 13, 11, 36, 1, "conv_px3"),        # three words padded to four, ragged everything
    (3, 300, 9, 7, 68, 2, "conv_px3"),         # last chunk partial
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("value", [False, True])
def test_conv_over_word_planes_equals_prescan_path(case, value):
    N, C, H, W, Co, s, kern = case
    announce(f"planes conv {case} value={value}")
    x = spikes((N, C, H, W), 0.01, seed=C + H + s)
    if value:  # a non-binary stretch: those chunks read x and multiply
        x[N - 1, :, H // 2] *= torch.linspace(-2.0, 2.0, W)
    w = _weights(Co, C, seed=Co)
    b = torch.randn(Co, generator=torch.Generator().manual_seed(1)) * 0.1
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    desc = _lib.conv_desc(N, C, H, W, Co, (H - 1) // s + 1, (W - 1) // s + 1, 3, s, 1, 0, 0)
    assert _lib.conv2d_bitmap_layout(desc) == PL
    wt = _lib.tap_major_weight(wd)
    bits, flags = _lib.prescan_pack(xd, 1e-6)
    cwp = _lib.words_per_pixel(C)
    pl = _planes(bits, N, H * W, cwp)
    y_pm = torch.empty((N, Co, desc.h_out, desc.w_out), device=DEV)
    y_pl = torch.empty_like(y_pm)
    _, k1 = _kernels(lambda: _lib.conv2d_sparse(desc, bits, flags, xd, wt, bd, y_pm))
    _, k2 = _kernels(lambda: _lib.conv2d_sparse(desc, pl, flags, xd, wt, bd, y_pl, layout=PL))
    y_fw, k3 = _kernels(lambda: sparse_conv2d_forward(xd, wd, bd, kernel_size=3, stride=s, padding=1)[0])
    assert kern in k1 and kern in k2 and kern in k3, (k1, k2, k3)
    assert torch.equal(y_pl, y_pm) and torch.equal(y_fw, y_pm)
    ok, err, _ = close(y_pl, oconv.sparse_conv2d_ref(x, w, b, s, 1), **FP32_TOL)
    assert ok, f"max abs err {err}"
    assert native_loaded()


def test_planes_refused_where_stage2_reads_pixel_major_words():
    N, C, H, W, Co = 4, 128, 8, 8, 64
    announce("planes refused on 1x1")
    x = spikes((N, C, H, W), 0.05, seed=3).to(DEV)
    desc = _lib.conv_desc(N, C, H, W, Co, H, W, 1, 1, 0, 0, 0)
    assert _lib.conv2d_bitmap_layout(desc) == PM
    bits, flags = _lib.prescan_pack(x, 1e-6)
    wt = _lib.tap_major_weight(_weights(Co, C, k=1).to(DEV))
    y = torch.empty((N, Co, H, W), device=DEV)
    with pytest.raises(_lib.UnsupportedError):
        _lib.conv2d_sparse(desc, _planes(bits, N, H * W, 4), flags, x, wt, None, y, layout=PL)
    # One word per pixel: the two layouts coincide and every kernel takes them.
    x1 = spikes((N, 32, H, W), 0.05, seed=4).to(DEV)
    d1 = _lib.conv_desc(N, 32, H, W, Co, H, W, 1, 1, 0, 0, 0)
    b1, f1 = _lib.prescan_pack(x1, 1e-6)
    w1 = _lib.tap_major_weight(_weights(Co, 32, k=1).to(DEV))
    ya, yb = torch.empty((N, Co, H, W), device=DEV), torch.empty((N, Co, H, W), device=DEV)
    _lib.conv2d_sparse(d1, b1, f1, x1, w1, None, ya)
    _lib.conv2d_sparse(d1, b1, f1, x1, w1, None, yb, layout=PL)
    assert torch.equal(ya, yb)


@pytest.mark.parametrize("shape", [(4, 3, 128, 14, 14), (2, 2, 96, 7, 9), (3, 2, 64, 28, 28)])
def test_lif_map_as_planes_is_the_transposed_prescan(shape):
    T, N, C, H, W = shape
    announce(f"lif planes {shape}")
    g = torch.Generator().manual_seed(C)
    x = (torch.randn(shape, generator=g) * 1.5).to(DEV)
    lif = _lib.LifParams(2.0, 1.0, 0.0, 1, 1)
    s_pm, v_pm, m_pm = _lib.lif_multistep(x, T, lif, spike_map=True, map_layout=PM)
    s_pl, v_pl, m_pl = _lib.lif_multistep(x, T, lif, spike_map=True, map_layout=PL)
    assert torch.equal(s_pm, s_pl) and torch.equal(v_pm, v_pl)
    cwp = _lib.words_per_pixel(C)
    want = opre.bitmap(s_pm.view(T * N, C, H, W).cpu().numpy(), 1e-6)
    assert np.array_equal(bits_numpy(m_pm[0], T * N, H * W, cwp), want)
    assert torch.equal(m_pl[0][: T * N * H * W * cwp], _planes(m_pm[0], T * N, H * W, cwp))
    assert int(m_pl[1].abs().sum()) == 0


def test_conv1x1_lif_planar_output_map():
    T, N, C, H, W, Co = 3, 2, 256, 14, 14, 128
    announce("conv1x1-lif planar map")
    x = spikes((T, N, C, H, W), 0.05, seed=7).to(DEV)
    w = (_weights(Co, C, k=1, seed=8) * 6.0).to(DEV)
    req = spike_map.LayoutRequests()
    spk_pm, v_pm = sparse_conv1x1_lif_multistep(x, w, None, map_requests=req)
    m_pm = spike_map.lookup(spk_pm.view(T * N, Co, H, W), 1e-6)
    assert m_pm is not None and m_pm[2] == PM
    req.note("next", PL)
    spk_pl, v_pl = sparse_conv1x1_lif_multistep(x, w, None, map_requests=req)
    assert torch.equal(spk_pm, spk_pl) and torch.equal(v_pm, v_pl)
    assert spike_map.lookup(spk_pl.view(T * N, Co, H, W), 1e-6) is None   # planes not accepted
    m_pl = spike_map.lookup(spk_pl.view(T * N, Co, H, W), 1e-6, accept=(PL,))
    assert m_pl is not None and m_pl[2] == PL
    cwp = _lib.words_per_pixel(Co)
    assert torch.equal(m_pl[0][: T * N * H * W * cwp], _planes(m_pm[0], T * N, H * W, cwp))
    assert 0.0 < float(spk_pm.float().mean()) < 1.0


@pytest.mark.parametrize("C, H, s", [(128, 28, 1), (256, 14, 1), (256, 28, 2)])
def test_neuron_to_conv_switches_to_planes_without_changing_a_bit(C, H, s):
    T, N = 4, 2
    announce(f"lif->conv negotiation C={C} H={H} s={s}")
    torch.manual_seed(C + H)
    node = LIFNode(step_mode="m", v_threshold=0.6)
    conv = SparseConv2d.from_dense(torch.nn.Conv2d(C, C, 3, s, 1, bias=True)).to(DEV)
    conv.set_inference_mode(True)
    g = torch.Generator().manual_seed(H)
    cur = (torch.randn(T, N, C, H, H, generator=g) * 0.5).to(DEV)
    outs, layouts = [], []
    with torch.no_grad():
        for _ in range(3):
            node.reset()
            spk = node(cur)
            layouts.append(spike_map.lookup(spk.flatten(0, 1), 1e-6, accept=(PM, PL))[2])
            outs.append(conv(spk))
        ref = sparse_conv2d_forward(spk.flatten(0, 1).clone(), conv.weight, conv.bias, kernel_size=3, stride=s,
                                    padding=1)[0]
    assert layouts == [PM, PL, PL] and node.map_requests.layout == PL
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    assert torch.equal(outs[2].flatten(0, 1), ref)
    assert 0.001 < float(spk.float().mean()) < 0.5
