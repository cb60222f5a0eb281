"""The C-ABI library: loads, exports the header, host utilities (CPU only).

No call here launches a kernel: only host-side functions and argument
validation paths that return before touching the device.
"""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from sparseflow_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "sparseflow.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sf_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    names = header_functions()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), f"{name} declared in sparseflow.h but not exported"
        assert name in _lib.EXPORTS, f"{name} has no ctypes signature in _lib.EXPORTS"
    assert set(_lib.EXPORTS) == set(names)


def test_version_and_empty_error():
    assert _lib.version() == 101
    assert isinstance(_lib.lib().sf_last_error(), bytes)


@pytest.mark.parametrize("thr", [1e-6, 0.0, 5e-7, 1e-3, 0.3, 1.0, 65504.0, 1e-9, -1.0, 2.0 ** -25])
def test_activity_cutoff_matches_fp16_semantics(thr):
    c = _lib.activity_cutoff(thr)
    # Oracle: |v| is active iff fp16(|v|) > fp16(thr).  Check around c.
    probes = np.array([c, np.nextafter(np.float32(c), np.float32(0)), np.nextafter(np.float32(c), np.float32(np.inf)),
                       0.0, 1e-9, 1e-6, 1.0, 7e4], dtype=np.float32)
    with np.errstate(over="ignore"):
        want = np.abs(probes.astype(np.float16)) > np.float16(thr)
    got = np.abs(probes) >= np.float32(c)
    np.testing.assert_array_equal(got, want)


def test_activity_cutoff_special_values():
    assert np.isnan(_lib.activity_cutoff(float("nan")))
    assert np.isnan(_lib.activity_cutoff(float("inf")))
    assert _lib.activity_cutoff(-0.5) == 0.0
    # f16(1e-6) = 17 * 2^-24; the boundary to 18 * 2^-24 ties to even (18).
    assert _lib.activity_cutoff(1e-6) == np.float32(17.5 * 2.0 ** -24)


def test_words_per_pixel_and_sizes():
    assert [_lib.words_per_pixel(c) for c in (1, 3, 32, 33, 64, 65, 96, 128, 256, 512, 2048)] == \
        [1, 1, 1, 2, 2, 4, 4, 4, 8, 16, 64]
    L = _lib.lib()
    assert L.sf_prescan_bitmap_bytes(32, 64, 32, 32) == 32 * 1024 * 2 * 4
    chunk = _lib.chunk_pixels(32, 64, 32, 32)
    assert chunk in (64, 128, 256)
    assert L.sf_prescan_flags_bytes(32, 64, 32, 32) == 32 * (-(-1024 // chunk)) * 4
    d = _lib.conv_desc(32, 64, 32, 32, 64, 32, 32, 3, 1, 1, 0, 0)
    ws = _lib.conv2d_workspace_size(d)
    assert ws >= L.sf_prescan_bitmap_bytes(32, 64, 32, 32) + L.sf_prescan_flags_bytes(32, 64, 32, 32)
    assert ws % 256 == 0
    assert _lib.conv_lif_workspace_size(d, 4) == _lib.conv2d_workspace_size(
        _lib.conv_desc(128, 64, 32, 32, 64, 32, 32, 3, 1, 1, 0, 0))


def _status(fn, *args):
    return int(fn(*args))


def test_validation_rejects_bad_descriptors_without_touching_the_device():
    L = _lib.lib()
    dummy = ctypes.c_void_p(16)
    bad_pattern = _lib.conv_desc(1, 8, 8, 8, 8, 8, 8, 5, 1, 2, 0, 0)
    assert _status(L.sf_conv2d_sparse, ctypes.byref(bad_pattern), dummy, dummy, dummy, dummy, None, dummy, None) \
        == _lib.SF_ERR_UNSUPPORTED
    assert b"supported patterns" in L.sf_last_error()
    wrong_out = _lib.conv_desc(1, 8, 8, 8, 8, 7, 8, 3, 1, 1, 0, 0)
    assert _status(L.sf_conv2d_sparse, ctypes.byref(wrong_out), dummy, dummy, dummy, dummy, None, dummy, None) \
        == _lib.SF_ERR_INVALID
    bad_dtype = _lib.conv_desc(1, 8, 8, 8, 8, 8, 8, 3, 1, 1, 7, 0)
    assert _status(L.sf_conv2d_sparse, ctypes.byref(bad_dtype), dummy, dummy, dummy, dummy, None, dummy, None) \
        == _lib.SF_ERR_INVALID
    mixed = _lib.conv_desc(1, 8, 8, 8, 8, 8, 8, 3, 1, 1, 0, 1)  # f32 in -> f16 out
    assert _status(L.sf_conv2d_sparse, ctypes.byref(mixed), dummy, dummy, dummy, dummy, None, dummy, None) \
        == _lib.SF_ERR_UNSUPPORTED
    too_wide = _lib.conv_desc(1, 4096, 8, 8, 8, 8, 8, 3, 1, 1, 0, 0)
    assert _status(L.sf_conv2d_sparse, ctypes.byref(too_wide), dummy, dummy, dummy, dummy, None, dummy, None) \
        == _lib.SF_ERR_UNSUPPORTED
    ok = _lib.conv_desc(1, 8, 8, 8, 8, 8, 8, 3, 1, 1, 0, 0)
    assert _status(L.sf_conv2d_sparse, ctypes.byref(ok), None, dummy, dummy, dummy, None, dummy, None) \
        == _lib.SF_ERR_INVALID
    assert _status(L.sf_conv2d_forward, ctypes.byref(ok), dummy, dummy, None, 1e-6, dummy, 16, dummy, None) \
        == _lib.SF_ERR_WORKSPACE
    # Fused conv-LIF: stride 2 unsupported, T < 1 invalid.
    s2 = _lib.conv_desc(1, 8, 8, 8, 8, 4, 4, 3, 2, 1, 0, 0)
    lif = _lib.LifParams(2.0, 1.0, 0.0, 1, 1)
    assert _status(L.sf_conv_lif_forward, ctypes.byref(s2), 2, dummy, dummy, None, ctypes.byref(lif), 1e-6, None,
                   dummy, dummy, dummy, 1 << 20, None) == _lib.SF_ERR_UNSUPPORTED
    assert _status(L.sf_conv_lif_forward, ctypes.byref(ok), 0, dummy, dummy, None, ctypes.byref(lif), 1e-6, None,
                   dummy, dummy, dummy, 1 << 20, None) == _lib.SF_ERR_INVALID
    # Tiles: group size must be a power of two >= 16; kernel < stride rejected.
    assert _status(L.sf_prescan_tiles, dummy, 1, 8, 8, 8, 8, 8, 3, 1, 1, 8, 8, 12, None, None, None, dummy, None,
                   None) == _lib.SF_ERR_UNSUPPORTED
    assert _status(L.sf_prescan_tiles, dummy, 1, 8, 8, 8, 4, 4, 1, 2, 0, 8, 8, 16, None, None, None, dummy, None,
                   None) == _lib.SF_ERR_UNSUPPORTED


def test_zero_frames_is_a_noop():
    L = _lib.lib()
    empty = _lib.conv_desc(0, 8, 8, 8, 8, 8, 8, 3, 1, 1, 0, 0)
    assert _status(L.sf_conv2d_sparse, ctypes.byref(empty), None, None, None, None, None, None, None) == _lib.SF_OK
    assert _status(L.sf_prescan_pack, None, 0, 0, 8, 8, 8, 1e-6, None, None, None) == _lib.SF_OK


def test_linear_bmm_attention_sizes_and_validation():
    L = _lib.lib()
    # Row bitmap: ceil(k/32) words, rounded up to a multiple of 4 beyond two.
    assert L.sf_linear_bitmap_bytes(10, 20) == 10 * 1 * 4
    assert L.sf_linear_bitmap_bytes(10, 64) == 10 * 2 * 4
    assert L.sf_linear_bitmap_bytes(10, 65) == 10 * 4 * 4
    assert L.sf_linear_bitmap_bytes(10, 384) == 10 * 12 * 4
    assert L.sf_linear_flags_bytes(33) == 3 * 4
    assert L.sf_linear_workspace_size(0, 10) == 0
    assert L.sf_linear_workspace_size(10, 384) == 512 + 256
    p = ctypes.c_void_p(1)  # never dereferenced: every call below fails validation or has no work
    # c_out not a multiple of 4 -> unsupported; m = 0 -> nothing to do.
    assert L.sf_linear_sparse(p, p, p, 0, 8, 32, p, None, 6, p, 0, None) == _lib.SF_ERR_UNSUPPORTED
    assert L.sf_linear_sparse(p, p, p, 0, 0, 32, p, None, 8, p, 0, None) == _lib.SF_OK
    assert L.sf_linear_forward(p, 0, 8, 32, p, None, 8, 1e-6, p, 1, p, 0, None) == _lib.SF_ERR_WORKSPACE
    # MFMA linear: kp must be k rounded up to 32; k <= 8192.
    assert L.sf_linear_mfma(p, 0, 8, 40, p, p, 40, None, 8, 1e-6, p, 0, None) == _lib.SF_ERR_INVALID
    assert L.sf_linear_mfma(p, 0, 8, 9000, p, p, 9024, None, 8, 1e-6, p, 0, None) == _lib.SF_ERR_UNSUPPORTED
    assert L.sf_linear_mfma(p, 0, 0, 40, p, p, 64, None, 8, 1e-6, p, 0, None) == _lib.SF_OK
    assert L.sf_linear_mfma_bits(p, p, p, 0, 8, 40, p, p, 40, None, 8, 1e-6, p, 0, None) == _lib.SF_ERR_INVALID
    assert L.sf_linear_mfma_bits(p, p, p, 0, 8, 9000, p, p, 9024, None, 8, 1e-6, p, 0, None) == _lib.SF_ERR_UNSUPPORTED
    assert L.sf_linear_mfma_bits(None, p, p, 0, 8, 40, p, p, 64, None, 8, 1e-6, p, 0, None) == _lib.SF_ERR_INVALID
    assert L.sf_linear_mfma_bits(p, p, p, 0, 0, 40, p, p, 64, None, 8, 1e-6, p, 0, None) == _lib.SF_OK
    # The output leaves as 16-byte row pieces: c_out must be a multiple of 4
    # (rejected before any launch).
    for c_out in (1, 130):
        assert L.sf_linear_mfma(p, 0, 8, 40, p, p, 64, None, c_out, 1e-6, p, 0, None) == _lib.SF_ERR_UNSUPPORTED
        assert L.sf_linear_mfma_bits(p, p, p, 0, 8, 40, p, p, 64, None, c_out, 1e-6, p, 0, None) == _lib.SF_ERR_UNSUPPORTED
    # Batched matmul: B's 64-column block of k rows must fit 64 KB of LDS.
    assert L.sf_bmm_supported(252, 10) and not L.sf_bmm_supported(253, 10)
    assert L.sf_bmm_sparse(p, p, 0, 2, 4, 300, 8, 0, 1, 300, 1e-6, 1.0, p, 0, None) == _lib.SF_ERR_UNSUPPORTED
    assert L.sf_bmm_sparse(p, p, 0, 0, 4, 30, 8, 0, 8, 1, 1e-6, 1.0, p, 0, None) == _lib.SF_OK
    assert L.sf_bmm_sparse(p, p, 0, 2, 4, 30, 8, 0, -1, 1, 1e-6, 1.0, p, 0, None) == _lib.SF_ERR_INVALID
    # Fused attention: head_dim 16/32/64 and k, v within LDS.
    assert L.sf_spike_attention_supported(196, 32) and not L.sf_spike_attention_supported(196, 48)
    assert not L.sf_spike_attention_supported(700, 64)
    st = (ctypes.c_int64 * 3)(0, 0, 0)
    assert L.sf_spike_attention(p, p, p, 0, 2, 196, 12, 48, st, 0.2, 1e-6, p, st, 0, None) == _lib.SF_ERR_UNSUPPORTED
    assert L.sf_spike_attention(p, p, p, 0, 0, 196, 12, 32, st, 0.2, 1e-6, p, st, 0, None) == _lib.SF_OK
    assert L.sf_spike_attention(p, p, p, 0, 2, 196, 12, 32, None, 0.2, 1e-6, p, st, 0, None) == _lib.SF_ERR_INVALID


def test_fused_conv1x1_lif_validation_without_touching_the_device():
    L = _lib.lib()
    d = ctypes.c_void_p(16)
    lif = _lib.LifParams(2.0, 1.0, 0.0, 1, 1)
    ok = _lib.conv_desc(2, 64, 8, 8, 64, 8, 8, 1, 1, 0, 0, 0)
    k3 = _lib.conv_desc(2, 64, 8, 8, 64, 8, 8, 3, 1, 1, 0, 0)
    args = (d, d, d, d, None)  # bits, flags, x, wt, bias
    for fn, extra in ((L.sf_conv1x1_lif_sparse, None), (L.sf_conv1x1_lif_sparse_binres, d)):
        # 3x3 is not this entry's pattern; T < 1 and a NULL spikes pointer are invalid.
        assert _status(fn, ctypes.byref(k3), 2, *args, extra, ctypes.byref(lif), None, d, d, None, None, None) \
            == _lib.SF_ERR_UNSUPPORTED
        assert _status(fn, ctypes.byref(ok), 0, *args, extra, ctypes.byref(lif), None, d, d, None, None, None) \
            == _lib.SF_ERR_INVALID
        assert _status(fn, ctypes.byref(ok), 2, *args, extra, ctypes.byref(lif), None, None, d, None, None, None) \
            == _lib.SF_ERR_INVALID
        # out_bits and out_flags go together.
        assert _status(fn, ctypes.byref(ok), 2, *args, extra, ctypes.byref(lif), None, d, d, d, None, None) \
            == _lib.SF_ERR_INVALID
    # The binary-residual entry needs its residual map.
    assert _status(L.sf_conv1x1_lif_sparse_binres, ctypes.byref(ok), 2, *args, None, ctypes.byref(lif), None, d, d,
                   None, None, None) == _lib.SF_ERR_INVALID
    assert b"res_bits" in L.sf_last_error()


def test_noalloc_entry_point_refuses_oversized_bitmaps_on_the_host():
    # Returns SF_ERR_WORKSPACE from the size check, before any device call.
    L = _lib.lib()
    d = _lib.conv_desc(4096, 256, 56, 56, 64, 56, 56, 3, 1, 1, 0, 0)
    assert _lib.conv2d_workspace_size(d) > _lib.NOALLOC_SCRATCH_BYTES
    dummy = ctypes.c_void_p(16)
    rc = L.sf_conv2d_forward_noalloc(ctypes.byref(d), dummy, dummy, None, ctypes.c_float(1e-6), dummy, None)
    assert rc == _lib.SF_ERR_WORKSPACE
    assert b"scratch" in L.sf_last_error()
    # Bad descriptors are refused before the size check, as sf_conv2d_forward does.
    bad = _lib.conv_desc(1, 8, 8, 8, 8, 8, 8, 5, 1, 2, 0, 0)
    assert L.sf_conv2d_forward_noalloc(ctypes.byref(bad), dummy, dummy, None, ctypes.c_float(1e-6), dummy,
                                       None) == _lib.SF_ERR_UNSUPPORTED


def test_bitmap_layout_query_follows_the_stage2_choice():
    P, M = _lib.SF_BITMAP_PLANES, _lib.SF_BITMAP_PIXEL_MAJOR

    def q(n, ci, h, w, co, ho, wo, k, s, p):
        return _lib.conv2d_bitmap_layout(_lib.conv_desc(n, ci, h, w, co, ho, wo, k, s, p, 0, 0))

    # Pixel-tile 3x3 (layer1, layer2, the stride-2 layers) and the K-chunked
    # row kernel (layer3 at 14x14) read word planes.
    assert q(512, 64, 56, 56, 64, 56, 56, 3, 1, 1) == P
    assert q(512, 128, 28, 28, 128, 28, 28, 3, 1, 1) == P
    assert q(512, 256, 14, 14, 256, 14, 14, 3, 1, 1) == P
    assert q(512, 512, 14, 14, 512, 7, 7, 3, 2, 1) == P
    # The row-band kernel (32-wide frames, C_in <= 64), the matrix-core stem
    # and the 1x1 kernels read pixel-major words.
    assert q(32, 64, 32, 32, 64, 32, 32, 3, 1, 1) == M
    assert q(64, 3, 32, 32, 384, 32, 32, 3, 1, 1) == M
    assert q(512, 256, 56, 56, 64, 56, 56, 1, 1, 0) == M
    assert q(0, 64, 56, 56, 64, 56, 56, 3, 1, 1) == P  # no frames: still the shape's choice
    with pytest.raises(_lib.SparseFlowLibError):       # inconsistent output size
        q(4, 64, 56, 56, 64, 9, 9, 3, 1, 1)
    d = _lib.conv_desc(4, 64, 56, 56, 64, 9, 9, 3, 1, 1, 0, 0)
    assert _lib.lib().sf_conv2d_bitmap_layout(ctypes.byref(d)) == -_lib.SF_ERR_INVALID


def test_layout_entry_points_reject_unknown_layouts_before_launching():
    L = _lib.lib()
    d = _lib.conv_desc(2, 64, 8, 8, 64, 8, 8, 3, 1, 1, 0, 0)
    dummy = ctypes.c_void_p(16)
    assert L.sf_conv2d_sparse_layout(ctypes.byref(d), dummy, 7, dummy, dummy, dummy, None, dummy, None) == \
        _lib.SF_ERR_INVALID
    lif = _lib.LifParams(2.0, 1.0, 0.0, 1, 1)
    assert L.sf_lif_multistep_layout(dummy, None, 0, 2, 1, 64, 64, ctypes.byref(lif), None, dummy, 0, dummy, dummy,
                                     dummy, 5, None) == _lib.SF_ERR_INVALID
    d1 = _lib.conv_desc(2, 64, 8, 8, 64, 8, 8, 1, 1, 0, 0, 0)
    assert L.sf_conv1x1_lif_sparse_layout(ctypes.byref(d1), 2, dummy, dummy, dummy, dummy, None, None,
                                          ctypes.byref(lif), None, dummy, dummy, dummy, dummy, -1, None) == \
        _lib.SF_ERR_INVALID


def test_layout_requests_pick_planes_only_when_every_consumer_asks():
    from sparseflow_amd.Kernels.spike_map import PIXEL_MAJOR, PLANES, LayoutRequests

    r = LayoutRequests()
    assert r.layout == PIXEL_MAJOR                    # nobody asked yet
    r.note("conv2", PLANES)
    assert r.layout == PLANES
    r.note("pool", PIXEL_MAJOR)
    assert r.layout == PIXEL_MAJOR                    # one consumer reads pixel-major words
    r.note("pool", PLANES)
    assert r.layout == PLANES
    for i in range(40):                               # bounded: old consumers drop out
        r.note(("c", i), PLANES)
    assert r.layout == PLANES and len(r._wants) == LayoutRequests._MAX
    r.clear()
    assert r.layout == PIXEL_MAJOR
