"""Stage-1 prescan on the GPU vs the oracle: bit-exact.

Covers the bitmap (pack), the non-binary flags, reference-geometry
ag_mask / tile_class (drop-in build_rf_prescan_metadata) and the per-tile
active-channel lists at block geometry.
"""

import numpy as np
import pytest
import torch

from oracle import prescan as op
from sparseflow_amd import _lib
from sparseflow_amd.Kernels import _prescan_common as pc
from tests.gpu_helpers import DEV, announce, bits_numpy, clustered_spikes, native_loaded, spikes

pytestmark = pytest.mark.gpu

PACK_SHAPES = [
    (32, 64, 32, 32),   # BASELINE config 1 (frames = T*N)
    (2, 3, 7, 9),       # odd plane, C < 32
    (4, 70, 5, 6),      # C not a multiple of 32, 3 words -> padded to 4
    (2, 33, 14, 14),
    (3, 512, 7, 7),     # 49-pixel plane (scalar lanes)
    (1, 1, 1, 1),
    (2, 2048, 3, 4),    # widest supported C
    (64, 128, 28, 28),  # config 4 frame shape
]


@pytest.mark.parametrize("shape", PACK_SHAPES)
@pytest.mark.parametrize("density", [0.0, 0.02, 0.5, 1.0])
def test_pack_bitmap_matches_oracle(shape, density):
    announce(f"pack {shape} p={density}")
    x = spikes(shape, density, seed=hash((shape, density)) % 1000)
    bits, flags = _lib.prescan_pack(x.to(DEV), 1e-6)
    torch.cuda.synchronize()
    n, c, h, w = shape
    got = bits_numpy(bits, n, h * w, _lib.words_per_pixel(c))
    np.testing.assert_array_equal(got, op.bitmap(x.numpy(), 1e-6))
    assert native_loaded()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_pack_half_inputs(dtype):
    shape = (8, 96, 12, 12)
    announce(f"pack {dtype}")
    x = spikes(shape, 0.1, seed=3) * torch.randn(shape, generator=torch.Generator().manual_seed(4))
    x[0, 0, 0, :4] = torch.tensor([1e-7, 1.04e-6, 1.05e-6, -3e-6])
    xd = x.to(dtype)
    bits, _ = _lib.prescan_pack(xd.to(DEV), 1e-6)
    torch.cuda.synchronize()
    got = bits_numpy(bits, 8, 144, 4)
    np.testing.assert_array_equal(got, op.bitmap(xd.float().numpy(), 1e-6))


def test_pack_unaligned_pointer_and_threshold_boundary():
    shape = (4, 40, 8, 8)
    n = int(np.prod(shape))
    base = torch.zeros(n + 1)
    vals = torch.tensor([0.0, 1.0, 1.0133e-6, 1.0431e-6, 1.0432e-6, -1.0432e-6, 7e4, float("nan")])
    idx = torch.randint(0, len(vals), (n,), generator=torch.Generator().manual_seed(9))
    base[1:] = vals[idx]
    xd = base.to(DEV)[1:].view(shape)  # 4-byte offset: scalar-load path
    announce("pack unaligned")
    bits, _ = _lib.prescan_pack(xd, 1e-6)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_numpy(bits, 4, 64, 2), op.bitmap(base[1:].view(shape).numpy(), 1e-6))


@pytest.mark.parametrize("shape", [(6, 64, 32, 32), (3, 5, 7, 7), (2, 256, 56, 56)])
def test_pack_nonbinary_flags(shape):
    n, c, h, w = shape
    x = spikes(shape, 0.05, seed=5)
    announce(f"flags {shape}")
    _, flags = _lib.prescan_pack(x.to(DEV), 1e-6)
    chunk = _lib.chunk_pixels(n, c, h, w)
    cpf = -(-(h * w) // chunk)
    f = flags[: n * cpf].cpu().numpy().reshape(n, cpf)
    assert not f.any()
    frame, ci, hh, ww = n - 1, c // 2, h - 1, w // 3
    x[frame, ci, hh, ww] = 0.5
    _, flags = _lib.prescan_pack(x.to(DEV), 1e-6)
    f = flags[: n * cpf].cpu().numpy().reshape(n, cpf)
    expect = np.zeros((n, cpf), bool)
    expect[frame, (hh * w + ww) // chunk] = True
    np.testing.assert_array_equal(f.astype(bool), expect)


TILE_CASES = [
    # (shape, k, s, p)
    ((8, 64, 32, 32), 3, 1, 1),
    ((4, 128, 28, 28), 3, 1, 1),
    ((2, 64, 56, 56), 3, 1, 1),    # 8x16 reference tiles
    ((2, 128, 56, 56), 3, 2, 1),   # stride 2
    ((3, 256, 14, 14), 3, 2, 1),
    ((2, 256, 56, 56), 1, 1, 0),   # 1x1
    ((5, 48, 13, 11), 3, 1, 1),    # ragged tiles, 3 groups of 16
    ((2, 512, 9, 9), 3, 1, 1),
]


@pytest.mark.parametrize("shape,k,s,p", TILE_CASES)
@pytest.mark.parametrize("density", [0.0, 0.005, 0.05])
def test_tiles_reference_geometry(shape, k, s, p, density):
    announce(f"tiles {shape} k{k}s{s} p={density}")
    x = spikes(shape, density, seed=11)
    n, c, h, w = shape
    ag_ref, tc_ref, (bh, bw, gs, ng) = op.prescan_reference_geometry(x.numpy(), k, s, p)
    xd = x.to(DEV)
    tile_class, ag_mask, stats = pc._build_rf_prescan_metadata_impl(
        xd.half().permute(0, 2, 3, 1), op.out_hw(h, w, k, s, p), (k, k), s, p, (bh, bw), gs, ng, 1e-6,
        return_debug_stats=True)
    np.testing.assert_array_equal(ag_mask.cpu().numpy(), ag_ref)
    np.testing.assert_array_equal(tile_class.cpu().numpy(), tc_ref)
    assert stats["total_tiles"] == len(ag_ref)
    assert stats["final_zero"] == int((tc_ref == 0).sum())


def test_tiles_clustered_and_bit31():
    x = clustered_spikes((4, 256, 56, 56), seed=2)
    announce("tiles clustered")
    ag_ref, tc_ref, (bh, bw, gs, ng) = op.prescan_reference_geometry(x.numpy(), 1, 1, 0)
    tc, ag = pc.build_rf_prescan_metadata(x.to(DEV).permute(0, 2, 3, 1), (56, 56), 1, 1, 0, (bh, bw), gs, ng, 1e-6)
    np.testing.assert_array_equal(ag.cpu().numpy(), ag_ref)
    np.testing.assert_array_equal(tc.cpu().numpy(), tc_ref)
    # Clustered input: most tiles have some, but not all, channel groups live.
    assert (tc_ref == 1).mean() > 0.5
    # 32 groups of 16 channels: the top group lands in bit 31 (negative int32).
    x = torch.zeros(2, 512, 8, 8)
    x[1, 511, 2, 2] = 1.0
    tc, ag = pc.build_rf_prescan_metadata(x.to(DEV).permute(0, 2, 3, 1), (8, 8), 3, 1, 1, (8, 8), 16, 32, 1e-6)
    assert ag.cpu().tolist() == [0, -(1 << 31)]
    assert tc.cpu().tolist() == [0, 1]


def test_tiles_output_buffers_and_extra_groups():
    x = spikes((2, 40, 16, 16), 1.0, seed=1)
    out_tc = torch.full((64,), -7, dtype=torch.int32, device=DEV)
    out_ag = torch.full((64,), -7, dtype=torch.int32, device=DEV)
    announce("tiles out buffers")
    tc, ag = pc.build_rf_prescan_metadata(x.to(DEV).permute(0, 2, 3, 1), (16, 16), 3, 1, 1, (8, 8), 16, 4, 1e-6,
                                          tile_class_out=out_tc, ag_mask_out=out_ag)
    # 40 channels -> 3 real groups of 16; num_groups=4 adds an empty group, so no
    # tile can be all-active (reference pads C with zeros).
    ag_ref, tc_ref, _ = op.prescan_2d(x.numpy(), 3, 1, 1, 8, 8, 16, 4, 1e-6)
    np.testing.assert_array_equal(out_ag[:8].cpu().numpy(), ag_ref)
    np.testing.assert_array_equal(out_tc[:8].cpu().numpy(), tc_ref)
    assert (out_tc[8:] == -7).all()
    with pytest.raises(ValueError):
        pc.build_rf_prescan_metadata(x.to(DEV).permute(0, 2, 3, 1), (16, 16), 3, 1, 1, (8, 8), 16, 4, 1e-6,
                                     tile_class_out=out_tc[:3])


@pytest.mark.parametrize("shape,k,s,p,block", [
    ((4, 64, 32, 32), 3, 1, 1, 16),
    ((4, 128, 28, 28), 3, 1, 1, 8),
    ((3, 256, 14, 14), 3, 2, 1, 4),
    ((2, 200, 13, 17), 1, 1, 0, 4),
])
@pytest.mark.parametrize("density", [0.0, 0.001, 0.02])
def test_block_channel_lists(shape, k, s, p, block, density):
    announce(f"lists {shape} b{block} p={density}")
    x = spikes(shape, density, seed=21)
    mask, count, lists = pc.block_channel_lists(x.to(DEV), k, s, p, block, 1e-6)
    m_ref, c_ref, l_ref = op.tile_channel_lists(x.numpy(), k, s, p, block, block, 1e-6)
    np.testing.assert_array_equal(mask.cpu().numpy().view(np.uint32), m_ref)
    np.testing.assert_array_equal(count.cpu().numpy(), c_ref)
    got = lists.cpu().numpy()
    for t, ref in enumerate(l_ref):
        assert got[t, : len(ref)].tolist() == ref.tolist()
        assert (got[t, len(ref):] == -1).all()


def test_golden_prescan_fixture():
    from tests.golden import load_golden

    g = load_golden("prescan_golden.npz")
    for i in range(int(g["count"])):
        x = torch.from_numpy(g[f"x{i}"])
        k, s, p, bh, bw, gs, ng = (int(v) for v in g[f"geom{i}"])
        n, c, h, w = x.shape
        announce(f"golden prescan case {i} {tuple(x.shape)}")
        tc, ag = pc.build_rf_prescan_metadata(x.to(DEV).permute(0, 2, 3, 1), op.out_hw(h, w, k, s, p), k, s, p,
                                              (bh, bw), gs, ng, 1e-6)
        np.testing.assert_array_equal(ag.cpu().numpy(), g[f"ag{i}"])
        np.testing.assert_array_equal(tc.cpu().numpy(), g[f"tc{i}"])
        bits, _ = _lib.prescan_pack(x.to(DEV), 1e-6)
        np.testing.assert_array_equal(bits_numpy(bits, n, h * w, _lib.words_per_pixel(c)), g[f"bits{i}"])


def test_nan_masks_only_its_own_element():
    # Documented divergence from the reference: its metadata cascade takes a
    # max-pool over each channel group's window, which propagates a NaN and
    # reads the whole group as inactive (Kernels/_prescan_common.py:32-45,
    # 167-188).  Here the bit of each element is |x| >= cutoff, false for a
    # NaN, so the NaN element alone is inactive: the other channels of its
    # pixel and of its group, and its channel at other pixels, keep their
    # bits; the NaN marks its pixel chunk non-binary; the tile metadata keeps
    # the group live; and the convolution gives the output of the input with
    # that element zeroed.
    from oracle import conv as oconv

    n, c, h, w = 2, 64, 8, 8
    x = torch.zeros(n, c, h, w)
    x[1, 0:16, 3, 4] = 1.0          # the NaN's whole 16-channel group, same pixel
    x[1, 5, 3, 5] = 1.0             # the NaN's channel at the next pixel
    x[1, 5, 3, 4] = float("nan")
    announce("pack NaN element")
    xd = x.to(DEV)
    bits, flags = _lib.prescan_pack(xd, 1e-6)
    torch.cuda.synchronize()
    got = bits_numpy(bits, n, h * w, 2)
    p = 3 * w + 4
    assert got[1, p, 0] == 0xFFFF & ~(1 << 5)      # channels 0-15 but 5
    assert got[1, p + 1, 0] == 1 << 5
    np.testing.assert_array_equal(got, op.bitmap(x.numpy(), 1e-6))
    chunk = _lib.chunk_pixels(n, c, h, w)
    cpf = -(-(h * w) // chunk)
    f = flags[: n * cpf].cpu().numpy().reshape(n, cpf)
    assert f[1, p // chunk] != 0 and not f[0].any()

    # Tile metadata: the group of channels 0-15 stays live in the NaN's tile.
    tc, ag = pc.build_rf_prescan_metadata(xd.permute(0, 2, 3, 1), (h, w), 3, 1, 1, (8, 8), 16, 4, 1e-6)
    assert ag.cpu().tolist() == [0, 1] and tc.cpu().tolist() == [0, 1]

    # The convolution: the NaN element contributes nothing.
    from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward

    g = torch.Generator().manual_seed(31)
    wgt = torch.randn(16, c, 3, 3, generator=g) * 0.05
    y = sparse_conv2d_forward(xd, wgt.to(DEV), None, kernel_size=3, stride=1, padding=1)[0]
    ref = oconv.conv2d_ref(torch.nan_to_num(x, nan=0.0), wgt, None, 1, 1)
    assert torch.isfinite(y).all()
    assert torch.allclose(y.cpu().double(), ref, atol=1e-5, rtol=1e-5)
