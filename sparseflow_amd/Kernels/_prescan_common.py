"""Stage-1 prescan metadata on the GPU (drop-in for Kernels/_prescan_common.py).

The reference builds per-tile metadata with a cascade of ~15 PyTorch ops
(group amax -> receptive-field max-pool -> ceil-mode tile max-pool ->
threshold -> bit-pack -> classify; Kernels/_prescan_common.py:32-189).  Here
the same contract is produced by two HIP kernels behind the C ABI:

  sf_prescan_pack   x -> channel-packed spike bitmap (one pass over x)
  sf_prescan_tiles  bitmap -> ag_mask / tile_class (and channel lists)

Outputs are bit-identical to the cascade for NaN-free input.  (With a NaN
in a window the torch max-pool propagates NaN and the group reads inactive;
here the NaN element alone is inactive.)
"""

from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from .. import _lib
from ..Utils.sparse_helpers import TILE_DENSEISH, TILE_SPARSE, TILE_ZERO

__all__ = [
    "build_rf_prescan_metadata",
    "_build_rf_prescan_metadata_impl",
    "prescan_bitmap",
    "block_channel_lists",
]


def _tuple(value, ndim: int) -> Tuple[int, ...]:
    if isinstance(value, int):
        return (int(value),) * ndim
    if len(value) != ndim:
        raise ValueError(f"Expected {ndim} values, got {value}")
    return tuple(int(v) for v in value)


def prescan_bitmap(x_nchw: torch.Tensor, threshold: float):
    """Stage 1a: (bits, flags) for a 4-D NCHW device tensor."""
    return _lib.prescan_pack(x_nchw, threshold)


def _square(name: str, t: Tuple[int, int]) -> int:
    if t[0] != t[1]:
        raise NotImplementedError(f"{name}={t}: only square kernels/strides/paddings are supported")
    return t[0]


def _build_rf_prescan_metadata_impl(
    x_channels_last: torch.Tensor,
    spatial_dims,
    kernel_dims,
    stride,
    padding,
    block_dims,
    group_size_c: int,
    num_groups: int,
    threshold: float,
    return_debug_stats: bool = False,
    tile_class_out: Optional[torch.Tensor] = None,
    ag_mask_out: Optional[torch.Tensor] = None,
):
    """Same arguments and returns as Kernels/_prescan_common.py:231-275:
    (tile_class, ag_mask, debug_stats) for a channels-last [N, H, W, C]
    device tensor.  Only 2-D spatial inputs are implemented."""
    spatial_ndim = len(spatial_dims) if not isinstance(spatial_dims, int) else 1
    if x_channels_last.dim() != spatial_ndim + 2:
        raise ValueError(
            f"Expected channels-last tensor with {spatial_ndim + 2} dims, got {tuple(x_channels_last.shape)}"
        )
    if spatial_ndim != 2:
        raise NotImplementedError("SparseFlow-AMD implements the 2-D prescan only")
    if not x_channels_last.is_cuda:
        raise _lib.SparseFlowLibError("the prescan runs on ROCm device tensors only")

    spatial_dims = _tuple(spatial_dims, 2)
    k = _square("kernel_dims", _tuple(kernel_dims, 2))
    s = _square("stride", _tuple(stride, 2))
    p = _square("padding", _tuple(padding, 2))
    bh, bw = _tuple(block_dims, 2)

    n, h_in, w_in, c = (int(v) for v in x_channels_last.shape)
    gs = int(group_size_c)
    ng = int(num_groups)
    if c > ng * gs:
        raise ValueError(f"C_in={c} exceeds num_groups*group_size_c={ng * gs}")
    h_out = (h_in + 2 * p - k) // s + 1
    w_out = (w_in + 2 * p - k) // s + 1
    if (h_out, w_out) != tuple(spatial_dims):
        raise ValueError(f"Output spatial mismatch: expected {tuple(spatial_dims)}, got {(h_out, w_out)}")

    gh = -(-h_out // bh)
    gw = -(-w_out // bw)
    n_tiles = n * gh * gw
    dev = x_channels_last.device

    x_nchw = x_channels_last.permute(0, 3, 1, 2)
    bits, _flags = _lib.prescan_pack(x_nchw.contiguous(), threshold)
    ag_mask = torch.empty(max(n_tiles, 1), dtype=torch.int32, device=dev)[:n_tiles]
    tile_class = torch.empty(max(n_tiles, 1), dtype=torch.int32, device=dev)[:n_tiles]
    if n_tiles > 0:
        _lib.prescan_tiles(bits, n, c, h_in, w_in, h_out, w_out, k, s, p, bh, bw, gs,
                           ag_mask=ag_mask, tile_class=tile_class)
        real_groups = -(-c // gs)
        if ng > real_groups:
            # Zero-padded groups can never be active, so no tile is all-active.
            tile_class.masked_fill_(tile_class == TILE_DENSEISH, TILE_SPARSE)

    debug_stats: Optional[Dict[str, float]] = None
    if return_debug_stats:
        zero_tiles = int((tile_class == TILE_ZERO).sum().item())
        dense_tiles = int((tile_class == TILE_DENSEISH).sum().item())
        sparse_tiles = int((tile_class == TILE_SPARSE).sum().item())
        from ..Utils.sparse_helpers import popcount_buf

        active_groups = float(popcount_buf(ag_mask, n_tiles).sum().item()) if n_tiles else 0.0
        debug_stats = {
            "stage1_zero_candidate": zero_tiles,
            "stage1_denseish": dense_tiles,
            "stage1_uncertain": sparse_tiles,
            "stage1_avg_active_group_ratio_lower_bound": active_groups / max(float(n_tiles * ng), 1.0),
            "final_zero": zero_tiles,
            "final_sparse": sparse_tiles,
            "final_denseish": dense_tiles,
            "stage2_zero_refine_tiles": 0,
            "stage2_uncertain_tiles": 0,
            "total_tiles": n_tiles,
        }

    if tile_class_out is not None:
        if int(tile_class_out.numel()) < n_tiles:
            raise ValueError(f"tile_class_out is too small: {int(tile_class_out.numel())} < {n_tiles}")
        tile_class_out[:n_tiles].copy_(tile_class)
        tile_class = tile_class_out[:n_tiles]
    if ag_mask_out is not None:
        if int(ag_mask_out.numel()) < n_tiles:
            raise ValueError(f"ag_mask_out is too small: {int(ag_mask_out.numel())} < {n_tiles}")
        ag_mask_out[:n_tiles].copy_(ag_mask)
        ag_mask = ag_mask_out[:n_tiles]
    return tile_class, ag_mask, debug_stats


def build_rf_prescan_metadata(
    x_channels_last: torch.Tensor,
    spatial_dims,
    kernel_dims,
    stride,
    padding,
    block_dims,
    group_size_c: int,
    num_groups: int,
    threshold: float,
    tile_class_out: Optional[torch.Tensor] = None,
    ag_mask_out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(tile_class, ag_mask) on device without host sync
    (Kernels/_prescan_common.py:278-306)."""
    tile_class, ag_mask, _ = _build_rf_prescan_metadata_impl(
        x_channels_last, spatial_dims, kernel_dims, stride, padding, block_dims,
        group_size_c, num_groups, threshold, False, tile_class_out, ag_mask_out,
    )
    return tile_class, ag_mask


def block_channel_lists(
    x_nchw: torch.Tensor,
    kernel_size: int,
    stride: int,
    padding: int,
    block_size: int,
    threshold: float,
    bits: Optional[torch.Tensor] = None,
):
    """Per-(n, tile) active-channel metadata at block_size x block_size output
    tiles, receptive field included, group size 1:

      ch_mask  int32 [n_tiles, cwp]  bitmask of active input channels
      ch_count int32 [n_tiles]       number of active channels
      ch_list  int32 [n_tiles, C]    ascending active channel ids (first
                                     ch_count entries valid, rest -1)
    """
    n, c, h_in, w_in = (int(v) for v in x_nchw.shape)
    h_out = (h_in + 2 * padding - kernel_size) // stride + 1
    w_out = (w_in + 2 * padding - kernel_size) // stride + 1
    if bits is None:
        bits, _ = _lib.prescan_pack(x_nchw.contiguous(), threshold)
    gh = -(-h_out // block_size)
    gw = -(-w_out // block_size)
    n_tiles = n * gh * gw
    cwp = _lib.words_per_pixel(c)
    dev = x_nchw.device
    ch_mask = torch.empty((n_tiles, cwp), dtype=torch.int32, device=dev)
    ch_count = torch.empty((n_tiles,), dtype=torch.int32, device=dev)
    ch_list = torch.full((n_tiles, c), -1, dtype=torch.int32, device=dev)
    if n_tiles > 0:
        _lib.prescan_tiles(bits, n, c, h_in, w_in, h_out, w_out, kernel_size, stride, padding,
                           block_size, block_size, 16, ch_mask=ch_mask, ch_count=ch_count, ch_list=ch_list)
    return ch_mask, ch_count, ch_list
