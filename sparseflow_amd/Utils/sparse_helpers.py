"""Prescan metadata primitives (Utils/sparse_helpers.py of the reference).

Tile classes, channel-group sizing and the bitmask popcount keep the
reference's values and contracts (Utils/sparse_helpers.py:28-76).
"""

from __future__ import annotations

import torch

TILE_ZERO = 0
TILE_SPARSE = 1
TILE_DENSEISH = 2
TILE_UNCERTAIN = 3
TILE_ZERO_CANDIDATE = 4


def choose_group_size(k_dim: int) -> int:
    """Channels per group: 16 up to 128 channels, else 32, doubled until at
    most 32 groups remain (so a group bitmask fits one int32).
    Contract of Utils/sparse_helpers.py:39-53."""
    gs = 16 if k_dim <= 128 else 32
    while -(-k_dim // gs) > 32:
        gs *= 2
    return gs


def popcount_buf(ag_mask_buf: torch.Tensor, count: int) -> torch.Tensor:
    """Set bits per int32 mask of the first `count` entries (int32 result).
    Contract of Utils/sparse_helpers.py:60-76."""
    v = ag_mask_buf[:count].to(torch.int64) & 0xFFFFFFFF
    v = v - ((v >> 1) & 0x55555555)
    v = (v & 0x33333333) + ((v >> 2) & 0x33333333)
    v = (v + (v >> 4)) & 0x0F0F0F0F
    v = (v * 0x01010101) & 0xFFFFFFFF
    return (v >> 24).to(torch.int32)
