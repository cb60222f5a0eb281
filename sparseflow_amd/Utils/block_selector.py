"""Feature-map size -> prescan block size.

The reference documents this rule (README.md:37-41, Instructions.md:136-144)
but ships no implementation (its `block_size` is inert,
Ops/sparse_conv2d.py:114-119).  Here it is live: the block is the square
output tile at which Stage 1b reports per-(n, tile) active-channel lists,
and the analyzer skips feature maps the rule rejects.

    H >= 32       -> 16
    16 <= H < 32  -> 8
    8 <= H < 16   -> 4
    H < 8         -> None (not replaced: per-tile gating does not pay off)
"""

from __future__ import annotations

from typing import Optional

MIN_REPLACE_H = 8


def select_block_size(h: int, w: Optional[int] = None) -> Optional[int]:
    """Block size for an input feature map of height h (and width w, when
    given the smaller side decides).  h <= 0 means unknown -> 16."""
    size = int(h)
    if w is not None and int(w) > 0 and size > 0:
        size = min(size, int(w))
    if size <= 0:
        return 16
    if size >= 32:
        return 16
    if size >= 16:
        return 8
    if size >= MIN_REPLACE_H:
        return 4
    return None


def should_replace(h: int, w: Optional[int] = None) -> bool:
    """False when the rule says the layer is too small to replace."""
    if int(h) <= 0:
        return True
    return select_block_size(h, w) is not None
