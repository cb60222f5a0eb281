"""Pure-Python loop forms for tiny inputs (test infrastructure only).

Written independently of oracle.prescan's pooling cascade: each tile is
visited, its output pixels enumerated, each pixel's receptive field walked
and each element tested.  Agreement between the two forms pins the
restatement of Kernels/_prescan_common.py:153-189.
"""

from __future__ import annotations

import struct


def f16(v: float) -> float:
    """Round-to-nearest-even to IEEE binary16 and back."""
    return struct.unpack("<e", struct.pack("<e", v))[0] if abs(v) < 65520.0 or v != v else (
        float("inf") if v > 0 else float("-inf"))


def element_active(v: float, threshold: float) -> bool:
    a = f16(abs(v))
    return a == a and a > f16(threshold)


def prescan_tiles(x, k, s, p, th, tw, group_size, threshold):
    """x nested lists [N][C][H][W] -> (ag_mask list[int32], tile_class list)."""
    N, C, H, W = len(x), len(x[0]), len(x[0][0]), len(x[0][0][0])
    Ho = (H + 2 * p - k) // s + 1
    Wo = (W + 2 * p - k) // s + 1
    GH, GW = -(-Ho // th), -(-Wo // tw)
    G = -(-C // group_size)
    ags, classes = [], []
    for n in range(N):
        for gh in range(GH):
            for gw in range(GW):
                mask = 0
                for g in range(G):
                    active = False
                    nan_seen = False
                    for oh in range(gh * th, min(gh * th + th, Ho)):
                        for ow in range(gw * tw, min(gw * tw + tw, Wo)):
                            for kh in range(k):
                                for kw in range(k):
                                    ih, iw = oh * s - p + kh, ow * s - p + kw
                                    if not (0 <= ih < H and 0 <= iw < W):
                                        continue
                                    for c in range(g * group_size, min((g + 1) * group_size, C)):
                                        v = x[n][c][ih][iw]
                                        if v != v:
                                            nan_seen = True
                                        elif element_active(v, threshold):
                                            active = True
                    if active and not nan_seen:
                        mask |= 1 << g
                if mask >= 1 << 31:
                    mask -= 1 << 32
                ags.append(mask)
                full = (1 << G) - 1
                m = mask & 0xFFFFFFFF
                classes.append(0 if m == 0 else (2 if m == full else 1))
    return ags, classes


def conv2d(x, w, b, s, p):
    """Direct convolution, float64, nested lists."""
    N, C, H, W = len(x), len(x[0]), len(x[0][0]), len(x[0][0][0])
    Co, k = len(w), len(w[0][0])
    Ho = (H + 2 * p - k) // s + 1
    Wo = (W + 2 * p - k) // s + 1
    y = [[[[0.0] * Wo for _ in range(Ho)] for _ in range(Co)] for _ in range(N)]
    for n in range(N):
        for co in range(Co):
            for oh in range(Ho):
                for ow in range(Wo):
                    acc = 0.0 if b is None else float(b[co])
                    for ci in range(C):
                        for kh in range(k):
                            for kw in range(k):
                                ih, iw = oh * s - p + kh, ow * s - p + kw
                                if 0 <= ih < H and 0 <= iw < W:
                                    acc += float(x[n][ci][ih][iw]) * float(w[co][ci][kh][kw])
                    y[n][co][oh][ow] = acc
    return y
