"""Numpy restatement of the Stage-1 prescan (test infrastructure only).

Reference algorithm (Kernels/_prescan_common.py, 2-D path):
  xh      = fp16(x)                                   Kernels/conv2d.py:986
  gmax    = max over each channel group of |xh|       :32-45 (zero-padded C)
  rf      = max_pool2d(gmax, k, s, p)  (-inf padding)  :169-177 (skipped for 1x1 s1 p0, :112-113)
  tmax    = max_pool2d(rf, (BH,BW), (BH,BW), ceil)    :182-187
  act     = tmax > thr   (fp16 tensor vs Python float: compared in fp16)  :188
  ag_mask = sum_g act_g << g  (int32)                 :48-54
  class   = 0 none / 2 all groups / else 1            :57-70
Tile index (n*GH + gh)*GW + gw                        Kernels/conv2d.py:585-586

This build's own Stage-1 formats are restated alongside:
  bitmap  bits[n, p, w] bit (c & 31) of word (c >> 5) = fp16|x[n,c,p]| > fp16(thr),
          words per pixel = next power of two of ceil(C/32)
  lists   per output tile (group size 1): channel mask, count, ascending ids
"""

from __future__ import annotations

import numpy as np
from numpy.lib.stride_tricks import sliding_window_view


def choose_group_size(c: int) -> int:
    """Utils/sparse_helpers.py:39-53."""
    gs = 16 if c <= 128 else 32
    while -(-c // gs) > 32:
        gs *= 2
    return gs


def select_tile_sizes(h: int, w: int):
    """Kernels/conv2d.py:80-84."""
    return (8, 16) if h * w >= 3136 else (8, 8)


def select_block_size(h: int):
    """README.md:37-41 block rule (H>=32:16, >=16:8, >=8:4, else None)."""
    if h >= 32:
        return 16
    if h >= 16:
        return 8
    if h >= 8:
        return 4
    return None


def words_per_pixel(c: int) -> int:
    w = -(-c // 32)
    p = 1
    while p < w:
        p <<= 1
    return p


def out_hw(h, w, k, s, p):
    return (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1


def active_elements(x: np.ndarray, threshold: float) -> np.ndarray:
    """Elementwise fp16(|x|) > fp16(threshold) (overflow to inf is intended)."""
    with np.errstate(over="ignore"):
        return np.abs(x.astype(np.float16)) > np.float16(threshold)


def _max_pool(a: np.ndarray, kh, kw, sh, sw, ph, pw, ceil_mode=False) -> np.ndarray:
    """max_pool2d over the last two axes with -inf padding; NaN propagates
    (any NaN in a window gives NaN), as torch's max_pool2d does."""
    *lead, H, W = a.shape
    def osize(L, k, s, p):
        if ceil_mode:
            o = -(-(L + 2 * p - k) // s) + 1
            if (o - 1) * s >= L + p:
                o -= 1
            return o
        return (L + 2 * p - k) // s + 1
    Ho, Wo = osize(H, kh, sh, ph), osize(W, kw, sw, pw)
    need_h = (Ho - 1) * sh + kh
    need_w = (Wo - 1) * sw + kw
    pad_h_hi = max(0, need_h - H - ph)
    pad_w_hi = max(0, need_w - W - pw)
    af = a.astype(np.float32)
    padded = np.pad(af, [(0, 0)] * len(lead) + [(ph, pad_h_hi), (pw, pad_w_hi)], constant_values=-np.inf)
    win = sliding_window_view(padded, (kh, kw), axis=(-2, -1))
    win = win[..., ::sh, ::sw, :, :][..., :Ho, :Wo, :, :]
    return win.max(axis=(-2, -1))  # np.max propagates NaN


def prescan_2d(x: np.ndarray, k: int, s: int, p: int, bh: int, bw: int, group_size: int,
               num_groups: int, threshold: float):
    """(ag_mask int32 [N*GH*GW], tile_class int32 [N*GH*GW], act bool
    [N, GH, GW, G]) for NCHW x."""
    N, C, H, W = x.shape
    cpad = num_groups * group_size
    if C > cpad:
        raise ValueError("C exceeds num_groups * group_size")
    with np.errstate(over="ignore"):
        ax = np.abs(x.astype(np.float16))
    if cpad > C:
        ax = np.concatenate([ax, np.zeros((N, cpad - C, H, W), np.float16)], axis=1)
    gmax = ax.reshape(N, num_groups, group_size, H, W).max(axis=2)  # [N, G, H, W]
    if (k, s, p) == (1, 1, 0):
        rf = gmax.astype(np.float32)
    else:
        rf = _max_pool(gmax, k, k, s, s, p, p)
    Ho, Wo = out_hw(H, W, k, s, p)
    assert rf.shape[-2:] == (Ho, Wo)
    tmax = _max_pool(rf, bh, bw, bh, bw, 0, 0, ceil_mode=True)  # [N, G, GH, GW]
    act = tmax.astype(np.float16) > np.float16(threshold)
    act = np.moveaxis(act, 1, -1)  # [N, GH, GW, G]
    weights = (np.uint64(1) << np.arange(num_groups, dtype=np.uint64))
    ag = (act.astype(np.uint64) * weights).sum(axis=-1).astype(np.uint64)
    ag = (ag & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.int32).reshape(-1)
    any_a = act.any(axis=-1).reshape(-1)
    all_a = act.all(axis=-1).reshape(-1)
    tile_class = np.where(all_a, 2, np.where(any_a, 1, 0)).astype(np.int32)
    return ag, tile_class, act


def prescan_reference_geometry(x: np.ndarray, k: int, s: int, p: int, threshold: float = 1e-6):
    """ag_mask / tile_class at the reference's own tile and group sizing."""
    N, C, H, W = x.shape
    Ho, Wo = out_hw(H, W, k, s, p)
    bh, bw = select_tile_sizes(Ho, Wo)
    gs = choose_group_size(C)
    ng = -(-C // gs)
    ag, tc, _ = prescan_2d(x, k, s, p, bh, bw, gs, ng, threshold)
    return ag, tc, (bh, bw, gs, ng)


def bitmap(x: np.ndarray, threshold: float) -> np.ndarray:
    """bits uint32 [N, H*W, cwp] in this build's channel-packed layout."""
    N, C, H, W = x.shape
    cwp = words_per_pixel(C)
    act = active_elements(x, threshold).reshape(N, C, H * W)
    padded = np.zeros((N, cwp * 32, H * W), dtype=np.uint64)
    padded[:, :C] = act
    shifts = np.arange(32, dtype=np.uint64)
    words = (padded.reshape(N, cwp, 32, H * W) << shifts[None, None, :, None]).sum(axis=2)
    return np.ascontiguousarray(np.moveaxis(words.astype(np.uint32), 1, -1))  # [N, HW, cwp]


def tile_channel_lists(x: np.ndarray, k: int, s: int, p: int, th: int, tw: int, threshold: float):
    """Per output tile at th x tw, group size 1: (mask uint32 [T, cwp],
    count int32 [T], lists: list of ascending int arrays)."""
    N, C, H, W = x.shape
    ag, tc, act = prescan_2d(x, k, s, p, th, tw, 1, C, threshold)
    act = act.reshape(-1, C)
    cwp = words_per_pixel(C)
    padded = np.zeros((act.shape[0], cwp * 32), dtype=np.uint64)
    padded[:, :C] = act
    shifts = np.arange(32, dtype=np.uint64)
    mask = (padded.reshape(-1, cwp, 32) << shifts[None, None, :]).sum(axis=-1).astype(np.uint32)
    count = act.sum(axis=-1).astype(np.int32)
    lists = [np.nonzero(row)[0].astype(np.int32) for row in act]
    return mask, count, lists

