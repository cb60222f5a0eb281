"""Sparse Conv2d entry point on MI355X (drop-in for Kernels/conv2d.py).

`sparse_conv2d_forward` keeps the reference's signature, return tuple and
fallback reasons (Kernels/conv2d.py:893-1178).  Under it, device tensors go
through the C ABI of libsparseflow_hip.so:

  Stage 1  sf_prescan_pack    x -> spike bitmap (+ non-binary flags)
           sf_prescan_tiles   bitmap -> ag_mask / tile_class (only when the
                              caller asks for metadata or statistics)
  Stage 2  sf_conv2d_sparse   bitmap -> y (deterministic gather)

Numerics differ from the reference on purpose: weights stay fp32 and the
sum is fp32, so results match F.conv2d to ~1e-6 instead of fp16 tl.dot
(Kernels/conv2d.py:986,1129-1133).  Inputs with f16(|x|) <= f16(threshold)
count as zero, which is the reference's prescan activity test applied per
element.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .. import _lib
from . import spike_map
from ..Utils.config import PRESCAN_ACTIVITY_EPS, SPARSE_DENSE_RATIO_THRESHOLD
from ..Utils.sparse_helpers import (
    TILE_DENSEISH,
    TILE_SPARSE,
    TILE_UNCERTAIN,
    TILE_ZERO,
    TILE_ZERO_CANDIDATE,
    choose_group_size,
    popcount_buf,
)

__all__ = [
    "sparse_conv2d_forward",
    "choose_group_size",
    "_select_tile_sizes",
    "_select_block_sizes",
    "_popcount_buf",
    "_check_dense_fallback",
    "_build_active_tile_ids",
    "_build_two_stage_metadata",
    "TILE_ZERO",
    "TILE_SPARSE",
    "TILE_DENSEISH",
    "TILE_UNCERTAIN",
    "TILE_ZERO_CANDIDATE",
    "FALLBACK_RATIO",
    "BACKEND_NAME",
]

FALLBACK_RATIO = SPARSE_DENSE_RATIO_THRESHOLD
AUTO_LAUNCH_ALL_ACTIVE_TILE_RATIO = 0.75
GROUP_SIZE = 32
BACKEND_NAME = "sparse_hip"


def _select_tile_sizes(H: int, W: int):
    """Reference metadata tile: 8x16 when H*W >= 3136, else 8x8
    (Kernels/conv2d.py:80-84)."""
    return (8, 16) if H * W >= 3136 else (8, 8)


def _select_block_sizes(H, W, C_IN, C_OUT, kernel_size, N):
    BH, BW = _select_tile_sizes(H, W)
    return BH, BW, BH * BW, 64, choose_group_size(C_IN)


def _popcount_buf(ag_mask_buf: torch.Tensor, N_TILES: int) -> torch.Tensor:
    return popcount_buf(ag_mask_buf, N_TILES)


def _check_dense_fallback(ag_mask_buf, N_TILES, NUM_GROUPS, fallback_ratio=FALLBACK_RATIO) -> bool:
    """Host-syncing test used only by the (disabled) runtime policy."""
    if NUM_GROUPS == 0:
        return False
    avg = _popcount_buf(ag_mask_buf, N_TILES).float().mean().item()
    return avg > fallback_ratio * NUM_GROUPS


def _build_active_tile_ids(tile_class_buf, N_TILES, active_tile_ids_buf=None):
    """Ascending ids of non-zero tiles (torch.nonzero order; host sync).
    Kept for callers of the reference helper (Kernels/conv2d.py:113-123);
    the HIP path itself never compacts on the host."""
    active = torch.nonzero(tile_class_buf[:N_TILES] != TILE_ZERO, as_tuple=False).flatten().to(torch.int32)
    count = int(active.numel())
    if count and active_tile_ids_buf is not None and active_tile_ids_buf.numel() >= count:
        active_tile_ids_buf[:count].copy_(active)
        return active_tile_ids_buf[:count], count
    return active.contiguous(), count


_layout_cache: dict = {}


def _bitmap_layout(desc) -> int:
    """sf_conv2d_bitmap_layout(desc), cached by shape (a pure function of it)."""
    key = (desc.n, desc.c_in, desc.h_in, desc.w_in, desc.c_out, desc.h_out, desc.w_out, desc.kernel, desc.stride,
           desc.pad, desc.in_dtype, desc.out_dtype)
    v = _layout_cache.get(key)
    if v is None:
        if len(_layout_cache) > 256:
            _layout_cache.clear()
        v = _layout_cache[key] = _lib.conv2d_bitmap_layout(desc)
    return v


def _out_hw(H, W, k, s, p, d=1):
    return (H + 2 * p - d * (k - 1) - 1) // s + 1, (W + 2 * p - d * (k - 1) - 1) // s + 1


def _build_two_stage_metadata(x, N, C_IN, H_IN, W_IN, H_OUT, W_OUT, BH, BW, GH, GW, kernel_size, stride,
                              padding, threshold, ag_mask_buf, tile_class_buf, prescan_stats=None,
                              allow_stage1_dense_fallback=False, fallback_ratio=FALLBACK_RATIO, bits=None):
    """Fill ag_mask_buf / tile_class_buf at the reference geometry
    (Kernels/conv2d.py:157-206).  Returns (group_size, num_groups,
    dense_fallback=False, stage1_summary)."""
    gs = choose_group_size(C_IN)
    ng = -(-C_IN // gs)
    if bits is None:
        bits, _ = _lib.prescan_pack(x, threshold)
    n_tiles = N * GH * GW
    if n_tiles:
        _lib.prescan_tiles(bits, N, C_IN, H_IN, W_IN, H_OUT, W_OUT, kernel_size, stride, padding, BH, BW, gs,
                           ag_mask=ag_mask_buf[:n_tiles], tile_class=tile_class_buf[:n_tiles])
    summary = None
    if prescan_stats is not None:
        tc = tile_class_buf[:n_tiles]
        z = int((tc == TILE_ZERO).sum().item())
        d = int((tc == TILE_DENSEISH).sum().item())
        sp = int((tc == TILE_SPARSE).sum().item())
        ratio = float(popcount_buf(ag_mask_buf, n_tiles).sum().item()) / max(float(n_tiles * ng), 1.0)
        summary = {
            "stage1_zero_candidate": z,
            "stage1_denseish": d,
            "stage1_uncertain": sp,
            "stage1_avg_active_group_ratio_lower_bound": ratio,
        }
        prescan_stats.update(summary)
        prescan_stats.update({"final_zero": z, "final_sparse": sp, "final_denseish": d,
                              "stage2_zero_refine_tiles": 0, "stage2_uncertain_tiles": 0,
                              "total_tiles": n_tiles})
    return gs, ng, False, summary


def sparse_conv2d_forward(
    x, weight, bias,
    kernel_size=3, stride=1, padding=0, dilation=1, groups=1,
    threshold=PRESCAN_ACTIVITY_EPS, w_cl=None,
    ag_mask_buf=None, tile_class_buf=None,
    return_ms=False, fallback_ratio=FALLBACK_RATIO,
    return_avg_active_ratio=False, return_tile_stats=False,
    return_backend_meta=False,
    x_nhwc=None, active_tile_ids_buf=None,
    launch_all_tiles=False,
    output_dtype=None,
    workspace=None,
):
    """Sparse conv2d; returns (y, ms) + optional (ratio,), (tile_stats,),
    (backend_meta,) in that order, like Kernels/conv2d.py:893-922.

    `w_cl` may carry this library's cached fp32 tap-major weight
    [C_in*k*k, C_out]; a reference-style fp16 channel-last cache is ignored.
    `x_nhwc`, `active_tile_ids_buf` and `launch_all_tiles` are accepted for
    signature compatibility: the HIP path reads NCHW directly and never
    compacts tiles on the host.  `workspace` (uint8 device tensor) is an
    optional reusable scratch buffer for the bitmap.
    """
    N, C_IN, H_IN, W_IN = (int(v) for v in x.shape)
    C_OUT = int(weight.shape[0])
    out_dtype = x.dtype if output_dtype is None else output_dtype
    if isinstance(stride, (tuple, list)):
        stride = stride[0]
    if isinstance(padding, (tuple, list)):
        padding = padding[0]
    if isinstance(dilation, (tuple, list)):
        dilation = dilation[0]
    stride, padding, dilation, kernel_size = int(stride), int(padding), int(dilation), int(kernel_size)

    def _finalize(y, ms, ratio=None, stats=None, meta=None):
        ret = (y, ms)
        if return_avg_active_ratio:
            ret = ret + (ratio,)
        if return_tile_stats:
            ret = ret + (stats,)
        if return_backend_meta:
            ret = ret + (meta,)
        return ret

    def _dense(reason):
        ms = 0.0
        if return_ms and x.is_cuda:
            se, ee = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            se.record()
        y = F.conv2d(x, weight, bias, stride=stride, padding=padding, dilation=dilation, groups=groups)
        if y.dtype != out_dtype:
            y = y.to(out_dtype)
        if return_ms and x.is_cuda:
            ee.record()
            torch.cuda.synchronize(x.device)
            ms = se.elapsed_time(ee)
        return _finalize(y, ms, 1.0, None, {"backend": "dense_fallback", "reason": reason})

    if groups != 1 or dilation != 1:
        return _dense("unsupported_groups_or_dilation")
    H_OUT, W_OUT = _out_hw(H_IN, W_IN, kernel_size, stride, padding)
    if H_OUT <= 0 or W_OUT <= 0:
        return _dense("invalid_output_shape")
    supported = (kernel_size, stride, padding) in ((1, 1, 0), (1, 2, 0), (3, 1, 1), (3, 2, 1))
    if not supported:
        return _dense("unsupported_pattern")
    if kernel_size == 1 and stride == 2:
        return _dense("split_1x1s2_downsample")
    if not x.is_cuda:
        return _dense("host_tensor")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return _dense("unsupported_dtype")

    lib_out = out_dtype if out_dtype in (x.dtype, torch.float32) else torch.float32
    x = x.contiguous()
    if (
        w_cl is not None and w_cl.dtype == torch.float32 and w_cl.dim() == 2
        and tuple(w_cl.shape) == (C_IN * kernel_size * kernel_size, C_OUT) and w_cl.is_contiguous()
    ):
        wt = w_cl
    else:
        wt = _lib.tap_major_weight(weight)
    b = None if bias is None else bias.detach().to(torch.float32).contiguous()

    desc = _lib.conv_desc(N, C_IN, H_IN, W_IN, C_OUT, H_OUT, W_OUT, kernel_size, stride, padding,
                          _lib.dtype_code(x.dtype), _lib.dtype_code(lib_out))
    ws_bytes = _lib.conv2d_workspace_size(desc)
    if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    y = torch.empty((N, C_OUT, H_OUT, W_OUT), dtype=lib_out, device=x.device)

    BH, BW = _select_tile_sizes(H_OUT, W_OUT)
    GH, GW = -(-H_OUT // BH), -(-W_OUT // BW)
    N_TILES = N * GH * GW
    need_stats = return_avg_active_ratio or return_tile_stats
    need_meta = need_stats or ag_mask_buf is not None or tile_class_buf is not None

    meta = {
        "backend": BACKEND_NAME,
        "reason": "bitmap_gather",
        "total_tiles": N_TILES,
        "launch_count": N * (-(-(H_OUT * W_OUT) // 64)),
        "launch_mode": "all_tiles",
        "launch_mode_reason": "device_side_zero_skip",
    }
    ratio = None
    stats = None
    ms = 0.0

    handed = None
    if not (need_meta or return_ms) and spike_map.recorded(x):
        # The neuron layer that produced x may have written its spike map;
        # tell it which word layout this shape's Stage-2 kernel reads
        # fastest (it writes that layout from its next forward on).
        want = _bitmap_layout(desc)
        accept = (spike_map.PIXEL_MAJOR, spike_map.PLANES) if want == spike_map.PLANES else (spike_map.PIXEL_MAJOR,)
        handed = spike_map.lookup(x, threshold, accept=accept, want=want, consumer=("conv2d", weight.data_ptr()))
    if handed is not None:
        meta["reason"] = "bitmap_gather_handed_spike_map"
        meta["bitmap_layout"] = "planes" if handed[2] == spike_map.PLANES else "pixel_major"
        _lib.conv2d_sparse(desc, handed[0], handed[1], x, wt, b, y, layout=handed[2])
    elif not (need_meta or return_ms):
        _lib.conv2d_forward(desc, x, wt, b, threshold, workspace, y)
    else:
        off = (int(_lib.lib().sf_prescan_bitmap_bytes(N, C_IN, H_IN, W_IN)) + 255) // 256 * 256
        nflags = (int(_lib.lib().sf_prescan_flags_bytes(N, C_IN, H_IN, W_IN)) + 255) // 256 * 256
        bits_t = workspace[:off].view(torch.int32)
        flags_t = workspace[off:off + nflags].view(torch.int32)
        _lib.prescan_pack(x, threshold, bits=bits_t, flags=flags_t)
        if need_meta:
            if ag_mask_buf is None or ag_mask_buf.numel() < N_TILES:
                ag_mask_buf = torch.empty(max(N_TILES, 1), dtype=torch.int32, device=x.device)
            if tile_class_buf is None or tile_class_buf.numel() < N_TILES:
                tile_class_buf = torch.empty(max(N_TILES, 1), dtype=torch.int32, device=x.device)
            prescan_stats = {} if return_tile_stats else None
            gs, ng, _, _ = _build_two_stage_metadata(
                x, N, C_IN, H_IN, W_IN, H_OUT, W_OUT, BH, BW, GH, GW, kernel_size, stride, padding,
                threshold, ag_mask_buf, tile_class_buf, prescan_stats=prescan_stats, bits=bits_t)
            if need_stats:
                tc = tile_class_buf[:N_TILES]
                zc = int((tc == TILE_ZERO).sum().item())
                sc = int((tc == TILE_SPARSE).sum().item())
                dc = int((tc == TILE_DENSEISH).sum().item())
                ratio = float(popcount_buf(ag_mask_buf, N_TILES).sum().item()) / max(float(N_TILES * ng), 1.0)
                meta["active_tiles"] = sc + dc
                if return_tile_stats:
                    stats = {
                        "zero_tiles": zc, "sparse_tiles": sc, "denseish_tiles": dc,
                        "total_tiles": N_TILES, "prescan_mode": "hip_bitmap_v1",
                        "active_tiles": sc + dc,
                        "active_tile_ratio": float(sc + dc) / max(float(N_TILES), 1.0),
                        "denseish_ratio_nonzero": float(dc) / max(float(sc + dc), 1.0),
                    }
                    stats.update(prescan_stats or {})
                if sc + dc == 0:
                    meta["backend"] = "zero_tiles_only"
                    meta["reason"] = "all_tiles_zero_after_metadata"
        if return_ms:
            se, ee = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            se.record()
        _lib.conv2d_sparse(desc, bits_t, flags_t, x, wt, b, y)
        if return_ms:
            ee.record()
            torch.cuda.synchronize(x.device)
            ms = se.elapsed_time(ee)

    if y.dtype != out_dtype:
        y = y.to(out_dtype)
    return _finalize(y, ms, ratio, stats, meta)
