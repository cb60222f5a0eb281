"""Sparse Linear entry point on MI355X (drop-in for Kernels/linear.py).

`sparse_linear_forward` keeps the reference's signature and return tuple
(Kernels/linear.py:460-778): (y, ms) + optional (ratio,), (tile_stats,),
(backend_meta,).  Device tensors go through the C ABI:

  "walk"  sf_linear_prescan  x [m, k] -> row bitmap (+ non-binary flags)
          sf_linear_sparse   bitmap -> y [m, c_out] (lane = row walk of the
                             active elements, weight rows from LDS)
  "mfma"  sf_linear_mfma     the matrix cores with W split into bf16 hi + lo
                             parts (dense tiles), x read and split in the
                             kernel
  "mfma_bits" sf_linear_prescan, then sf_linear_mfma_bits: the same product
                             with the A operand of spike row blocks from the
                             bitmap (flagged blocks read x, split the same
                             way); the row prescan (one read of x) pays off
                             when the output is wide: config 5's 384 -> 1536
                             MLP fc1 takes 18 + 134 us against 207 us, its
                             384 -> 384 projections 19 + 47 against 52 us

The walk does ~density x the MACs on the VALU; the MFMA tile paths do them
all on the matrix cores and win once every 32-wide K slice of a 128-row tile
is live (transformer densities, p ~ 0.1).  `kernel="auto"` takes the walk
for k < 32, "mfma_bits" for c_out >= 2 k and "mfma" otherwise.

Weights stay fp32 and the sum is fp32 (the reference casts x and W to fp16
for tl.dot, Kernels/linear.py:572,720).  Elements with f16(|x|) <=
f16(threshold) count as zero, the reference's activity test per element.
Group metadata (ag_mask / tile_class over BLOCK_M-row tiles) is derived
from the bitmap only when statistics are requested.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .. import _lib
from ..Utils.config import PRESCAN_ACTIVITY_EPS, SPARSE_DENSE_RATIO_THRESHOLD
from ..Utils.sparse_helpers import TILE_DENSEISH, TILE_SPARSE, TILE_ZERO, choose_group_size, popcount_buf

FALLBACK_RATIO = SPARSE_DENSE_RATIO_THRESHOLD
BACKEND_NAME = "sparse_hip"


def _select_linear_block_m(n_rows: int) -> int:
    """Row tile of the metadata (Kernels/linear.py:37-42)."""
    if n_rows >= 1024:
        return 128
    if n_rows >= 256:
        return 64
    return 32


def unpack_row_bits(bits: torch.Tensor, m: int, k: int) -> torch.Tensor:
    """Row bitmap (int32 words, the layout of sf_linear_prescan) -> bool [m, k]."""
    words = int(_lib.lib().sf_linear_bitmap_bytes(m, k)) // 4 // max(m, 1)
    w = bits[: m * words].view(m, words).to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(32, device=bits.device, dtype=torch.int64)
    b = ((w.unsqueeze(-1) >> shifts) & 1).bool().reshape(m, words * 32)
    return b[:, :k]


def group_metadata(active: torch.Tensor, block_m: int, group_size: int):
    """ag_mask / tile_class over block_m-row tiles and group_size-column
    groups of a bool activity matrix [rows, cols] (bit g of a tile's mask =
    any active element in its rows and group g; class 0 / 2 / 1 for none /
    all / some groups): the closed form of the reference's three-stage
    linear metadata (Kernels/linear.py:110-357) and of the bmm prescan
    (Kernels/bmm.py:66-109)."""
    rows, cols = active.shape
    ng = -(-cols // group_size)
    nt = -(-rows // block_m)
    pad = torch.zeros(nt * block_m, ng * group_size, dtype=torch.bool, device=active.device)
    pad[:rows, :cols] = active
    g = pad.view(nt, block_m, ng, group_size).any(dim=3).any(dim=1)  # [nt, ng]
    weights = (1 << torch.arange(ng, device=active.device, dtype=torch.int64))
    mask = (g.to(torch.int64) * weights).sum(dim=1)
    mask = torch.where(mask >= (1 << 31), mask - (1 << 32), mask).to(torch.int32)
    cnt = g.sum(dim=1)
    tile_class = torch.full((nt,), TILE_SPARSE, dtype=torch.int32, device=active.device)
    tile_class[cnt == 0] = TILE_ZERO
    tile_class[cnt == ng] = TILE_DENSEISH
    return mask, tile_class, ng


def tap_weight(weight: torch.Tensor) -> torch.Tensor:
    """Linear weight [c_out, k] -> f32 [k, c_out] (contiguous)."""
    return weight.detach().to(torch.float32).t().contiguous()


def split_weight_bf16(weight: torch.Tensor):
    """Linear weight [c_out, k] -> (hi, lo) bf16 [c_out, kp] with
    hi = bf16(W), lo = bf16(W - hi), kp = k rounded up to 32 (zero padded):
    hi + lo carries ~16 bits of each fp32 weight."""
    w = weight.detach().to(torch.float32)
    c_out, k = w.shape
    kp = -(-k // 32) * 32
    hi = torch.zeros(c_out, kp, dtype=torch.bfloat16, device=w.device)
    lo = torch.zeros(c_out, kp, dtype=torch.bfloat16, device=w.device)
    hi[:, :k] = w.to(torch.bfloat16)
    lo[:, :k] = (w - hi[:, :k].float()).to(torch.bfloat16)
    return hi, lo


def sparse_linear_forward(
    x,
    weight,
    bias=None,
    threshold=PRESCAN_ACTIVITY_EPS,
    w_t=None,
    ag_mask_buf=None,
    tile_class_buf=None,
    return_ms=False,
    fallback_ratio=FALLBACK_RATIO,
    return_avg_active_ratio=False,
    return_tile_stats=False,
    return_backend_meta=False,
    active_tile_ids_buf=None,
    launch_all_tiles=False,
    output_dtype=None,
    workspace=None,
    w_split=None,
    kernel="auto",
):
    """Sparse linear y = x @ weight^T + bias for x [N, C_IN].

    `kernel` picks "walk", "mfma", "mfma_bits" or "auto" (see the module
    docstring);
    `w_split` may carry the cached (hi, lo) of split_weight_bf16.

    `w_t` may carry a cached weight^T [C_IN, C_OUT] (f32 is used as is,
    other dtypes are converted).  `active_tile_ids_buf` and
    `launch_all_tiles` are accepted for signature compatibility: every row
    tile is launched and zero rows cost only their store.  `workspace`
    (uint8 device tensor) optionally holds the bitmap between calls.
    """
    out_dtype = x.dtype if output_dtype is None else output_dtype
    need_stats = return_avg_active_ratio or return_tile_stats

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
        y = F.linear(x, weight.to(x.dtype), None if bias is None else bias.to(x.dtype))
        if y.dtype != out_dtype:
            y = y.to(out_dtype)
        if return_ms and x.is_cuda:
            ee.record()
            torch.cuda.synchronize(x.device)
            ms = se.elapsed_time(ee)
        return _finalize(y, ms, 1.0, None, {"backend": "dense_fallback", "reason": reason})

    if x.dim() != 2:
        return _dense("expected_2d_input")
    N, C_IN = (int(v) for v in x.shape)
    C_OUT = int(weight.shape[0])
    if N <= 0 or C_IN <= 0 or C_OUT <= 0:
        y = torch.zeros(max(N, 0), max(C_OUT, 0), dtype=out_dtype, device=x.device)
        return _finalize(y, 0.0, 0.0, None, {"backend": "zero_tiles_only", "reason": "empty_shape", "total_tiles": 0})
    if not x.is_cuda:
        return _dense("host_tensor")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return _dense("unsupported_dtype")
    if C_OUT % 4 != 0:
        return _dense("c_out_not_multiple_of_4")

    x = x.contiguous()
    lib_out = out_dtype if out_dtype in (x.dtype, torch.float32) else torch.float32
    use_mfma = kernel in ("mfma", "mfma_bits") or (kernel == "auto" and C_IN >= 32)
    mfma_bits = kernel == "mfma_bits" or (kernel == "auto" and C_IN >= 32 and C_OUT >= 2 * C_IN)
    wt = None
    if not use_mfma:
        if w_t is not None and tuple(w_t.shape) == (C_IN, C_OUT):
            wt = w_t if (w_t.dtype == torch.float32 and w_t.is_contiguous()) else w_t.detach().float().contiguous()
        else:
            wt = tap_weight(weight)
    b = None if bias is None else bias.detach().to(torch.float32).contiguous()
    y = torch.empty((N, C_OUT), dtype=lib_out, device=x.device)

    BLOCK_M = _select_linear_block_m(N)
    N_TILES = -(-N // BLOCK_M)
    meta = {
        "backend": BACKEND_NAME,
        "reason": "linear_row_bitmap",
        "total_tiles": int(N_TILES),
        "launch_count": int(-(-N // 64)),
        "launch_mode": "all_tiles",
        "launch_mode_reason": "device_side_zero_skip",
    }
    ratio = stats = None
    ms = 0.0
    if use_mfma:
        if w_split is None or tuple(w_split[0].shape) != (C_OUT, -(-C_IN // 32) * 32):
            w_split = split_weight_bf16(weight)
        meta["reason"] = "linear_mfma_bitmap" if mfma_bits else "linear_mfma_bf16x2"
        meta["launch_count"] = int(-(-N // 128) * -(-C_OUT // 128))
    if use_mfma and not need_stats:
        if return_ms:
            se, ee = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            se.record()
        if mfma_bits:
            bits, flags = _lib.linear_prescan(x, threshold)
            _lib.linear_mfma_bits(bits, flags, x, w_split[0], w_split[1], b, y, threshold)
        else:
            _lib.linear_mfma(x, w_split[0], w_split[1], b, y, threshold)
        if return_ms:
            ee.record()
            torch.cuda.synchronize(x.device)
            ms = se.elapsed_time(ee)
    elif not (need_stats or return_ms):
        ws_bytes = _lib.linear_workspace_size(N, C_IN)
        if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
            workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        _lib.linear_forward(x, wt, b, threshold, y, workspace)
    else:
        bits, flags = _lib.linear_prescan(x, threshold)
        if need_stats:
            gs = choose_group_size(C_IN)
            mask, tc, ng = group_metadata(unpack_row_bits(bits, N, C_IN), BLOCK_M, gs)
            if ag_mask_buf is not None and ag_mask_buf.numel() >= N_TILES:
                ag_mask_buf[:N_TILES].copy_(mask)
            if tile_class_buf is not None and tile_class_buf.numel() >= N_TILES:
                tile_class_buf[:N_TILES].copy_(tc)
            zc = int((tc == TILE_ZERO).sum().item())
            sc = int((tc == TILE_SPARSE).sum().item())
            dc = int((tc == TILE_DENSEISH).sum().item())
            ratio = float(popcount_buf(mask, N_TILES).sum().item()) / max(float(N_TILES * ng), 1.0)
            meta["active_tiles"] = sc + dc
            meta["avg_active_group_ratio"] = ratio
            if return_tile_stats:
                stats = {
                    "zero_tiles": zc, "sparse_tiles": sc, "denseish_tiles": dc,
                    "total_tiles": int(N_TILES), "prescan_mode": "hip_row_bitmap_v1",
                    "active_tiles": sc + dc,
                    "active_tile_ratio": float(sc + dc) / max(float(N_TILES), 1.0),
                    "denseish_ratio_nonzero": float(dc) / max(float(sc + dc), 1.0),
                    "avg_active_group_ratio": ratio,
                    "block_m": int(BLOCK_M), "group_size_c": int(gs), "num_groups": int(ng),
                }
        if return_ms:
            se, ee = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            se.record()
        if mfma_bits:
            _lib.linear_mfma_bits(bits, flags, x, w_split[0], w_split[1], b, y, threshold)
        elif use_mfma:
            _lib.linear_mfma(x, w_split[0], w_split[1], b, y, threshold)
        else:
            _lib.linear_sparse(bits, flags, x, wt, b, y)
        if return_ms:
            ee.record()
            torch.cuda.synchronize(x.device)
            ms = se.elapsed_time(ee)
    if y.dtype != out_dtype:
        y = y.to(out_dtype)
    return _finalize(y, ms, ratio, stats, meta)
