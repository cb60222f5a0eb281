"""Sparse batched matmul on MI355X (drop-in for Kernels/bmm.py).

`sparse_bmm_forward(a, b, ...)` keeps the reference's signature and return
tuple (Kernels/bmm.py:195-361): C[b] = A[b] @ B[b] with A [B, M, K]
spike-sparse.  Device tensors run one of two kernels, B read through
strides (K^T views need no copy) and staged in LDS per batch:
  sf_bmm_mfma    16-row tiles of A on the matrix cores, both operands split
                 into bf16 hi + lo parts (attention densities: q at p ~ 0.1,
                 the seq x seq scores), chosen when it takes the shape;
  sf_bmm_sparse  each wavefront walks the active elements of A's rows in
                 f32 (very sparse A, or K up to 252).
(The reference casts both operands to fp16 for tl.dot, Kernels/bmm.py:
162-172,305-306.)  Shapes neither kernel takes run torch.bmm, as the
reference's own fallbacks do (Kernels/bmm.py:221-270).
"""

from __future__ import annotations

import torch

from .. import _lib
from ..Utils.config import PRESCAN_ACTIVITY_EPS, SPARSE_DENSE_RATIO_THRESHOLD
from ..Utils.sparse_helpers import TILE_DENSEISH, TILE_SPARSE, TILE_ZERO, choose_group_size, popcount_buf
from .linear import group_metadata

FALLBACK_RATIO = SPARSE_DENSE_RATIO_THRESHOLD


def _bmm_block_m(M: int) -> int:
    """Row tile of the metadata (Kernels/bmm.py:233-238)."""
    return 64 if M >= 128 else (32 if M >= 32 else 16)


def sparse_bmm_forward(
    a: torch.Tensor,
    b: torch.Tensor,
    threshold: float = PRESCAN_ACTIVITY_EPS,
    ag_mask_buf: torch.Tensor = None,
    tile_class_buf: torch.Tensor = None,
    return_ms: bool = False,
    return_avg_active_ratio: bool = False,
    return_tile_stats: bool = False,
    fallback_ratio: float = FALLBACK_RATIO,
    output_dtype=None,
    alpha: float = 1.0,
    kernel: str = "auto",
):
    """Sparse BMM: C[b] = alpha * (A[b] @ B[b]), where A is expected sparse
    (`alpha` folds a following scale, such as attention's, into the
    kernel's store).  `kernel`: "walk" (spike walk over A's active
    elements), "mfma" (matrix-core tiles, for attention densities) or
    "auto" (mfma where it takes the shape, else walk)."""
    if a.ndim != 3 or b.ndim != 3:
        raise ValueError(f"sparse_bmm_forward expects 3-D operands, got {tuple(a.shape)} and {tuple(b.shape)}")
    B_dim, M, K = (int(v) for v in a.shape)
    B2, K2, N = (int(v) for v in b.shape)
    if B_dim != B2 or K != K2:
        raise ValueError(f"bmm shape mismatch: {tuple(a.shape)} @ {tuple(b.shape)}")
    out_dtype = a.dtype if output_dtype is None else output_dtype
    need_stats = return_avg_active_ratio or return_tile_stats

    def _finalize(c, ms, ratio=None, stats=None):
        ret = (c, ms)
        if return_avg_active_ratio:
            ret = ret + (ratio,)
        if return_tile_stats:
            ret = ret + (stats,)
        return ret

    def _dense(reason):
        c = torch.bmm(a.float(), b.float())
        if alpha != 1.0:
            c = c * alpha
        if c.dtype != out_dtype:
            c = c.to(out_dtype)
        stats = {"total_tiles": B_dim * -(-M // _bmm_block_m(M)), "fallback": True, "reason": reason} \
            if return_tile_stats else None
        return _finalize(c, 0.0, 1.0 if return_avg_active_ratio else None, stats)

    if not a.is_cuda:
        return _dense("host_tensor")
    if a.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return _dense("unsupported_dtype")
    if B_dim == 0 or M == 0 or N == 0 or K == 0:
        return _dense("empty_shape")
    use_mfma = kernel == "mfma" or (kernel == "auto" and _lib.bmm_mfma_supported(K, N))
    if use_mfma and not _lib.bmm_mfma_supported(K, N):
        use_mfma = False
    if not use_mfma and not _lib.bmm_supported(K, N):
        return _dense(f"k_too_large_for_lds(k={K})")

    a = a.contiguous()
    if b.dtype != a.dtype:
        b = b.to(a.dtype)
    lib_out = out_dtype if out_dtype in (a.dtype, torch.float32) else torch.float32
    c = torch.empty((B_dim, M, N), dtype=lib_out, device=a.device)

    ratio = stats = None
    if need_stats:
        BM = _bmm_block_m(M)
        gs = choose_group_size(K)
        active = a.abs() >= _lib.activity_cutoff(threshold)
        tiles_m = -(-M // BM)
        pad = torch.zeros(B_dim, tiles_m * BM, K, dtype=torch.bool, device=a.device)
        pad[:, :M] = active
        mask, tc, ng = group_metadata(pad.reshape(B_dim * tiles_m * BM, K), BM, gs)
        total = B_dim * tiles_m
        if ag_mask_buf is not None and ag_mask_buf.numel() >= total:
            ag_mask_buf[:total].copy_(mask)
        if tile_class_buf is not None and tile_class_buf.numel() >= total:
            tile_class_buf[:total].copy_(tc)
        ratio = float(popcount_buf(mask, total).float().mean().item()) / max(ng, 1)
        if return_tile_stats:
            stats = {
                "total_tiles": total,
                "zero_tiles": int((tc == TILE_ZERO).sum().item()),
                "sparse_tiles": int((tc == TILE_SPARSE).sum().item()),
                "denseish_tiles": int((tc == TILE_DENSEISH).sum().item()),
                "fallback": False,
            }
    ms = 0.0
    if return_ms:
        se, ee = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        se.record()
    _lib.bmm_sparse(a, b, threshold, c, alpha, mfma=use_mfma)
    if return_ms:
        ee.record()
        torch.cuda.synchronize(a.device)
        ms = se.elapsed_time(ee)
    if c.dtype != out_dtype:
        c = c.to(out_dtype)
    return _finalize(c, ms, ratio, stats)
