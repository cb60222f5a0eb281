"""SparseLinear: spike-sparse Linear module (drop-in for Ops/sparse_linear.py).

Interface kept from the reference module (Ops/sparse_linear.py:68-890): the
constructor keywords, `from_dense`, inputs of shape [..., in_features] or
[T, B, C, H, W] with C*H*W == in_features, `_last_sparse_ms` /
`_last_dense_ms` / `_last_diag`, `set_inference_mode`, `get_profile_summary`
and the observability attributes the replacer and dispatch read.

On ROCm device tensors the forward runs Kernels.linear.sparse_linear_forward
(row-bitmap prescan + matrix-core or spike-walk Stage 2); without the native
library that call raises.  Host tensors run F.linear, the reference module's
own CPU behaviour (Ops/sparse_linear.py:821-836).  The optional runtime
fallback policy, path profile and weight caches are the shared helpers of
Ops._runtime.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..Kernels.linear import BACKEND_NAME, sparse_linear_forward, split_weight_bf16, tap_weight
from ..Utils import config as _config
from ..Utils.config import PRESCAN_ACTIVITY_EPS, SPARSE_DENSE_RATIO_THRESHOLD
from ._runtime import DispatchAudit, FallbackPolicy, OpReporting, PathProfile, WeightLayout, bias_rows


def _rows_of(x: torch.Tensor, in_features: int) -> Tuple[torch.Tensor, Tuple[int, ...]]:
    """(x as [rows, in_features], the leading shape the output keeps)."""
    if x.dim() >= 2 and x.shape[-1] == in_features:
        return x.reshape(-1, in_features), tuple(x.shape[:-1])
    if x.dim() == 5 and x.shape[2] * x.shape[3] * x.shape[4] == in_features:
        return x.reshape(-1, in_features), tuple(x.shape[:2])
    raise ValueError(f"SparseLinear(in_features={in_features}) cannot take input of shape {tuple(x.shape)}: "
                     f"the last dimension, or C*H*W of a [T, B, C, H, W] input, must equal in_features")


class SparseLinear(OpReporting, nn.Module):
    """Linear whose forward skips inactive (zero) input elements."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 threshold: float = PRESCAN_ACTIVITY_EPS, return_ms: bool = False,
                 dense_threshold: float = SPARSE_DENSE_RATIO_THRESHOLD,
                 fallback_ratio: float = SPARSE_DENSE_RATIO_THRESHOLD, launch_all_tiles: bool = False,
                 warmup_steps: int = 8, calib_every: int = 32, ema_decay: float = 0.9,
                 zero_streak_needed: int = 2, profile_runtime: bool = False):
        super().__init__()
        lin = nn.Linear(int(in_features), int(out_features), bias=bias)  # torch's default init
        self.in_features, self.out_features = lin.in_features, lin.out_features
        self.weight = lin.weight
        self.bias = lin.bias
        self.threshold = float(threshold)
        self.return_ms = bool(return_ms)
        self.fallback_ratio = float(fallback_ratio)
        self.launch_all_tiles = bool(launch_all_tiles)
        # Stage-2 kernel: "auto" (matrix cores for in_features >= 32, over the
        # row bitmap when out_features >= 2 in_features), "mfma", "mfma_bits"
        # or "walk" (the spike walk; fewer MACs at very low densities).
        self.kernel = "auto"
        self.policy = FallbackPolicy(_config.ENABLE_RUNTIME_FALLBACK_POLICY, warmup_steps, calib_every, ema_decay,
                                     dense_threshold, zero_streak_needed, zero_sticky=False)
        self._profile = PathProfile("SparseLinear")
        self._profile.enabled = bool(profile_runtime)
        self._audit = DispatchAudit()
        self._w_t = WeightLayout(tap_weight)
        self._w_split = WeightLayout(split_weight_bf16)
        self._workspace: Optional[torch.Tensor] = None
        self._init_reporting("sparse_linear", "runtime", "linear")
        self._last_dense_ms = 0.0
        self.backend_mode = "sparse"

    @classmethod
    def from_dense(cls, linear: nn.Linear, threshold: float = PRESCAN_ACTIVITY_EPS, return_ms: bool = False,
                   **kwargs) -> "SparseLinear":
        mod = cls(linear.in_features, linear.out_features, bias=linear.bias is not None, threshold=threshold,
                  return_ms=return_ms, **kwargs).to(linear.weight.device)
        with torch.no_grad():
            mod.weight.copy_(linear.weight)
            if linear.bias is not None:
                mod.bias.copy_(linear.bias)
        return mod

    # ---- switches ---------------------------------------------------------------
    @property
    def runtime_policy(self) -> bool:
        return self.policy.enabled

    @runtime_policy.setter
    def runtime_policy(self, on: bool) -> None:
        self.policy.enabled = bool(on)

    @property
    def profile_runtime(self) -> bool:
        return self._profile.enabled

    @profile_runtime.setter
    def profile_runtime(self, on: bool) -> None:
        self._profile.enabled = bool(on)

    @property
    def _last_avg_active_ratio(self) -> float:
        return self.policy.last_ratio

    def get_profile_summary(self) -> str:
        return self._profile.summary()

    def _supports_sparse(self) -> bool:
        return self.in_features > 0 and self.out_features > 0 and self.out_features % 4 == 0

    def _workspace_for(self, rows: int, device) -> torch.Tensor:
        from .. import _lib
        need = max(_lib.linear_workspace_size(rows, self.in_features), 256)
        ws = self._workspace
        if ws is None or ws.device != device or ws.numel() < need:
            ws = self._workspace = torch.empty(need, dtype=torch.uint8, device=device)
        return ws

    # ---- forward ---------------------------------------------------------------
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2d, lead = _rows_of(x, self.in_features)
        dev = x2d.device
        t0 = self._profile.start(dev)
        self.fallback_reason = ""
        ratio = None
        forced = self.policy.forced
        if forced == FallbackPolicy.ZERO:
            y2d = bias_rows(self.bias, (x2d.shape[0],), self.out_features, (), x2d.dtype, dev)
            path, self.fallback_reason = "zero(force)", "force_zero_policy"
            self._audit.record(self, "staticzero")
        elif x2d.is_cuda and self._supports_sparse() and self.backend_mode != "dense" and forced is None:
            y2d, ratio = self._sparse(x2d)
            path = "sparse"
            self._audit.record(self, "sparse")
        else:
            y2d = self._dense(x2d)
            path = "dense"
            self.fallback_reason = {FallbackPolicy.DENSE: "force_dense"}.get(
                forced, "dispatch_dense" if self.backend_mode == "dense" else "module_dense_path")
            self._audit.record(self, "dense")
        if forced != FallbackPolicy.ZERO:
            self.policy.forwards += 1
            self.policy.observe(ratio)
            if ratio == 0.0 and self.policy.forced == FallbackPolicy.ZERO:
                # This forward's input was already all-zero: its output is the
                # bias rows the zero path would give.
                path, self.fallback_reason = "zero(promoted)", "zero_promoted_policy"
        self._profile.finish(path, self._profile.elapsed(t0, dev), self.policy.last_ratio)
        if self.collect_diag:
            self._last_diag.update(fallback_reason=str(self.fallback_reason),
                                   egd_runtime_calls=self._audit.seen,
                                   egd_runtime_disagree_count=self._audit.mismatch)
        return y2d.reshape(*lead, self.out_features)

    def _sparse(self, x2d: torch.Tensor):
        diag = self.collect_diag and not self._inference_mode
        want_ratio = diag or (x2d.is_cuda and self.policy.wants_ratio(self._inference_mode))
        walk = self.kernel == "walk" or self.in_features < 32
        out = sparse_linear_forward(
            x2d, self.weight, self.bias, threshold=self.threshold,
            w_t=self._w_t(self.weight) if walk else None,
            w_split=None if walk else self._w_split(self.weight),
            kernel=self.kernel, return_ms=self.return_ms, return_avg_active_ratio=want_ratio,
            return_tile_stats=diag, return_backend_meta=True, output_dtype=x2d.dtype,
            workspace=self._workspace_for(int(x2d.shape[0]), x2d.device))
        y2d, ms, rest = out[0], float(out[1]), list(out[2:])
        ratio = rest.pop(0) if want_ratio else None
        stats = rest.pop(0) if diag else None
        meta = rest.pop(0)
        self._last_sparse_ms, self._last_dense_ms = ms, 0.0
        self._profile.add("sparse_kernel", ms)
        if diag:
            st = stats or {}
            total = int(st.get("total_tiles", 0))
            zero = int(st.get("zero_tiles", 0))
            self._last_diag = {
                "sparse_path_executed": True, "backend": meta.get("backend", BACKEND_NAME),
                "backend_reason": meta.get("reason"), "active_group_ratio": float(ratio),
                "total_tile_count": total, "tile_zero_count": zero, "tile_zero_ratio": zero / max(total, 1),
                "sparse_tiles": int(st.get("sparse_tiles", 0)), "denseish_tiles": int(st.get("denseish_tiles", 0)),
                "backend_family": self.backend_family, "diag_path": self.diag_path, "sparse_compute_ms": ms,
            }
        return y2d, ratio

    def _dense(self, x2d: torch.Tensor) -> torch.Tensor:
        t0 = self._profile.start(x2d.device)
        b = None if self.bias is None else self.bias.to(x2d.dtype)
        y = F.linear(x2d, self.weight.to(x2d.dtype), b)
        self._last_sparse_ms = 0.0
        self._last_dense_ms = self._profile.elapsed(t0, x2d.device)
        self._profile.add("dense_fallback", self._last_dense_ms)
        return y

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, threshold={self.threshold}, return_ms={self.return_ms}, "
                f"kernel={self.kernel}, inference_mode={self._inference_mode}")
