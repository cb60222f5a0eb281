"""SparseLinear: spike-sparse Linear module (drop-in for Ops/sparse_linear.py).

Same constructor, `from_dense`, input flattening ([..., in_features], or a
[T, B, C, H, W] input with C*H*W == in_features), runtime policy state and
diagnostics as the reference module (Ops/sparse_linear.py:68-890).  On ROCm
device tensors the forward runs Kernels.linear.sparse_linear_forward (the
library's row-bitmap kernels); if the native library is not built the call
raises.  Host tensors run F.linear, the reference module's own CPU
behaviour (Ops/sparse_linear.py:821-836).
"""

from __future__ import annotations

import time
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..Kernels.linear import BACKEND_NAME, sparse_linear_forward, split_weight_bf16, tap_weight
from ..Utils import config as _config
from ..Utils.config import PRESCAN_ACTIVITY_EPS, SPARSE_DENSE_RATIO_THRESHOLD
from .sparse_conv2d import _ProfileStats


class SparseLinear(nn.Module):
    """Linear whose forward skips inactive (zero) input elements."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        bias: bool = True,
        threshold: float = PRESCAN_ACTIVITY_EPS,
        return_ms: bool = False,
        dense_threshold: float = SPARSE_DENSE_RATIO_THRESHOLD,
        fallback_ratio: float = SPARSE_DENSE_RATIO_THRESHOLD,
        launch_all_tiles: bool = False,
        warmup_steps: int = 8,
        calib_every: int = 32,
        ema_decay: float = 0.9,
        zero_streak_needed: int = 2,
        profile_runtime: bool = False,
    ):
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.threshold = float(threshold)
        self.return_ms = bool(return_ms)
        self.fallback_ratio = float(fallback_ratio)
        self.launch_all_tiles = bool(launch_all_tiles)
        self.weight = nn.Parameter(torch.empty(self.out_features, self.in_features))
        if bias:
            self.bias = nn.Parameter(torch.empty(self.out_features))
        else:
            self.register_parameter("bias", None)
        nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)
        if self.bias is not None:
            bound = 1.0 / max(float(self.in_features), 1.0) ** 0.5
            nn.init.uniform_(self.bias, -bound, bound)

        self._last_sparse_ms = 0.0
        self._last_dense_ms = 0.0
        self._last_avg_active_ratio = -1.0
        self._w_t = None
        self._w_t_key = None
        self._w_split = None
        self._w_split_key = None
        # Stage-2 kernel: "auto" (matrix cores for in_features >= 32), "mfma"
        # or "walk" (the spike walk; fewer MACs at very low densities).
        self.kernel = "auto"
        self._workspace = None
        self._warmup_left = int(max(0, warmup_steps))
        self._calib_every = int(max(1, calib_every))
        self._ema_decay = float(ema_decay)
        self._dense_threshold = float(dense_threshold)
        self._zero_streak_needed = int(max(1, zero_streak_needed))
        self._zero_streak = 0
        self._forward_count = 0
        self._ema_active_ratio: Optional[float] = None
        self._force_zero = False
        self._force_dense = False
        self._inference_mode = False
        self.runtime_policy = bool(_config.ENABLE_RUNTIME_FALLBACK_POLICY)

        self.collect_diag = False
        self._last_diag: Dict[str, Any] = {}
        self.profile_runtime = bool(profile_runtime)
        self._profile = _ProfileStats()
        self.backend_family = "sparse_linear"
        self.diag_path = "runtime"
        self.fallback_reason = ""
        self.meta_source = "measured"
        self.diag_source = "measured"
        self.support_status = "supported"
        self.score_family = "linear"
        self.backend_mode = "sparse"
        self._runtime_dispatch_calls = 0
        self._runtime_dispatch_disagree = 0

    @classmethod
    def from_dense(cls, linear: nn.Linear, threshold: float = PRESCAN_ACTIVITY_EPS, return_ms: bool = False,
                   **kwargs) -> "SparseLinear":
        sparse = cls(in_features=linear.in_features, out_features=linear.out_features,
                     bias=linear.bias is not None, threshold=threshold, return_ms=return_ms,
                     **kwargs).to(linear.weight.device)
        with torch.no_grad():
            sparse.weight.copy_(linear.weight)
            if linear.bias is not None:
                sparse.bias.copy_(linear.bias)
        return sparse

    def set_inference_mode(self, enabled: bool):
        self._inference_mode = bool(enabled)
        if enabled:
            self.collect_diag = False
            self.profile_runtime = False

    def _stamp(self) -> float:
        if self.profile_runtime and self.weight.is_cuda:
            torch.cuda.synchronize(self.weight.device)
        return time.perf_counter()

    def _elapsed_ms(self, t0: float) -> float:
        if self.profile_runtime and self.weight.is_cuda:
            torch.cuda.synchronize(self.weight.device)
        return (time.perf_counter() - t0) * 1000.0

    def get_profile_summary(self) -> str:
        p = self._profile
        if p.calls == 0:
            return "SparseLinear runtime profile: no calls"
        avg = lambda v: v / max(1, p.calls)  # noqa: E731
        return (
            "SparseLinear runtime profile\n"
            f"  calls={p.calls}, last_path={p.last_path}\n"
            f"  hits: zero={p.zero_path_hits}, sparse={p.sparse_path_hits}, dense={p.dense_path_hits}\n"
            f"  avg total={avg(p.total_ms):.4f} ms, last total={p.last_total_ms:.4f} ms\n"
            f"  avg sparse_kernel={avg(p.sparse_kernel_ms):.4f} ms\n"
            f"  avg dense_fallback={avg(p.dense_fallback_ms):.4f} ms\n"
            f"  last avg_active_ratio={p.last_avg_active_ratio:.6f}"
        )

    def _supports_sparse(self) -> bool:
        return self.in_features > 0 and self.out_features > 0 and self.out_features % 4 == 0

    def _get_w_t(self) -> torch.Tensor:
        """f32 weight^T [in, out], rebuilt when the weight changes (the
        reference keys its fp16 cache on weight._version,
        Ops/sparse_linear.py:251-257)."""
        key = (self.weight._version, self.weight.data_ptr(), self.weight.device)
        if self._w_t is None or self._w_t_key != key:
            self._w_t = tap_weight(self.weight)
            self._w_t_key = key
        return self._w_t

    def _get_w_split(self):
        key = (self.weight._version, self.weight.data_ptr(), self.weight.device)
        if self._w_split is None or self._w_split_key != key:
            self._w_split = split_weight_bf16(self.weight)
            self._w_split_key = key
        return self._w_split

    def _flatten_input(self, x: torch.Tensor) -> Tuple[torch.Tensor, Tuple]:
        if x.dim() < 2:
            raise ValueError(f"Expected at least 2D input, got {x.dim()}D")
        if x.shape[-1] == self.in_features:
            return x.reshape(-1, self.in_features), ("lastdim", x.shape[:-1])
        if x.dim() == 5 and x.shape[2] * x.shape[3] * x.shape[4] == self.in_features:
            t, b = x.shape[0], x.shape[1]
            return x.reshape(t * b, self.in_features), ("tbchw", t, b)
        raise ValueError(
            f"Input shape {tuple(x.shape)} is incompatible with in_features={self.in_features}. "
            f"Need x.shape[-1] == in_features, or for 5D input C*H*W == in_features.")

    def _restore_output(self, y2d: torch.Tensor, meta: Tuple) -> torch.Tensor:
        if meta[0] == "lastdim":
            return y2d.reshape(*meta[1], self.out_features)
        return y2d.reshape(meta[1], meta[2], self.out_features)

    def _zero_output_2d(self, x2d: torch.Tensor) -> torch.Tensor:
        y = torch.zeros(x2d.shape[0], self.out_features, dtype=x2d.dtype, device=x2d.device)
        if self.bias is not None:
            y = y + self.bias.detach().to(y.dtype).view(1, -1)
        return y

    # ---- runtime policy (Ops/sparse_linear.py:357-410), off by default --------
    def _should_collect_ratio(self) -> bool:
        if not self.runtime_policy or self._inference_mode:
            return False
        if self._warmup_left > 0:
            return True
        return (self._forward_count % self._calib_every) == 0

    def _update_policy(self, avg_active_ratio: Optional[float]):
        if avg_active_ratio is None:
            return
        self._last_avg_active_ratio = float(avg_active_ratio)
        if not self.runtime_policy:
            return
        if self._warmup_left > 0:
            self._warmup_left -= 1
            self._ema_active_ratio = avg_active_ratio
            return
        if self._ema_active_ratio is None:
            self._ema_active_ratio = avg_active_ratio
        else:
            self._ema_active_ratio = self._ema_decay * self._ema_active_ratio + (1 - self._ema_decay) * avg_active_ratio
        if avg_active_ratio == 0.0:
            self._zero_streak += 1
        else:
            self._zero_streak = 0
            self._force_zero = False
        if self._zero_streak >= self._zero_streak_needed:
            self._force_zero = True
        self._force_dense = self._ema_active_ratio > self._dense_threshold

    def _record_runtime_dispatch(self, runtime_backend: str):
        expected = str(getattr(self, "sf_dispatch_decision", getattr(self, "sf_backend_mode", "")))
        self._runtime_dispatch_calls += 1
        if expected and expected != runtime_backend:
            self._runtime_dispatch_disagree += 1

    def _get_workspace(self, x2d: torch.Tensor) -> torch.Tensor:
        from .. import _lib
        need = _lib.linear_workspace_size(int(x2d.shape[0]), self.in_features)
        ws = self._workspace
        if ws is None or ws.device != x2d.device or ws.numel() < need:
            ws = torch.empty(max(need, 256), dtype=torch.uint8, device=x2d.device)
            self._workspace = ws
        return ws

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        self.fallback_reason = ""
        if self.profile_runtime:
            self._profile.calls += 1
            t_total = self._stamp()
        x2d, restore = self._flatten_input(x)
        if self.runtime_policy and self._force_zero:
            y2d = self._zero_output_2d(x2d)
            self.fallback_reason = "force_zero_policy"
            self._record_runtime_dispatch("staticzero")
            if self.profile_runtime:
                self._profile.zero_path_hits += 1
                self._profile.last_path = "zero(force)"
            return self._restore_output(y2d, restore)

        forced_dense = self.runtime_policy and self._force_dense
        need_ratio = x2d.is_cuda and not forced_dense and self._should_collect_ratio()
        self._forward_count += 1
        ratio = None
        if x2d.is_cuda and self._supports_sparse() and self.backend_mode != "dense" and not forced_dense:
            want_diag = self.collect_diag and not self._inference_mode
            res = sparse_linear_forward(
                x2d, self.weight, self.bias, threshold=self.threshold,
                w_t=self._get_w_t() if self.kernel == "walk" or self.in_features < 32 else None,
                w_split=None if self.kernel == "walk" or self.in_features < 32 else self._get_w_split(),
                kernel=self.kernel,
                return_ms=self.return_ms, return_avg_active_ratio=want_diag or need_ratio,
                return_tile_stats=want_diag, return_backend_meta=True, output_dtype=x2d.dtype,
                workspace=self._get_workspace(x2d))
            y2d, ms = res[0], res[1]
            idx = 2
            stats = None
            if want_diag or need_ratio:
                ratio = res[idx]
                idx += 1
            if want_diag:
                stats = res[idx]
                idx += 1
            meta = res[idx]
            self._last_sparse_ms, self._last_dense_ms = float(ms), 0.0
            path = "sparse"
            self._record_runtime_dispatch("sparse")
            if self.profile_runtime:
                self._profile.sparse_path_hits += 1
                self._profile.sparse_kernel_ms += self._last_sparse_ms
            if want_diag:
                st = stats or {}
                self._last_diag = {
                    "sparse_path_executed": True, "backend": meta.get("backend", BACKEND_NAME),
                    "backend_reason": meta.get("reason"), "active_group_ratio": float(ratio),
                    "total_tile_count": int(st.get("total_tiles", 0)),
                    "tile_zero_count": int(st.get("zero_tiles", 0)),
                    "tile_zero_ratio": float(st.get("zero_tiles", 0)) / max(float(st.get("total_tiles", 1)), 1.0),
                    "sparse_tiles": int(st.get("sparse_tiles", 0)),
                    "denseish_tiles": int(st.get("denseish_tiles", 0)),
                    "backend_family": self.backend_family, "diag_path": self.diag_path,
                    "sparse_compute_ms": float(ms),
                }
        else:
            y2d = self._fallback_forward(x2d)
            path = "dense"
            self.fallback_reason = ("force_dense" if forced_dense else
                                    "dispatch_dense" if self.backend_mode == "dense" else "module_dense_path")
            self._record_runtime_dispatch("dense")
            if self.profile_runtime:
                self._profile.dense_path_hits += 1
        self._update_policy(ratio)
        if self.runtime_policy and self._force_zero and ratio == 0.0:
            y2d = self._zero_output_2d(x2d)
            path = "zero(promoted)"
            self.fallback_reason = "zero_promoted_policy"
        y = self._restore_output(y2d, restore)
        if self.profile_runtime:
            self._profile.last_path = path
            self._profile.last_avg_active_ratio = self._last_avg_active_ratio
            ms_total = self._elapsed_ms(t_total)
            self._profile.total_ms += ms_total
            self._profile.last_total_ms = ms_total
        if self.collect_diag:
            self._last_diag["fallback_reason"] = str(self.fallback_reason)
            self._last_diag["egd_runtime_calls"] = int(self._runtime_dispatch_calls)
            self._last_diag["egd_runtime_disagree_count"] = int(self._runtime_dispatch_disagree)
        return y

    def _fallback_forward(self, x2d: torch.Tensor) -> torch.Tensor:
        t0 = self._stamp() if self.profile_runtime else 0.0
        y = F.linear(x2d, self.weight.to(x2d.dtype), None if self.bias is None else self.bias.to(x2d.dtype))
        self._last_sparse_ms = 0.0
        self._last_dense_ms = self._elapsed_ms(t0) if self.profile_runtime else 0.0
        if self.profile_runtime:
            self._profile.dense_fallback_ms += self._last_dense_ms
        return y

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, threshold={self.threshold}, return_ms={self.return_ms}, "
                f"inference_mode={self._inference_mode}")
