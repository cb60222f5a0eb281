"""SparseConv2d: spike-sparse Conv2d module (drop-in for Ops/sparse_conv2d.py).

Same constructor, `from_dense`, 4-D / 5-D forward, public state and
diagnostics as the reference module (Ops/sparse_conv2d.py:109-848).  On ROCm
device tensors the forward runs the HIP two-stage path through
Kernels.conv2d.sparse_conv2d_forward; if the native library is not built
the call raises instead of silently running dense.  Host (CPU) tensors run
F.conv2d, which is the reference module's own CPU behaviour
(Ops/sparse_conv2d.py:557,819-834).

`block_size` is live here: it is the square output tile at which
diagnostics report per-(n, tile) active-channel lists (the reference
carries it but never uses it, Ops/sparse_conv2d.py:114-119).
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _lib
from ..Kernels.conv2d import BACKEND_NAME, _select_tile_sizes, choose_group_size, sparse_conv2d_forward
from ..Utils import config as _config
from ..Utils.block_selector import select_block_size
from .static_zero_conv2d import ZERO_BACKEND_FAMILY, make_zero_conv_output  # noqa: F401


@dataclass
class _ProfileStats:
    calls: int = 0
    zero_path_hits: int = 0
    sparse_path_hits: int = 0
    dense_path_hits: int = 0
    triton_supported_calls: int = 0  # name kept for readers of the reference stats
    total_ms: float = 0.0
    policy_ms: float = 0.0
    reshape_ms: float = 0.0
    buffer_ms: float = 0.0
    sparse_kernel_ms: float = 0.0
    dense_fallback_ms: float = 0.0
    output_pack_ms: float = 0.0
    last_path: str = "none"
    last_total_ms: float = 0.0
    last_sparse_kernel_ms: float = 0.0
    last_dense_fallback_ms: float = 0.0
    last_avg_active_ratio: float = -1.0


def _pair(v):
    return (int(v), int(v)) if isinstance(v, int) else tuple(int(t) for t in v)


class SparseConv2d(nn.Module):
    """Conv2d whose forward skips inactive (zero) spikes.

    Supported sparse patterns: 3x3/s1/p1, 3x3/s2/p1, 1x1/s1/p0 with
    groups=1, dilation=1.  Anything else runs dense F.conv2d, as in the
    reference (Kernels/conv2d.py:955-973).
    """

    def __init__(
        self,
        in_channels, out_channels, kernel_size,
        stride=1, padding=0, dilation=1, groups=1, bias=True,
        block_size=None, threshold=1e-6, return_ms=False,
        dense_threshold: float = 0.85,
        warmup_steps: int = 8, calib_every: int = 32,
        ema_decay: float = 0.9, zero_streak_needed: int = 2,
        profile_runtime: bool = False,
        allow_sparse_1x1: bool = True,
        launch_all_tiles: bool = False,
    ):
        super().__init__()
        self.in_channels = int(in_channels)
        self.out_channels = int(out_channels)
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        self.groups = int(groups)
        self.block_size = block_size
        self.threshold = float(threshold)
        self.return_ms = bool(return_ms)
        self.allow_sparse_1x1 = bool(allow_sparse_1x1)
        self.launch_all_tiles = bool(launch_all_tiles)

        self.weight = nn.Parameter(torch.empty(self.out_channels, self.in_channels // self.groups, *self.kernel_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(self.out_channels))
        else:
            self.register_parameter("bias", None)
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            fan_in = self.in_channels * self.kernel_size[0] * self.kernel_size[1]
            bound = 1 / math.sqrt(fan_in) if fan_in > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

        self._w_tap = None
        self._w_tap_key = None
        self._workspace = None
        self._last_sparse_ms = 0.0
        self._last_dense_ms = 0.0
        self._last_avg_active_ratio = -1.0
        self._dense_threshold = float(dense_threshold)
        self._warmup_left = int(max(0, warmup_steps))
        self._calib_every = int(max(1, calib_every))
        self._ema_decay = float(ema_decay)
        self._zero_streak_needed = int(max(1, zero_streak_needed))
        self._forward_count = 0
        self._inference_mode = False
        # Runtime fallback policy (Ops/sparse_conv2d.py:449-496): an EMA of
        # the active-group ratio forces dense above dense_threshold, a streak
        # of all-zero inputs forces the zero output.  Off unless enabled in
        # Utils.config or per module via `runtime_policy`, as in the reference.
        self.runtime_policy = bool(_config.ENABLE_RUNTIME_FALLBACK_POLICY)
        self._ema_active_ratio = None
        self._zero_streak = 0
        self._force_dense = False
        self._force_zero = False
        self._runtime_dispatch_seen = 0
        self._runtime_dispatch_mismatch = 0

        self.collect_diag = False
        self._last_diag = {}
        self.profile_runtime = bool(profile_runtime)
        self._profile = _ProfileStats()
        self.backend_family = "sparse_kernel"
        self.diag_path = "conv2d_two_stage_hip"
        self.fallback_reason = ""
        self.meta_source = "measured"
        self.diag_source = "measured"
        self.support_status = "supported"
        self.score_family = "conv"
        # "sparse" (library kernels) or "dense" (F.conv2d), set per layer by
        # Utils.dispatch from measurements.
        self.backend_mode = "sparse"

    # ---- runtime switches (Ops/sparse_conv2d.py:234-250) --------------------
    def set_launch_all_tiles(self, enabled: bool):
        """Kept for API compatibility: the HIP path always launches every
        tile group and skips zero work on the device."""
        self.launch_all_tiles = bool(enabled)

    def set_inference_mode(self, enabled: bool):
        """Disable diagnostics/profiling so a forward never syncs the host."""
        self._inference_mode = bool(enabled)
        if enabled:
            self.collect_diag = False
            self.profile_runtime = False

    # ---- profiling ----------------------------------------------------------
    def _stamp(self):
        if self.profile_runtime and self.weight.is_cuda:
            torch.cuda.synchronize(self.weight.device)
        return time.perf_counter()

    def _elapsed_ms(self, t0):
        if self.profile_runtime and self.weight.is_cuda:
            torch.cuda.synchronize(self.weight.device)
        return (time.perf_counter() - t0) * 1000.0

    def get_profile_summary(self):
        p = self._profile
        if p.calls == 0:
            return "SparseConv2d runtime profile: no calls"
        avg = lambda v: v / max(1, p.calls)  # noqa: E731
        return (
            "SparseConv2d runtime profile\n"
            f"  calls={p.calls}, last_path={p.last_path}\n"
            f"  hits: zero={p.zero_path_hits}, sparse={p.sparse_path_hits}, dense={p.dense_path_hits}\n"
            f"  avg: total={avg(p.total_ms):.3f}, sparse_kernel={avg(p.sparse_kernel_ms):.3f}, "
            f"dense_fallback={avg(p.dense_fallback_ms):.3f}\n"
            f"  last: total={p.last_total_ms:.3f}, path={p.last_path}, active_ratio={p.last_avg_active_ratio:.4f}"
        )

    # ---- helpers --------------------------------------------------------------
    def _supports_sparse(self) -> bool:
        if self.groups != 1 or self.dilation != (1, 1):
            return False
        k, s, p = self.kernel_size, self.stride, self.padding
        if k == (1, 1):
            return self.allow_sparse_1x1 and s == (1, 1) and p == (0, 0)
        return k == (3, 3) and p == (1, 1) and s in ((1, 1), (2, 2))

    def _output_hw(self, h_in: int, w_in: int):
        (kh, kw), (sh, sw), (ph, pw), (dh, dw) = self.kernel_size, self.stride, self.padding, self.dilation
        return (h_in + 2 * ph - dh * (kh - 1) - 1) // sh + 1, (w_in + 2 * pw - dw * (kw - 1) - 1) // sw + 1

    def _get_w_tap(self):
        """fp32 tap-major weight [C_in*k*k, C_out], rebuilt when the weight
        changes (the reference keys its fp16 cache on weight._version,
        Ops/sparse_conv2d.py:339-350)."""
        key = (self.weight._version, self.weight.data_ptr(), self.weight.device)
        if self._w_tap is None or self._w_tap_key != key:
            self._w_tap = _lib.tap_major_weight(self.weight)
            self._w_tap_key = key
        return self._w_tap

    def _get_workspace(self, x4d):
        n, c, h, w = (int(v) for v in x4d.shape)
        need = _lib.conv2d_workspace_size(_lib.conv_desc(n, c, h, w, self.out_channels, 1, 1, 1, 1, 0, 0, 0))
        ws = self._workspace
        if ws is None or ws.device != x4d.device or ws.numel() < need:
            ws = torch.empty(max(need, 256), dtype=torch.uint8, device=x4d.device)
            self._workspace = ws
        return ws

    def _zero_output_4d(self, x):
        h_out, w_out = self._output_hw(int(x.shape[2]), int(x.shape[3]))
        return make_zero_conv_output(int(x.shape[0]), self.out_channels, h_out, w_out, self.bias, x.device, x.dtype)

    def _zero_output_5d(self, x):
        T, B = int(x.shape[0]), int(x.shape[1])
        y = self._zero_output_4d(x.reshape(T * B, *x.shape[2:]))
        return y.reshape(T, B, *y.shape[1:])

    @classmethod
    def from_dense(cls, conv: nn.Conv2d, block_size=None, threshold=1e-6, return_ms=False, **kwargs):
        sparse = cls(
            in_channels=conv.in_channels, out_channels=conv.out_channels,
            kernel_size=conv.kernel_size, stride=conv.stride,
            padding=conv.padding, dilation=conv.dilation,
            groups=conv.groups, bias=conv.bias is not None,
            block_size=block_size, threshold=threshold,
            return_ms=return_ms, **kwargs,
        ).to(conv.weight.device)
        with torch.no_grad():
            sparse.weight.copy_(conv.weight)
            if conv.bias is not None:
                sparse.bias.copy_(conv.bias)
        return sparse

    # ---- runtime policy (Ops/sparse_conv2d.py:323-334,449-496) ---------------------
    def _should_collect_ratio(self) -> bool:
        if not self.runtime_policy or self._inference_mode:
            return False
        if self._warmup_left > 0:
            return True
        return (self._forward_count % self._calib_every) == 0

    def _update_policy(self, avg_active_ratio):
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
        self._zero_streak = self._zero_streak + 1 if avg_active_ratio == 0.0 else 0
        if self._zero_streak >= self._zero_streak_needed:
            self._force_zero = True
        self._force_dense = self._ema_active_ratio > self._dense_threshold

    def _record_runtime_dispatch(self, runtime_backend: str):
        """Count forwards whose path differs from the dispatch decision
        stamped on the module (sf_dispatch_decision / sf_backend_mode)."""
        expected = str(getattr(self, "sf_dispatch_decision", getattr(self, "sf_backend_mode", ""))).strip().lower()
        if not expected:
            return
        self._runtime_dispatch_seen += 1
        if expected != runtime_backend:
            self._runtime_dispatch_mismatch += 1

    # ---- forward ----------------------------------------------------------------
    def forward(self, x: torch.Tensor):
        self.fallback_reason = ""
        if self.profile_runtime:
            self._profile.calls += 1
            t_total = self._stamp()
        if x.dim() not in (4, 5):
            raise ValueError(f"Expected 4D or 5D input, got {x.dim()}D")
        if self.runtime_policy and self._force_zero:
            y = self._zero_output_5d(x) if x.dim() == 5 else self._zero_output_4d(x)
            self._last_sparse_ms = 0.0
            self.fallback_reason = "force_zero"
            self._record_runtime_dispatch("staticzero")
            if self.profile_runtime:
                self._profile.zero_path_hits += 1
                self._profile.last_path = "zero(force)"
                ms = self._elapsed_ms(t_total)
                self._profile.total_ms += ms
                self._profile.last_total_ms = ms
            return y
        if x.dim() == 5:
            T, B = int(x.shape[0]), int(x.shape[1])
            x4d = x.reshape(T * B, *x.shape[2:])
        elif x.dim() == 4:
            x4d = x
        else:
            raise ValueError(f"Expected 4D or 5D input, got {x.dim()}D")

        forced_dense = self.runtime_policy and self._force_dense
        need_ratio = x4d.is_cuda and not forced_dense and self._should_collect_ratio()
        self._forward_count += 1

        ratio = None
        if x4d.is_cuda and self._supports_sparse() and self.backend_mode != "dense" and not forced_dense:
            y4d, backend, ratio = self._hip_forward(x4d, need_ratio)
            path = {"dense_fallback": "dense(fallback)", "zero_tiles_only": "zero(tile_compaction)"}.get(
                backend, "sparse")
            self._record_runtime_dispatch({"dense_fallback": "dense", "zero_tiles_only": "staticzero"}.get(
                backend, "sparse"))
            if self.profile_runtime:
                if path == "sparse":
                    self._profile.sparse_path_hits += 1
                elif path.startswith("zero"):
                    self._profile.zero_path_hits += 1
                else:
                    self._profile.dense_path_hits += 1
        else:
            y4d = self._fallback_forward(x4d)
            path = "dense"
            self.fallback_reason = ("force_dense" if forced_dense else
                                    "dispatch_dense" if self.backend_mode == "dense" else "module_dense_path")
            self._record_runtime_dispatch("dense")
            if self.profile_runtime:
                self._profile.dense_path_hits += 1

        self._update_policy(ratio)
        if self.runtime_policy and self._force_zero and ratio == 0.0:
            y4d = self._zero_output_4d(x4d)
            path = "zero(promoted)"
            self.fallback_reason = "zero_promoted"

        y = y4d.reshape(T, B, *y4d.shape[1:]) if x.dim() == 5 else y4d
        if self.profile_runtime:
            self._profile.last_path = path
            self._profile.last_avg_active_ratio = self._last_avg_active_ratio
            ms = self._elapsed_ms(t_total)
            self._profile.total_ms += ms
            self._profile.last_total_ms = ms
        if self.collect_diag:
            self._last_diag["runtime_dispatch_seen"] = int(self._runtime_dispatch_seen)
            self._last_diag["runtime_dispatch_mismatch"] = int(self._runtime_dispatch_mismatch)
            self._last_diag["fallback_reason"] = str(self.fallback_reason)
        return y

    def _hip_forward(self, x4d, need_ratio=False):
        want_diag = self.collect_diag and not self._inference_mode
        k = self.kernel_size[0]
        result = sparse_conv2d_forward(
            x4d, self.weight, self.bias,
            kernel_size=k, stride=self.stride[0], padding=self.padding[0],
            dilation=self.dilation[0], groups=self.groups, threshold=self.threshold,
            w_cl=self._get_w_tap(),
            return_ms=self.return_ms,
            return_avg_active_ratio=want_diag or need_ratio,
            return_tile_stats=want_diag,
            return_backend_meta=True,
            output_dtype=x4d.dtype,
            workspace=self._get_workspace(x4d),
        )
        y, ms = result[0], result[1]
        idx = 2
        ratio = stats = None
        if want_diag:
            ratio, stats = result[2], result[3]
            idx = 4
        elif need_ratio:
            ratio = result[2]
            idx = 3
        meta = result[idx]
        backend = meta.get("backend", BACKEND_NAME)
        if backend == "dense_fallback":
            self._last_sparse_ms, self._last_dense_ms = 0.0, float(ms)
        else:
            self._last_sparse_ms, self._last_dense_ms = float(ms), 0.0
        if self.profile_runtime:
            self._profile.sparse_kernel_ms += self._last_sparse_ms
            self._profile.last_sparse_kernel_ms = self._last_sparse_ms
        if want_diag:
            self._collect_diag(x4d, ms, ratio, stats, meta)
        return y, backend, ratio

    def _collect_diag(self, x4d, ms, ratio, stats, meta):
        """Diagnostics with host syncs; never enabled on timed runs."""
        from ..Kernels._prescan_common import block_channel_lists

        n, c_in, h, w = (int(v) for v in x4d.shape)
        gs = choose_group_size(c_in)
        ng = -(-c_in // gs)
        h_out, w_out = self._output_hw(h, w)
        bh, bw = _select_tile_sizes(h_out, w_out)
        n_tiles = n * (-(-h_out // bh)) * (-(-w_out // bw))
        stats = stats or {}
        zt = int(stats.get("zero_tiles", 0))
        diag = {
            "sparse_path_executed": True,
            "metadata_kind": "hip_bitmap_v1",
            "group_size": gs, "num_groups": ng,
            "active_group_ratio": float(ratio if ratio is not None else -1.0),
            "nonzero_group_count": float(ratio or 0.0) * n_tiles * ng,
            "total_group_count": float(n_tiles * ng),
            "tile_zero_count": zt, "total_tile_count": n_tiles,
            "tile_zero_ratio": zt / max(n_tiles, 1),
            "effective_k_ratio": float(ratio if ratio is not None else -1.0),
            "sparse_compute_ms": float(ms), "sparse_total_ms": float(ms),
            "zero_tiles": zt,
            "sparse_tiles": int(stats.get("sparse_tiles", 0)),
            "denseish_tiles": int(stats.get("denseish_tiles", 0)),
            "prescan_mode": "hip_bitmap_v1",
            "kernel_type": f"{self.kernel_size[0]}x{self.kernel_size[0]}/s{self.stride[0]}",
            "backend": meta.get("backend"), "backend_reason": meta.get("reason"),
            "launch_tile_count": meta.get("launch_count"),
            "launch_mode_reason": meta.get("launch_mode_reason"),
            "backend_family": self.backend_family, "diag_path": self.diag_path,
        }
        if "active_tiles" in meta:
            diag["active_tiles"] = meta["active_tiles"]
        block = self.block_size or select_block_size(h, w) or 4
        _mask, counts, _lists = block_channel_lists(
            x4d, self.kernel_size[0], self.stride[0], self.padding[0], block, self.threshold)
        diag["block_size"] = int(block)
        diag["block_tiles"] = int(counts.numel())
        diag["block_zero_tiles"] = int((counts == 0).sum().item())
        diag["block_active_channel_ratio"] = float(counts.float().mean().item()) / max(c_in, 1)
        self._last_diag = diag

    def _fallback_forward(self, x):
        if self.profile_runtime:
            t0 = self._stamp()
        y = F.conv2d(x, self.weight, self.bias, self.stride, self.padding, self.dilation, self.groups)
        self._last_sparse_ms = 0.0
        self._last_dense_ms = self._elapsed_ms(t0) if self.profile_runtime else 0.0
        if self.profile_runtime:
            self._profile.dense_fallback_ms += self._last_dense_ms
            self._profile.last_dense_fallback_ms = self._last_dense_ms
        return y

    def extra_repr(self):
        bs = self.block_size if self.block_size is not None else "auto"
        return (
            f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
            f"stride={self.stride}, padding={self.padding}, block_size={bs}, "
            f"return_ms={self.return_ms}, sparse=True, backend=hip_two_stage, "
            f"allow_sparse_1x1={self.allow_sparse_1x1}, inference_mode={self._inference_mode}"
        )
