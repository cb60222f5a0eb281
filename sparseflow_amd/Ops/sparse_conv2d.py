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

import ctypes
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _lib
from ..Kernels import spike_map
from ..Kernels.conv2d import BACKEND_NAME, _select_tile_sizes, choose_group_size, sparse_conv2d_forward
from ..Utils import config as _config
from ..Utils.block_selector import select_block_size
from ._runtime import DispatchAudit, FallbackPolicy, OpReporting, PathProfile, WeightLayout, bias_rows
from .static_zero_conv2d import ZERO_BACKEND_FAMILY, make_zero_conv_output  # noqa: F401


def _pair(v):
    return (int(v), int(v)) if isinstance(v, int) else tuple(int(t) for t in v)


class _InferencePlan:
    """The steady-state inference forward of one input shape, resolved once.

    After a full forward that ran the library's one-call path
    (sf_conv2d_forward: prescan + Stage 2, or the fused kernel) in inference
    mode, everything that call needed except x and y is fixed: the
    descriptor, the cached tap-major weight, the fp32 bias, the workspace,
    the output shape.  `run` repeats that call for a new x of the same
    shape, dtype and device with one allocation (y) and one foreign call, and
    returns None -- the full forward then runs -- whenever anything the plan
    was built from has changed: the weight or bias (object or in-place
    version), the threshold, or a module switch that selects another path.
    Inputs that a neuron layer handed a spike map for take the full forward,
    which reads the map instead of x.
    """

    __slots__ = ("shape", "out_shape", "dtype", "device", "index", "threshold", "weight", "wver", "bias", "bver",
                 "desc", "desc_addr", "wt", "wt_ptr", "b32", "b_ptr", "ws", "ws_ptr", "ws_bytes", "fn")

    def __init__(self, module, x, desc, wt, b32, ws):
        self.shape = x.shape
        self.out_shape = (*x.shape[:-3], desc.c_out, desc.h_out, desc.w_out)
        self.dtype = x.dtype
        self.device = x.device
        self.index = x.get_device()
        self.threshold = module.threshold
        self.weight = module.weight
        self.wver = module.weight._version
        self.bias = module.bias
        self.bver = None if module.bias is None else module.bias._version
        self.desc = desc
        self.desc_addr = ctypes.addressof(desc)
        self.wt, self.wt_ptr = wt, wt.data_ptr()
        self.b32, self.b_ptr = b32, (None if b32 is None else b32.data_ptr())
        self.ws, self.ws_ptr, self.ws_bytes = ws, ws.data_ptr(), ws.numel() * ws.element_size()
        self.fn = _lib.lib().sf_conv2d_forward

    def run(self, module, x):
        params = module._parameters  # plain dict reads: nn.Module attribute lookups are slow
        if (x.shape != self.shape or x.dtype != self.dtype or x.get_device() != self.index
                or not x.is_contiguous() or params["weight"] is not self.weight or self.weight._version != self.wver
                or params["bias"] is not self.bias or (self.bias is not None and self.bias._version != self.bver)
                or module.threshold != self.threshold or spike_map.recorded(x)):
            return None
        y = torch.empty(self.out_shape, dtype=self.dtype, device=self.device)
        rc = self.fn(self.desc_addr, x.data_ptr(), self.wt_ptr, self.b_ptr, self.threshold, self.ws_ptr,
                     self.ws_bytes, y.data_ptr(), _lib.raw_stream(self.index))
        if rc != _lib.SF_OK:
            _lib._check(rc, "sf_conv2d_forward")
        return y


class SparseConv2d(OpReporting, nn.Module):
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

        self._w_tap = WeightLayout(_lib.tap_major_weight)
        self._workspace = None
        self._plan = None  # _InferencePlan of the last eligible input shape
        self._plan_candidate = False
        self._last_dense_ms = 0.0
        # Runtime fallback policy (dense above an averaged active ratio, the
        # bias-only output after a run of all-zero inputs; sticky zero as in
        # Ops/sparse_conv2d.py:449-496).  Off unless enabled in Utils.config
        # or per module through `runtime_policy`.
        self.policy = FallbackPolicy(_config.ENABLE_RUNTIME_FALLBACK_POLICY, warmup_steps, calib_every, ema_decay,
                                     dense_threshold, zero_streak_needed, zero_sticky=True)
        self._audit = DispatchAudit()
        self._profile = PathProfile("SparseConv2d")
        self._profile.enabled = bool(profile_runtime)
        self._init_reporting("sparse_kernel", "conv2d_two_stage_hip", "conv")
        # "sparse" (library kernels) or "dense" (F.conv2d), set per layer by
        # Utils.dispatch from measurements.
        self.backend_mode = "sparse"

    # ---- runtime switches (Ops/sparse_conv2d.py:234-250) --------------------
    def set_launch_all_tiles(self, enabled: bool):
        """Kept for API compatibility: the HIP path always launches every
        tile group and skips zero work on the device."""
        self.launch_all_tiles = bool(enabled)

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

    def get_profile_summary(self):
        return self._profile.summary()

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
        changes."""
        return self._w_tap(self.weight)

    def _get_workspace(self, x4d):
        n, c, h, w = (int(v) for v in x4d.shape)
        need = _lib.conv2d_workspace_size(_lib.conv_desc(n, c, h, w, self.out_channels, 1, 1, 1, 1, 0, 0, 0))
        ws = self._workspace
        if ws is None or ws.device != x4d.device or ws.numel() < need:
            ws = torch.empty(max(need, 256), dtype=torch.uint8, device=x4d.device)
            self._workspace = ws
        return ws

    def _zero_output(self, x):
        """Bias-only output for x (4-D or 5-D): the exact result of an
        all-zero input."""
        h_out, w_out = self._output_hw(int(x.shape[-2]), int(x.shape[-1]))
        return bias_rows(self.bias, tuple(x.shape[:-3]), self.out_channels, (h_out, w_out), x.dtype, x.device)

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

    # ---- forward ----------------------------------------------------------------
    def _plan_allowed(self) -> bool:
        """Module switches under which a forward is the plain one-call
        library path (no diagnostics, timing, profiling or policy override)."""
        return (self._inference_mode and self.backend_mode == "sparse" and not self.collect_diag
                and not self.return_ms and not self._profile.enabled and self.policy.forced is None)

    def forward(self, x: torch.Tensor):
        plan = self._plan
        if plan is not None and self._plan_allowed():
            y = plan.run(self, x)
            if y is not None:
                # The bookkeeping of a full forward that took the sparse path
                # (assignments skipped when they change nothing: nn.Module's
                # attribute writes are slow).
                if self.fallback_reason:
                    self.fallback_reason = ""
                if self._last_sparse_ms or self._last_dense_ms:
                    self._last_sparse_ms = self._last_dense_ms = 0.0
                self.policy.forwards += 1
                self._audit.record(self, "sparse")
                return y
        return self._forward_full(x)

    def _forward_full(self, x: torch.Tensor):
        if x.dim() not in (4, 5):
            raise ValueError(f"Expected 4D or 5D input, got {x.dim()}D")
        t0 = self._profile.start(x.device)
        self.fallback_reason = ""
        self._plan = None
        self._plan_candidate = False
        forced = self.policy.forced
        if forced == FallbackPolicy.ZERO:
            y = self._zero_output(x)
            self._last_sparse_ms = 0.0
            self.fallback_reason = "force_zero"
            self._audit.record(self, "staticzero")
            self._profile.finish("zero(force)", self._profile.elapsed(t0, x.device), self.policy.last_ratio)
            return y
        x4d = x.reshape(-1, *x.shape[-3:]) if x.dim() == 5 else x
        ratio = None
        if x4d.is_cuda and self._supports_sparse() and self.backend_mode != "dense" and forced is None:
            y4d, backend, ratio = self._hip_forward(x4d, self.policy.wants_ratio(self._inference_mode))
            path = {"dense_fallback": "dense(fallback)", "zero_tiles_only": "zero(tile_compaction)"}.get(
                backend, "sparse")
            self._audit.record(self, {"dense_fallback": "dense", "zero_tiles_only": "staticzero"}.get(
                backend, "sparse"))
        else:
            y4d = self._fallback_forward(x4d)
            path = "dense"
            self.fallback_reason = ("force_dense" if forced == FallbackPolicy.DENSE else
                                    "dispatch_dense" if self.backend_mode == "dense" else "module_dense_path")
            self._audit.record(self, "dense")
        self.policy.forwards += 1
        self.policy.observe(ratio)
        if ratio == 0.0 and self.policy.forced == FallbackPolicy.ZERO:
            # This forward's input was already all-zero, so its output is the
            # bias-only output the zero path would give.
            path, self.fallback_reason = "zero(promoted)", "zero_promoted"
        y = y4d.reshape(*x.shape[:2], *y4d.shape[1:]) if x.dim() == 5 else y4d
        self._profile.finish(path, self._profile.elapsed(t0, x.device), self.policy.last_ratio)
        if self._plan_candidate and path == "sparse" and self._plan_allowed():
            self._plan = self._make_plan(x, x4d)
        if self.collect_diag:
            self._last_diag.update(runtime_dispatch_seen=self._audit.seen,
                                   runtime_dispatch_mismatch=self._audit.mismatch,
                                   fallback_reason=str(self.fallback_reason))
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
        # The one-call path ran (sf_conv2d_forward): later forwards of this
        # shape may repeat it directly.
        self._plan_candidate = meta.get("reason") == "bitmap_gather" and not (want_diag or need_ratio)
        if backend == "dense_fallback":
            self._last_sparse_ms, self._last_dense_ms = 0.0, float(ms)
        else:
            self._last_sparse_ms, self._last_dense_ms = float(ms), 0.0
        self._profile.add("sparse_kernel", self._last_sparse_ms)
        if want_diag:
            self._collect_diag(x4d, ms, ratio, stats, meta)
        return y, backend, ratio

    def _make_plan(self, x, x4d):
        n, c, h, w = (int(v) for v in x4d.shape)
        k, s, p = self.kernel_size[0], self.stride[0], self.padding[0]
        h_out, w_out = self._output_hw(h, w)
        code = _lib.dtype_code(x4d.dtype)
        desc = _lib.conv_desc(n, c, h, w, self.out_channels, h_out, w_out, k, s, p, code, code)
        b32 = None if self.bias is None else self.bias.detach().to(torch.float32).contiguous()
        return _InferencePlan(self, x, desc, self._get_w_tap(), b32, self._get_workspace(x4d))

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
        t0 = self._profile.start(x.device)
        y = F.conv2d(x, self.weight, self.bias, self.stride, self.padding, self.dilation, self.groups)
        self._last_sparse_ms = 0.0
        self._last_dense_ms = self._profile.elapsed(t0, x.device)
        self._profile.add("dense_fallback", self._last_dense_ms)
        return y

    def extra_repr(self):
        bs = self.block_size if self.block_size is not None else "auto"
        return (
            f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
            f"stride={self.stride}, padding={self.padding}, block_size={bs}, "
            f"return_ms={self.return_ms}, sparse=True, backend=hip_two_stage, "
            f"allow_sparse_1x1={self.allow_sparse_1x1}, inference_mode={self._inference_mode}"
        )
