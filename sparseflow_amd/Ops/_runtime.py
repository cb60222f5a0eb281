"""Per-module runtime state shared by the operator modules.

Three small pieces, one per concern:

* `FallbackPolicy` - the optional runtime switch between the sparse kernels,
  dense torch and the bias-only output, driven by the active ratios the
  module observes.  Behaviour follows the reference modules' runtime policy
  (Ops/sparse_conv2d.py:449-496, Ops/sparse_linear.py:357-410): the first
  `warmup` observed ratios seed the estimate, later ones are sampled every
  `period` forwards into an exponential average; an average above
  `dense_above` selects dense, `zero_after` consecutive all-zero inputs
  select the bias-only output.  The conv module's zero choice is sticky, the
  Linear module's is cleared by the next non-zero input, as in the two
  reference modules.  Off unless enabled (Utils/config.py:43).
* `PathProfile` - host wall-clock accounting of which path each forward took
  (`profile_runtime`); it synchronises the device around each measured span
  and is therefore never on for timed runs.
* `WeightLayout` - a derived weight layout (tap-major fp32, transposed,
  bf16 split) rebuilt only when the parameter changes, keyed on its version
  counter, storage and device (the reference keys its fp16 copy on
  `weight._version`, Ops/sparse_conv2d.py:339-350).

Two more are shared by every replaced operator module:

* `OpReporting` - the observability attributes a replaced module exposes
  (their names and defaults are the drop-in contract the reference's
  harness and replacer read) and `set_inference_mode`, set up in one call.
* `ExactZeroOp` + `bias_rows` - the exact-zero backends: an operator whose
  input is all zero returns its bias broadcast over the output (zeros
  without a bias); SparseConv2d's zero path, StaticZeroConv2d and
  StaticZeroLinear all build that tensor with `bias_rows`.
"""

from __future__ import annotations

import time
from collections import Counter
from typing import Callable, Optional

import torch


class FallbackPolicy:
    SPARSE, DENSE, ZERO = "sparse", "dense", "zero"

    def __init__(self, enabled: bool, warmup: int = 8, period: int = 32, decay: float = 0.9,
                 dense_above: float = 0.85, zero_after: int = 2, zero_sticky: bool = True):
        self.enabled = bool(enabled)
        self.warmup_left = max(0, int(warmup))
        self.period = max(1, int(period))
        self.decay = float(decay)
        self.dense_above = float(dense_above)
        self.zero_after = max(1, int(zero_after))
        self.zero_sticky = bool(zero_sticky)
        self.average: Optional[float] = None
        self.zero_run = 0
        self.choice = self.SPARSE
        self.forwards = 0
        self.last_ratio = -1.0

    def wants_ratio(self, inference: bool) -> bool:
        """Whether this forward should measure its input's active ratio."""
        if not self.enabled or inference:
            return False
        return self.warmup_left > 0 or self.forwards % self.period == 0

    def observe(self, ratio: Optional[float]) -> None:
        """Fold one measured active ratio (None: nothing was measured)."""
        if ratio is None:
            return
        r = float(ratio)
        self.last_ratio = r
        if not self.enabled:
            return
        if self.warmup_left > 0:
            self.warmup_left -= 1
            self.average = r
            return
        self.average = r if self.average is None else self.decay * self.average + (1.0 - self.decay) * r
        self.zero_run = self.zero_run + 1 if r == 0.0 else 0
        zero = self.zero_run >= self.zero_after or (self.zero_sticky and self.choice == self.ZERO)
        if zero:
            self.choice = self.ZERO
        else:
            self.choice = self.DENSE if self.average > self.dense_above else self.SPARSE

    @property
    def forced(self) -> Optional[str]:
        """'dense' or 'zero' when the policy overrides the sparse path."""
        if not self.enabled or self.choice == self.SPARSE:
            return None
        return self.choice


class PathProfile:
    """Counts and host wall-clock milliseconds per path taken."""

    def __init__(self, label: str):
        self.label = label
        self.enabled = False
        self.calls = 0
        self.hits: Counter = Counter()
        self.ms: Counter = Counter()
        self.last_path = "none"
        self.last_ms = 0.0
        self.last_ratio = -1.0

    @staticmethod
    def _sync(device) -> None:
        if device is not None and device.type == "cuda":
            torch.cuda.synchronize(device)

    def start(self, device) -> float:
        if not self.enabled:
            return 0.0
        self._sync(device)
        return time.perf_counter()

    def elapsed(self, t0: float, device) -> float:
        if not self.enabled:
            return 0.0
        self._sync(device)
        return (time.perf_counter() - t0) * 1e3

    def add(self, bucket: str, ms: float) -> None:
        if self.enabled:
            self.ms[bucket] += float(ms)

    def finish(self, path: str, ms: float, ratio: float = -1.0) -> None:
        if not self.enabled:
            return
        self.calls += 1
        self.hits[path.split("(")[0]] += 1
        self.ms["total"] += float(ms)
        self.last_path, self.last_ms, self.last_ratio = path, float(ms), float(ratio)

    def summary(self) -> str:
        if self.calls == 0:
            return f"{self.label} runtime profile: no calls"
        mean = {k: v / self.calls for k, v in self.ms.items()}
        hits = ", ".join(f"{k}={self.hits.get(k, 0)}" for k in ("zero", "sparse", "dense"))
        buckets = ", ".join(f"{k}={v:.3f}" for k, v in sorted(mean.items()))
        return (f"{self.label} runtime profile\n"
                f"  calls={self.calls}, last_path={self.last_path}\n"
                f"  hits: {hits}\n"
                f"  mean ms: {buckets}\n"
                f"  last: total={self.last_ms:.3f} ms, active_ratio={self.last_ratio:.4f}")


class WeightLayout:
    """`layout(param)` recomputed only when `param` changes."""

    def __init__(self, build: Callable[[torch.Tensor], object]):
        self._build = build
        self._key = None
        self._value = None

    def __call__(self, param: torch.Tensor):
        key = (param._version, param.data_ptr(), param.device)
        if self._value is None or key != self._key:
            self._value = self._build(param)
            self._key = key
        return self._value


class DispatchAudit:
    """Counts forwards whose path differs from the per-layer dispatch
    decision stamped on the module (`sf_dispatch_decision`)."""

    def __init__(self):
        self.seen = 0
        self.mismatch = 0

    def record(self, module, path: str) -> None:
        # The decision stamps are plain attributes: read them from the
        # instance dict (a missed nn.Module attribute lookup is slow).
        d = vars(module)
        expected = d.get("sf_dispatch_decision", d.get("sf_backend_mode", ""))
        if not expected:
            return
        expected = str(expected).strip().lower()
        if not expected:
            return
        self.seen += 1
        if expected != path:
            self.mismatch += 1


def bias_rows(bias: Optional[torch.Tensor], lead, channels: int, trailing, dtype, device) -> torch.Tensor:
    """A fresh tensor of shape (*lead, channels, *trailing) holding bias[c]
    at every position (zeros without a bias): the exact output of a conv or
    Linear whose input is all zero."""
    shape = (*lead, channels, *trailing)
    if bias is None:
        return torch.zeros(shape, dtype=dtype, device=device)
    b = bias.detach().to(device=device, dtype=dtype).reshape(channels, *([1] * len(trailing)))
    return b.expand(shape).clone()


class OpReporting:
    """Mixin for nn.Module operators: the reporting state a replaced module
    carries.  Attribute names and their defaults follow the reference
    modules' observability contract (Ops/sparse_conv2d.py:191-250,
    Ops/sparse_attention.py, Ops/sparse_bmm.py, Ops/sparse_fused_conv_lif.py);
    the values are this build's.  `_init_reporting` is called once from the
    module's constructor, after any `profile_runtime` property's backing
    state exists."""

    def _init_reporting(self, backend_family: str, diag_path: str, score_family: Optional[str] = None,
                        profile_runtime: Optional[bool] = None) -> None:
        self._last_sparse_ms = 0.0
        self._last_diag = {}
        self.collect_diag = False
        self._inference_mode = False
        self.backend_family = backend_family
        self.diag_path = diag_path
        self.fallback_reason = ""
        self.meta_source = self.diag_source = "measured"
        self.support_status = "supported"
        if score_family is not None:
            self.score_family = score_family
        if profile_runtime is not None:
            self.profile_runtime = bool(profile_runtime)

    def set_inference_mode(self, enabled: bool) -> None:
        """Inference mode turns diagnostics and host-timed profiling off, so
        a forward never waits on the device."""
        self._inference_mode = bool(enabled)
        if enabled:
            self.collect_diag = False
            self.profile_runtime = False


class ExactZeroOp:
    """Mixin for the exact-zero backends (StaticZeroConv2d,
    StaticZeroLinear): the bias kept as an fp32 buffer, a call counter and
    the diagnostics record.  Such a module never reads its input's values,
    only its shape."""

    backend_family = "exact_zero"

    def _init_exact_zero(self, bias: Optional[torch.Tensor], zero_reason: str, diag_path: str) -> None:
        self.register_buffer("bias_buf", None if bias is None else bias.detach().float().clone())
        self.zero_reason = zero_reason
        self.diag_path = diag_path
        self.fallback_reason = "exact_zero_shortcut"
        self.calls = 0
        self.collect_diag = False
        self.profile_runtime = False
        self._last_diag = {}
        self._last_sparse_ms = 0.0

    def _zero_output(self, lead, channels: int, trailing, like: torch.Tensor) -> torch.Tensor:
        self.calls += 1
        y = bias_rows(self.bias_buf, lead, channels, trailing, like.dtype, like.device)
        if self.collect_diag:
            self._last_diag = self.get_diag()
        return y

    def _zero_diag(self, **shape_keys) -> dict:
        return dict(backend_family=self.backend_family, zero_reason=self.zero_reason, diag_path=self.diag_path,
                    fallback_reason=self.fallback_reason, has_bias=self.bias_buf is not None,
                    forward_count=self.calls, sparse_path_executed=False, sparse_total_ms=0.0, **shape_keys)
