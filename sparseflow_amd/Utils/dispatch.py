"""Per-layer dispatch: sparse, dense or static-zero (drop-in for the
reference's execution-grounded dispatch, Utils/dispatch_model.py:814-1194,
and the exact-zero backend choice, Ops/static_zero_conv2d.py:31-205).

The reference scores each layer from calibration diagnostics (redundancy
R = tile-zero ratio + active-group ratio, work per tile I, S = R * I against
a per-family tau measured on its own GPU) because timing every layer both
ways is what the score approximates.  Here the decision is grounded in the
execution itself on the MI355X: a calibration forward measures each
candidate layer's input (exact zero, spike density, tile-zero and
active-group ratios from the prescan metadata) and times the layer on that
input with the library's sparse path and with F.conv2d (MIOpen); the faster
one wins, with the reference's gates kept around it (unsupported op,
missing measurements -> dense; exact-zero input -> static-zero when allowed).

    decisions = dispatch_model(model, sample_input)       # measure + decide
    static_zero, sparse = decisions_to_sets(decisions)
    apply_decisions(model, decisions)                     # set each layer's path
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field
from typing import Dict, Iterable, Optional, Set, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

# A sparse win must beat the dense time by this factor (hysteresis against
# timing noise on near-ties); the reference's tau margin plays this role.
SPARSE_MARGIN = 0.95
# Without timings: sparse below this spike density (fraction of non-zero
# input elements), dense above.
DENSITY_GATE = 0.2


@dataclass
class DispatchDecision:
    layer_name: str
    backend: str = "dense"             # "sparse" | "dense" | "staticzero"
    reason_code: str = ""
    reason: str = ""
    fallback_reason: str = ""
    confidence: float = 0.0
    op_type: str = "conv"
    density: float = -1.0              # fraction of non-zero input elements
    tzr: float = -1.0                  # zero-tile ratio (prescan metadata)
    agr: float = -1.0                  # active-group ratio (prescan metadata)
    sparse_ms: float = -1.0
    dense_ms: float = -1.0
    support_status: str = "supported"
    diag_source: str = "measured"
    extra: dict = field(default_factory=dict)

    def as_dict(self) -> dict:
        return asdict(self)


def make_dispatch_decision(name: str, diag: Dict, allow_static_zero: bool = True) -> DispatchDecision:
    """One layer's decision from its calibration diagnostics (keys: supported,
    exact_zero, density, tzr, agr, sparse_ms, dense_ms)."""
    d = DispatchDecision(layer_name=name, op_type=str(diag.get("op_type", "conv")))
    d.density = float(diag.get("density", -1.0))
    d.tzr = float(diag.get("tzr", -1.0))
    d.agr = float(diag.get("agr", -1.0))
    d.sparse_ms = float(diag.get("sparse_ms", -1.0))
    d.dense_ms = float(diag.get("dense_ms", -1.0))
    if not diag.get("supported", True):
        d.backend, d.reason_code, d.support_status, d.confidence = "dense", "unsupported_op", "unsupported", 1.0
        d.reason = d.fallback_reason = "unsupported_op_fallback_dense"
        return d
    if diag.get("exact_zero", False) and allow_static_zero:
        d.backend, d.reason_code, d.confidence = "staticzero", "exact_zero_input", 1.0
        d.reason = "all calibration inputs exactly zero"
        return d
    if d.sparse_ms > 0.0 and d.dense_ms > 0.0:
        d.confidence = 1.0
        if d.sparse_ms <= SPARSE_MARGIN * d.dense_ms:
            d.backend, d.reason_code = "sparse", "timed_faster"
            d.reason = f"sparse {d.sparse_ms:.3f} ms <= {SPARSE_MARGIN} x dense {d.dense_ms:.3f} ms"
        else:
            d.backend, d.reason_code = "dense", "timed_slower"
            d.reason = d.fallback_reason = f"sparse {d.sparse_ms:.3f} ms > {SPARSE_MARGIN} x dense {d.dense_ms:.3f} ms"
        return d
    if d.density >= 0.0:
        d.confidence = 0.5
        d.diag_source = "density_only"
        if d.density < DENSITY_GATE:
            d.backend, d.reason_code = "sparse", "density_gate"
            d.reason = f"density {d.density:.4f} < {DENSITY_GATE}"
        else:
            d.backend, d.reason_code = "dense", "density_gate"
            d.reason = d.fallback_reason = f"density {d.density:.4f} >= {DENSITY_GATE}"
        return d
    d.backend, d.reason_code, d.confidence, d.diag_source = "dense", "missing_diag", 0.2, "missing"
    d.reason = d.fallback_reason = "missing_diag_fallback_dense"
    return d


def _target_field(t, key: str, default=None):
    if isinstance(t, dict):
        return t.get(key, default)
    return getattr(t, key, default)


def _target_layer_name(t) -> str:
    """Layer name of a target: a name string, a ReplacementTarget or an
    analyzer dict (keys "name" / "conv_name" / "layer_name")."""
    if isinstance(t, str):
        return t
    for key in ("conv_name", "name", "layer_name"):
        v = _target_field(t, key)
        if v:
            return str(v)
    return ""


_POOL_OPS = ("maxpool2d", "avgpool2d")


def dispatch_all_layers(targets: Iterable, diags: Dict[str, Dict], zero_layers: Optional[Set[str]] = None,
                        allow_static_zero: bool = True) -> Dict[str, DispatchDecision]:
    """Decisions for every target layer (reference: dispatch_all_layers,
    Utils/dispatch_model.py:1141).  Targets are names, ReplacementTargets or
    analyzer dicts; pool targets stay dense; layers in `zero_layers` are
    static-zero regardless of measurements."""
    zero_layers = set(zero_layers or ())
    out: Dict[str, DispatchDecision] = {}
    for t in targets:
        name = _target_layer_name(t)
        if not name:
            continue
        op_type = "" if isinstance(t, str) else str(_target_field(t, "op_type", ""))
        if op_type in _POOL_OPS:
            out[name] = DispatchDecision(layer_name=name, backend="dense", reason_code="pool_dense_keep",
                                         reason="pool replacement disabled", op_type=op_type, confidence=1.0)
        elif name in zero_layers:
            out[name] = make_dispatch_decision(name, {"exact_zero": True}, allow_static_zero=True)
        else:
            out[name] = make_dispatch_decision(name, diags.get(name, {}), allow_static_zero)
    return out


def decisions_to_sets(decisions: Dict[str, DispatchDecision]) -> Tuple[Set[str], Set[str]]:
    """(static_zero_set, sparse_set) (reference: decisions_to_sets)."""
    zero = {n for n, d in decisions.items() if d.backend == "staticzero"}
    sparse = {n for n, d in decisions.items() if d.backend == "sparse"}
    return zero, sparse


def _time_ms(fn, repeats: int) -> float:
    fn()  # warm (algorithm selection, workspace growth)
    ts = []
    for _ in range(repeats):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    ts.sort()
    return ts[len(ts) // 2]


def measure_layers(model: nn.Module, sample_input, repeats: int = 3, time_layers: bool = True) -> Dict[str, Dict]:
    """Calibration forward: per SparseConv2d layer, the diagnostics of its
    input and (on the GPU) the time of one call each way on that input."""
    from ..Kernels.conv2d import sparse_conv2d_forward
    from ..Ops.sparse_conv2d import SparseConv2d
    from ..neuron import reset_net

    diags: Dict[str, Dict] = {}
    hooks = []

    def pre_hook(mod, inp, name):
        x = inp[0]
        x4 = x.reshape(-1, *x.shape[-3:]) if x.dim() == 5 else x
        nz = int(torch.count_nonzero(x4))
        d = diags.setdefault(name, {"supported": mod._supports_sparse(), "exact_zero": True, "density": 0.0})
        d["exact_zero"] = d["exact_zero"] and nz == 0
        d["density"] = max(d["density"], nz / max(1, x4.numel()))
        if not (x4.is_cuda and d["supported"]):
            return
        k, s, p = mod.kernel_size[0], mod.stride[0], mod.padding[0]
        res = sparse_conv2d_forward(x4, mod.weight, mod.bias, kernel_size=k, stride=s, padding=p,
                                    threshold=mod.threshold, return_avg_active_ratio=True, return_tile_stats=True)
        st = res[3] if len(res) > 3 else None
        if isinstance(st, dict) and st.get("total_tiles"):
            d["tzr"] = st["zero_tiles"] / st["total_tiles"]
            d["agr"] = float(res[2]) if res[2] is not None else -1.0
        if time_layers:
            x4c = x4.contiguous()
            wt = mod._get_w_tap()
            d["sparse_ms"] = _time_ms(lambda: sparse_conv2d_forward(
                x4c, mod.weight, mod.bias, kernel_size=k, stride=s, padding=p, threshold=mod.threshold, w_cl=wt),
                repeats)
            w32 = mod.weight.to(x4c.dtype)
            b32 = None if mod.bias is None else mod.bias.to(x4c.dtype)
            d["dense_ms"] = _time_ms(lambda: F.conv2d(x4c, w32, b32, s, p), repeats)

    for name, mod in model.named_modules():
        if isinstance(mod, SparseConv2d):
            hooks.append(mod.register_forward_pre_hook(lambda m, i, n=name: pre_hook(m, i, n)))
    try:
        reset_net(model)
        with torch.no_grad():
            model(sample_input)
    finally:
        for h in hooks:
            h.remove()
        reset_net(model)
    return diags


def _stamp(mod: nn.Module, d: DispatchDecision) -> None:
    """The observability attributes the replacer stamps (Core/replacer.py
    _attach_observability), updated to the decision."""
    mod.sf_backend_mode = d.backend
    mod.sf_dispatch_decision = d.backend
    mod.sf_backend_family = "exact_zero" if d.backend == "staticzero" else (
        "sparse_kernel" if d.backend == "sparse" else "dense_library")
    mod.sf_reason_code = d.reason_code
    mod.sf_fallback_reason = d.fallback_reason
    mod.sf_diag_source = d.diag_source
    mod.sf_support_status = d.support_status
    mod.sf_dispatch = d.as_dict()


def apply_decisions(model: nn.Module, decisions: Dict[str, DispatchDecision], verbose: bool = False) -> Dict[str, int]:
    """Set each SparseConv2d's path (sparse / dense) or replace it with
    StaticZeroConv2d; returns counts per backend."""
    from ..Core.replacer import _set_module_by_name
    from ..Ops.sparse_conv2d import SparseConv2d
    from ..Ops.static_zero_conv2d import StaticZeroConv2d

    counts = {"sparse": 0, "dense": 0, "staticzero": 0}
    modules = dict(model.named_modules())
    for name, d in decisions.items():
        mod = modules.get(name)
        if not isinstance(mod, SparseConv2d):
            continue
        if d.backend == "staticzero":
            new = StaticZeroConv2d.from_conv(mod, zero_reason=d.reason_code)
            for k, v in vars(mod).items():
                if k.startswith("sf_"):
                    setattr(new, k, v)
            _set_module_by_name(model, name, new)
            mod = new
        else:
            mod.backend_mode = d.backend
        _stamp(mod, d)
        counts[d.backend] += 1
        if verbose:
            print(f"  [{d.backend.upper():10s}] {name}: {d.reason}")
    return counts


def dispatch_model(model: nn.Module, sample_input, allow_static_zero: bool = False, repeats: int = 3,
                   apply: bool = True, verbose: bool = False) -> Dict[str, DispatchDecision]:
    """Measure every SparseConv2d of an optimized model on `sample_input`,
    decide its backend and (by default) apply the decisions.  Static-zero
    replacement is off by default: it is exact only while the layer's input
    stays zero, which one calibration batch cannot prove."""
    from ..Ops.sparse_conv2d import SparseConv2d

    diags = measure_layers(model, sample_input, repeats=repeats)
    names = [n for n, m in model.named_modules() if isinstance(m, SparseConv2d)]
    decisions = dispatch_all_layers(names, diags, allow_static_zero=allow_static_zero)
    if apply:
        apply_decisions(model, decisions, verbose=verbose)
    return decisions
