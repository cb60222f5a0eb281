"""Replacement-target discovery (drop-in for Core/analyzer.py).

Finds Conv2d layers fed by spike sources, with the reference's three
discovery modes tried in order (Core/analyzer.py:233-280):

  1. torch.fx graph: breadth-first search from every spike-source node to
     the next conv consumer, not crossing another spike source
     (Core/analyzer.py:347-418).  Spike sources are traced as leaf modules,
     so stateful neurons do not break the trace.
  2. Runtime order: forward hooks under a sample input pair each conv with
     the most recent spike event (Core/analyzer.py:424-500).
  3. Module order: a window of 15 modules after each spike source, skipping
     transparent layers (Core/analyzer.py:506-549).

Targets (Core/analyzer.py:575-700): Conv2d with groups == 1 and one of
3x3/s1/p1, 3x3/s2/p1, 1x1/s1/p0 (feature maps the block rule rejects,
input H < 8, Utils/block_selector.py, are skipped; the chosen block size is
recorded on the target); nn.Linear (op "linear"); and attention blocks --
modules carrying Linear q/k/v/proj and an attn_lif, traced as leaves --
with the variant inferred as the reference does (Core/analyzer.py:121-147).
Conv1d/Conv3d consumers end a search branch but are not targets here.
"""

from __future__ import annotations

import warnings
from dataclasses import dataclass
from typing import Dict, List, Optional, Set, Tuple

import torch
import torch.nn as nn

from ..Utils.block_selector import select_block_size, should_replace
from .registry import SpikeOpRegistry


@dataclass
class ReplacementTarget:
    """One replaceable module.  `conv_name` / `conv_module` keep the
    reference's field names (Core/analyzer.py:52-73)."""

    conv_name: str
    conv_module: nn.Module
    spike_name: str
    op_type: str
    block_size: Optional[int] = None
    input_h: int = 0
    input_w: int = 0
    input_d: int = 0
    extra: Optional[dict] = None


_TRANSPARENT_MODULES = (
    nn.Dropout, nn.Dropout2d, nn.Dropout3d, nn.Identity, nn.Flatten,
    nn.AdaptiveAvgPool1d, nn.AdaptiveAvgPool2d, nn.AdaptiveAvgPool3d,
    nn.AdaptiveMaxPool1d, nn.AdaptiveMaxPool2d, nn.AdaptiveMaxPool3d,
    nn.AvgPool1d, nn.AvgPool2d, nn.AvgPool3d, nn.MaxPool1d, nn.MaxPool2d, nn.MaxPool3d,
    nn.BatchNorm1d, nn.BatchNorm2d, nn.BatchNorm3d,
    nn.ReLU, nn.ReLU6, nn.LeakyReLU, nn.GELU, nn.SiLU, nn.Sequential,
)

CONV2D_OP_TYPES = ("conv2d_3x3", "conv2d_3x3_s2", "conv2d_1x1")


def _as_pair(x) -> Tuple[int, int]:
    if isinstance(x, (tuple, list)):
        return (int(x[0]), int(x[0])) if len(x) == 1 else (int(x[0]), int(x[1]))
    return int(x), int(x)


def conv2d_op_type(conv: nn.Conv2d) -> Optional[str]:
    """Sparse op type of a Conv2d, or None when the kernels do not apply."""
    if not isinstance(conv, nn.Conv2d) or int(conv.groups) != 1:
        return None
    if _as_pair(conv.dilation) != (1, 1):
        return None
    k, s, p = _as_pair(conv.kernel_size), _as_pair(conv.stride), _as_pair(conv.padding)
    if k == (3, 3) and s == (1, 1) and p == (1, 1):
        return "conv2d_3x3"
    if k == (3, 3) and s == (2, 2) and p == (1, 1):
        return "conv2d_3x3_s2"
    if k == (1, 1) and s == (1, 1) and p == (0, 0):
        return "conv2d_1x1"
    return None


def display_block_info(target: ReplacementTarget) -> str:
    if target.op_type in CONV2D_OP_TYPES:
        h = target.input_h
        bs = target.block_size if target.block_size is not None else "auto"
        return f"H={h if h > 0 else '?'} block={bs}"
    return ""


def is_attention_like_module(module: nn.Module) -> bool:
    """An attention block carries Linear q/k/v/proj and an attn_lif
    (Core/analyzer.py:121-131)."""
    if module is None:
        return False
    for attr in ("q", "k", "v", "proj"):
        if not isinstance(getattr(module, attr, None), nn.Linear):
            return False
    return hasattr(module, "attn_lif")


def infer_attention_variant(module: nn.Module) -> str:
    """Core/analyzer.py:139-145: class name with "qkmix" -> qkmix; a `scale`
    attribute -> q @ k^T @ v; else the linear-attention form."""
    if "qkmix" in module.__class__.__name__.lower():
        return "attention_qkmix"
    if hasattr(module, "scale"):
        return "attention_qkav"
    return "attention_linear"


ATTENTION_OP_TYPES = ("attention_qkav", "attention_linear", "attention_qkmix")


class _SpikeLeafTracer(torch.fx.Tracer):
    def __init__(self, registry: SpikeOpRegistry):
        super().__init__()
        self._registry = registry

    def is_leaf_module(self, m: nn.Module, qualname: str) -> bool:
        if self._registry.is_spike_op(m) or is_attention_like_module(m):
            return True
        if isinstance(m, nn.MaxPool2d):  # incl. Ops.spike_pool.SpikeMaxPool2d (data-dependent forward)
            return True
        return super().is_leaf_module(m, qualname)


class NetworkAnalyzer:
    FALLBACK_SEARCH_WINDOW = 15
    MAX_BFS_DEPTH = 20

    def __init__(self, registry: SpikeOpRegistry):
        self.registry = registry

    def analyze(self, model: nn.Module, sample_input: Optional[torch.Tensor] = None) -> List[ReplacementTarget]:
        input_shapes = self._infer_input_shapes(model, sample_input) if sample_input is not None else {}
        fx_error = None
        try:
            targets = self._analyze_fx(model, input_shapes)
            if targets:
                return self._dedup(targets)
        except Exception as err:  # tracing arbitrary user models may fail in many ways
            fx_error = err
            warnings.warn(f"[SparseFlow] torch.fx trace failed: {err}; falling back to runtime-order scan.")
        if sample_input is not None:
            try:
                targets = self._analyze_runtime_fallback(model, input_shapes, sample_input)
                if targets:
                    return self._dedup(targets)
            except Exception as err:
                warnings.warn(f"[SparseFlow] runtime-order scan failed: {err}; falling back to module order.")
        elif fx_error is None:
            warnings.warn("[SparseFlow] torch.fx found no targets and no sample input was given; "
                          "falling back to module-order scan.")
        return self._dedup(self._analyze_fallback(model, input_shapes))

    @staticmethod
    def _dedup(targets: List[ReplacementTarget]) -> List[ReplacementTarget]:
        seen: Set[str] = set()
        out = []
        for t in targets:
            if t.conv_name not in seen:
                seen.add(t.conv_name)
                out.append(t)
        return out

    # ---- mode 1: torch.fx -------------------------------------------------
    def _analyze_fx(self, model: nn.Module, input_shapes: dict) -> List[ReplacementTarget]:
        tracer = _SpikeLeafTracer(self.registry)
        graph = tracer.trace(model)
        modules = dict(model.named_modules())
        targets: List[ReplacementTarget] = []
        visited: Set[str] = set()
        for node in graph.nodes:
            if node.op != "call_module" or not self.registry.is_spike_op(modules.get(node.target)):
                continue
            for name in self._bfs_find_targets(node, modules, visited):
                t = self._make_target(name, modules[name], node.target, input_shapes)
                if t is not None:
                    targets.append(t)
                    visited.add(name)
        return targets

    def _bfs_find_targets(self, spike_node, modules: dict, visited: Set[str]) -> List[str]:
        found = []
        queue = [(u, 0) for u in spike_node.users]
        seen = set()
        while queue:
            node, depth = queue.pop(0)
            if depth > self.MAX_BFS_DEPTH or id(node) in seen:
                continue
            seen.add(id(node))
            mod = modules.get(node.target) if node.op == "call_module" else None
            if mod is not None:
                if isinstance(mod, (nn.Conv1d, nn.Conv2d, nn.Conv3d, nn.Linear)) or is_attention_like_module(mod):
                    if not isinstance(mod, (nn.Conv1d, nn.Conv3d)) and node.target not in visited:
                        found.append(node.target)
                    continue  # a consumer ends this branch
                if self.registry.is_spike_op(mod):
                    continue  # never cross another spike source
            queue.extend((u, depth + 1) for u in node.users)
        return found

    # ---- mode 2: runtime order --------------------------------------------
    def _analyze_runtime_fallback(self, model, input_shapes, sample_input) -> List[ReplacementTarget]:
        modules = dict(model.named_modules())
        events = []
        hooks = []
        for name, m in model.named_modules():
            if self.registry.is_spike_op(m):
                hooks.append(m.register_forward_hook(lambda _m, _i, _o, n=name: events.append(("spike", n))))
            elif isinstance(m, (nn.Conv2d, nn.Linear)) or is_attention_like_module(m):
                hooks.append(m.register_forward_hook(lambda _m, _i, _o, n=name: events.append(("target", n))))
        try:
            _reset_states(model)
            with torch.no_grad():
                model(sample_input)
        finally:
            for h in hooks:
                h.remove()
            _reset_states(model)
        attn_names = [n for n, m in modules.items() if n and is_attention_like_module(m)]
        targets, visited, last_spike = [], set(), None
        for kind, name in events:
            if kind == "spike":
                last_spike = name
                continue
            if name in visited or last_spike is None:
                continue
            if any(name.startswith(a + ".") for a in attn_names):
                continue  # inside an attention block: the block is the target
            t = self._make_target(name, modules[name], last_spike, input_shapes)
            if t is not None:
                targets.append(t)
                visited.add(name)
        return targets

    # ---- mode 3: module order ---------------------------------------------
    def _analyze_fallback(self, model: nn.Module, input_shapes: dict) -> List[ReplacementTarget]:
        mods = list(model.named_modules())
        attn_names = [n for n, m in mods if n and is_attention_like_module(m)]
        targets, visited = [], set()
        for i, (name, m) in enumerate(mods):
            if not self.registry.is_spike_op(m):
                continue
            for j in range(i + 1, min(i + self.FALLBACK_SEARCH_WINDOW, len(mods))):
                nxt_name, nxt = mods[j]
                if nxt_name in visited:
                    continue
                if self.registry.is_spike_op(nxt):
                    break
                if isinstance(nxt, _TRANSPARENT_MODULES) or not isinstance(nxt, (nn.Conv2d, nn.Linear)):
                    continue
                if any(nxt_name.startswith(a + ".") for a in attn_names):
                    continue
                t = self._make_target(nxt_name, nxt, name, input_shapes)
                if t is not None:
                    targets.append(t)
                    visited.add(nxt_name)
        return targets

    # ---- target construction ----------------------------------------------
    def _make_target(self, name, module, spike_name, input_shapes) -> Optional[ReplacementTarget]:
        if isinstance(module, nn.Conv2d):
            return self._make_conv2d_target(name, module, spike_name, input_shapes)
        if isinstance(module, nn.Linear):
            return ReplacementTarget(conv_name=name, conv_module=module, spike_name=str(spike_name),
                                     op_type="linear", block_size=None)
        if is_attention_like_module(module):
            shp = input_shapes.get(name)
            n, c = (int(shp[-2]), int(shp[-1])) if shp is not None and len(shp) >= 2 else (0, 0)
            return ReplacementTarget(conv_name=name, conv_module=module, spike_name=str(spike_name),
                                     op_type=infer_attention_variant(module), block_size=None,
                                     input_h=n, input_w=c)
        return None

    def _make_conv2d_target(self, conv_name, conv_module, spike_name, input_shapes) -> Optional[ReplacementTarget]:
        op_type = conv2d_op_type(conv_module)
        if op_type is None:
            return None
        h, w = self._extract_hw(input_shapes.get(conv_name))
        if h > 0 and w > 0 and not should_replace(h, w):
            return None
        block = select_block_size(h, w) if h > 0 and w > 0 else None
        return ReplacementTarget(conv_name=conv_name, conv_module=conv_module, spike_name=str(spike_name),
                                 op_type=op_type, block_size=block, input_h=h, input_w=w)

    @staticmethod
    def _extract_hw(ishape) -> Tuple[int, int]:
        if ishape is None or len(ishape) < 2:
            return 0, 0
        return int(ishape[-2]), int(ishape[-1])

    @staticmethod
    def _infer_input_shapes(model: nn.Module, sample_input: torch.Tensor) -> Dict[str, tuple]:
        shapes: Dict[str, tuple] = {}
        hooks = []
        for name, m in model.named_modules():
            def hook(_m, inp, _out, n=name):
                if isinstance(inp, (tuple, list)) and inp and isinstance(inp[0], torch.Tensor):
                    shapes[n] = tuple(inp[0].shape)
            hooks.append(m.register_forward_hook(hook))
        try:
            _reset_states(model)
            with torch.no_grad():
                model(sample_input)
        finally:
            for h in hooks:
                h.remove()
            _reset_states(model)
        return shapes


def _reset_states(model: nn.Module) -> None:
    from ..neuron import reset_net

    reset_net(model)
    try:
        from spikingjelly.activation_based import functional as sj_func  # optional dependency

        sj_func.reset_net(model)
    except ImportError:
        pass
