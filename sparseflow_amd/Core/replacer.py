"""Module replacement pass (drop-in for Core/replacer.py).

Swaps each ReplacementTarget in place by its dotted name: conv2d targets
become SparseConv2d.from_dense, linear targets SparseLinear.from_dense,
attention blocks SparseAttentionBlock.from_dense (StaticZeroConv2d /
StaticZeroLinear for layers listed as exact-zero), with the reference's
`sf_*` observability attributes and its 4-tuple return
(Core/replacer.py:83-292,320-370).
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional, Set, Tuple

import torch.nn as nn

from ..Ops.sparse_attention_block import SparseAttentionBlock
from ..Ops.sparse_conv2d import SparseConv2d
from ..Ops.sparse_linear import SparseLinear
from ..Ops.static_zero_conv2d import StaticZeroConv2d
from ..Ops.static_zero_linear import StaticZeroLinear
from .analyzer import ATTENTION_OP_TYPES, CONV2D_OP_TYPES, ReplacementTarget, display_block_info

_STATIC_ZERO_OP_TYPES = CONV2D_OP_TYPES + ("linear",)


def _set_module_by_name(model: nn.Module, name: str, new_module: nn.Module) -> None:
    parent = model
    parts = name.split(".")
    for part in parts[:-1]:
        parent = parent[int(part)] if part.isdigit() else getattr(parent, part)
    setattr(parent, parts[-1], new_module)


class ModuleReplacer:
    def __init__(self, verbose: bool = True):
        self.verbose = verbose

    @staticmethod
    def _score_family_from_op(op_type: str) -> str:
        if op_type in CONV2D_OP_TYPES or op_type in ("depthwise_conv2d", "conv1d", "conv3d"):
            return "conv"
        if op_type == "linear":
            return "linear"
        if op_type == "attention_linear":
            return "attn_linear"
        if op_type in ("attention_qkav", "attention_qkmix"):
            return "attn_matmul"
        return "unknown"

    def _attach_observability(self, module: nn.Module, target: ReplacementTarget, backend_mode: str,
                              backend_family: Optional[str] = None, fallback_reason: str = "") -> nn.Module:
        if backend_family is None:
            backend_family = "exact_zero" if backend_mode == "staticzero" else "sparse_kernel"
        fam = self._score_family_from_op(str(target.op_type))
        attrs = {
            "sf_layer_name": str(target.conv_name),
            "sf_operator_type": str(target.op_type),
            "sf_operator_family": fam,
            "sf_spike_source": str(target.spike_name),
            "sf_backend_mode": str(backend_mode),
            "sf_dispatch_decision": str(backend_mode),
            "sf_backend_family": str(backend_family),
            "sf_reason_code": "",
            "sf_meta_source": "measured",
            "sf_diag_source": "measured",
            "sf_support_status": "supported",
            "sf_score_family": fam,
            "sf_tile_source": "block_selector" if target.block_size is not None else "runtime",
            "sf_fallback_reason": str(fallback_reason),
        }
        for k, v in attrs.items():
            setattr(module, k, v)
        return module

    def replace(
        self,
        model: nn.Module,
        targets: List[ReplacementTarget],
        block_sizes: Optional[Dict[str, int]] = None,
        static_zero_layers: Optional[Set[str]] = None,
        disable_static_zero: bool = False,
        only_static_zero: bool = False,
        sparse_kwargs: Optional[Dict[str, Any]] = None,
    ) -> Tuple[int, int, int, int]:
        """Returns (replaced, sparse_count, static_zero_count, dense_keep_count)."""
        static_zero_layers = set() if (static_zero_layers is None or disable_static_zero) else set(static_zero_layers)
        sparse_kwargs = sparse_kwargs or {}
        replaced = sparse_count = static_zero_count = dense_keep = 0
        for target in targets:
            name, op = target.conv_name, target.op_type
            block = target.block_size
            if block_sizes and name in block_sizes:
                block = block_sizes[name]
            if name in static_zero_layers and op in _STATIC_ZERO_OP_TYPES:
                if op == "linear":
                    new, kind = StaticZeroLinear.from_linear(target.conv_module), "StaticZeroLinear"
                else:
                    new, kind = StaticZeroConv2d.from_conv(target.conv_module), "StaticZeroConv2d"
                self._attach_observability(new, target, "staticzero", "exact_zero")
                _set_module_by_name(model, name, new)
                replaced += 1
                static_zero_count += 1
                if self.verbose:
                    print(f"  [STATIC ] {name} ({op}) -> {kind}")
                continue
            if only_static_zero:
                dense_keep += 1
                if self.verbose:
                    print(f"  [KEEP   ] {name} ({op}) -> DenseKeep")
                continue
            new = self._create_sparse_module(target, block, sparse_kwargs)
            if new is None:
                dense_keep += 1
                if self.verbose:
                    print(f"  [KEEP   ] {name} ({op}) -> DenseKeep (unsupported)")
                continue
            self._attach_observability(new, target, "sparse", "sparse_kernel")
            _set_module_by_name(model, name, new)
            replaced += 1
            sparse_count += 1
            if self.verbose:
                print(f"  [REPLACE] {name} ({op}) <- {target.spike_name}, {display_block_info(target)}")
        return replaced, sparse_count, static_zero_count, dense_keep

    def _create_sparse_module(self, target: ReplacementTarget, block: Optional[int],
                              sparse_kwargs: Optional[Dict[str, Any]] = None) -> Optional[nn.Module]:
        sparse_kwargs = sparse_kwargs or {}
        thr = float(sparse_kwargs.get("threshold", 1e-6))
        rms = bool(sparse_kwargs.get("return_ms", False))
        if target.op_type == "linear" and isinstance(target.conv_module, nn.Linear):
            lin = SparseLinear.from_dense(target.conv_module, threshold=thr, return_ms=rms)
            lin.collect_diag = bool(sparse_kwargs.get("collect_diag", False))
            lin.profile_runtime = bool(sparse_kwargs.get("profile_runtime", False))
            return lin.to(target.conv_module.weight.device)
        if target.op_type in ATTENTION_OP_TYPES:
            blk = SparseAttentionBlock.from_dense(target.conv_module, variant=target.op_type, threshold=thr,
                                                  return_ms=rms,
                                                  profile_runtime=bool(sparse_kwargs.get("profile_runtime", False)))
            blk.collect_diag = bool(sparse_kwargs.get("collect_diag", False))
            return blk
        if target.op_type not in CONV2D_OP_TYPES or not isinstance(target.conv_module, nn.Conv2d):
            return None
        mod = target.conv_module
        sparse = SparseConv2d.from_dense(
            mod, block_size=block,
            threshold=float(sparse_kwargs.get("threshold", 1e-6)),
            return_ms=bool(sparse_kwargs.get("return_ms", False)),
        )
        sparse.collect_diag = bool(sparse_kwargs.get("collect_diag", False))
        sparse.profile_runtime = bool(sparse_kwargs.get("profile_runtime", False))
        return sparse.to(mod.weight.device)
