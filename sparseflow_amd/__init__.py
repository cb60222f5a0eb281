"""SparseFlow-AMD: spike-sparse convolution for MI355X (gfx950).

Drop-in for the reference package entry (__init__.py:16-74):

    import sparseflow_amd as sparseflow
    model = sparseflow.optimize(model, sample_input=x)

Layout mirrors the reference: Core/ (registry, analyzer, replacer), Ops/
(SparseConv2d, FusedSparseConvLIF, StaticZeroConv2d), Kernels/ (host entry
points over the HIP C ABI in libsparseflow_hip.so), Utils/ (constants,
block selector).
"""

from __future__ import annotations

__version__ = "0.1.0"


def optimize(
    model,
    sample_input=None,
    block_sizes=None,
    verbose=True,
    threshold=1e-6,
    return_ms=False,
    collect_diag=False,
    profile_runtime=False,
):
    """Replace, in place, every Conv2d fed by spike sources with SparseConv2d.

    Args mirror the reference's `optimize`: sample_input lets the analyzer
    infer per-layer input shapes (and so apply the H -> block rule),
    block_sizes overrides the block per layer name, threshold is the
    prescan activity threshold.  Returns the same model object.
    """
    from .Core.analyzer import NetworkAnalyzer
    from .Core.registry import SpikeOpRegistry
    from .Core.replacer import ModuleReplacer

    analyzer = NetworkAnalyzer(SpikeOpRegistry.default())
    replacer = ModuleReplacer(verbose=verbose)
    targets = analyzer.analyze(model, sample_input=sample_input)
    if verbose:
        print(f"[SparseFlow] Found {len(targets)} replaceable operators")
    replaced, sparse, static_zero, dense_keep = replacer.replace(
        model,
        targets,
        block_sizes=block_sizes,
        sparse_kwargs={
            "threshold": float(threshold),
            "return_ms": bool(return_ms),
            "collect_diag": bool(collect_diag),
            "profile_runtime": bool(profile_runtime),
        },
    )
    if verbose:
        print(f"[SparseFlow] Replacement summary: total={replaced}, sparse={sparse}, "
              f"static_zero={static_zero}, dense_keep={dense_keep}")
    return model


def native_library_path():
    from ._lib import LIB_PATH

    return LIB_PATH
