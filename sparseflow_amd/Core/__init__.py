"""Graph analysis and module replacement (Core/ of the reference)."""
from .analyzer import NetworkAnalyzer, ReplacementTarget  # noqa: F401
from .registry import SpikeOpRegistry  # noqa: F401
from .replacer import ModuleReplacer  # noqa: F401
