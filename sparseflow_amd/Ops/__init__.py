"""nn.Module wrappers of the sparse kernels (Ops/ of the reference)."""
from .sparse_conv2d import SparseConv2d  # noqa: F401
from .sparse_fused_conv_lif import FusedSparseConvLIF  # noqa: F401
from .static_zero_conv2d import StaticZeroConv2d, make_zero_conv_output  # noqa: F401
