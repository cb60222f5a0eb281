"""nn.Module wrappers of the sparse kernels (Ops/ of the reference)."""
from .sparse_attention import SparseAttention  # noqa: F401
from .sparse_attention_block import SparseAttentionBlock  # noqa: F401
from .sparse_bmm import SparseBMM, SparseMatmul  # noqa: F401
from .sparse_conv2d import SparseConv2d  # noqa: F401
from .sparse_fused_conv_lif import FusedSparseConvLIF  # noqa: F401
from .sparse_linear import SparseLinear  # noqa: F401
from .static_zero_conv2d import StaticZeroConv2d, make_zero_conv_output  # noqa: F401
from .static_zero_linear import StaticZeroLinear  # noqa: F401
