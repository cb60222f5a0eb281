"""sf_conv2d_forward_noalloc (the entry point that allocates nothing: bitmap
and flags in the library's per-GPU scratch area) against sf_conv2d_forward
with a caller workspace, through the C ABI.  Same kernels, so the outputs
must be equal bit for bit; two calls in a row, the second on a smaller input,
so stale scratch contents from the first call must not leak into the second.
"""

import pytest
import torch

from sparseflow_amd import _lib
from tests.gpu_helpers import DEV, announce, native_loaded, spikes

pytestmark = pytest.mark.gpu


def _run(n, c, h, w, co, k, s, dtype, seed, value=False):
    p = (k - 1) // 2
    ho, wo = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    g = torch.Generator().manual_seed(seed)
    x = spikes((n, c, h, w), 0.05, seed=seed)
    if value:
        x[0, :, 0, :] *= 1.5  # a non-binary chunk: the value path
    x = x.to(DEV, dtype)
    wgt = torch.randn(co, c, k, k, generator=g) * 0.3
    bias = (torch.randn(co, generator=g) * 0.1).to(DEV)
    wt = _lib.tap_major_weight(wgt.to(DEV))
    code = _lib.dtype_code(dtype)
    desc = _lib.conv_desc(n, c, h, w, co, ho, wo, k, s, p, code, code)
    ws = torch.empty(_lib.conv2d_workspace_size(desc), dtype=torch.uint8, device=DEV)
    y_ws = torch.full((n, co, ho, wo), float("nan"), dtype=dtype, device=DEV)
    y_na = torch.full((n, co, ho, wo), float("nan"), dtype=dtype, device=DEV)
    _lib.conv2d_forward(desc, x, wt, bias, 1e-6, ws, y_ws)
    _lib.conv2d_forward_noalloc(desc, x, wt, bias, 1e-6, y_na)
    torch.cuda.synchronize()
    return x, wgt, bias, y_ws, y_na


def test_noalloc_equals_workspace_entry_point_twice_second_smaller():
    # Call 1: 3x3 s1, 64 -> 64 on 16 frames of 28x28 (value path in frame 0).
    announce("noalloc call 1: 3x3 s1 16x64x28x28 f32")
    x1, w1, b1, ref1, out1 = _run(16, 64, 28, 28, 64, 3, 1, torch.float32, seed=1, value=True)
    assert not torch.isnan(out1).any()
    assert torch.equal(out1, ref1)
    # And against torch's conv on the same inputs (fp32 bar 1e-4).
    dense = torch.nn.functional.conv2d(x1.double(), w1.to(DEV).double(), b1.double(), 1, 1)
    assert torch.allclose(out1.double(), dense, atol=1e-4, rtol=1e-4)
    # Call 2, smaller: 3x3 s2, 96 -> 48 on 3 frames of 9x11 (f16).
    announce("noalloc call 2: 3x3 s2 3x96x9x11 f16")
    _, _, _, ref2, out2 = _run(3, 96, 9, 11, 48, 3, 2, torch.float16, seed=2)
    assert not torch.isnan(out2).any()
    assert torch.equal(out2, ref2)
    # Call 3, smaller still: 1x1 s1.
    announce("noalloc call 3: 1x1 s1 2x40x5x7 f32")
    _, _, _, ref3, out3 = _run(2, 40, 5, 7, 36, 1, 1, torch.float32, seed=3)
    assert torch.equal(out3, ref3)
    # Call 4: the matrix-core stem path (f32, C_in = 3: one bitmap word per
    # pixel, read from the scratch).
    announce("noalloc call 4: 3x3 s1 4x3x32x32 f32 (stem)")
    _, _, _, ref4, out4 = _run(4, 3, 32, 32, 24, 3, 1, torch.float32, seed=4)
    assert not torch.isnan(out4).any()
    assert torch.equal(out4, ref4)
    assert native_loaded()


def test_noalloc_warm_call_allocates_nothing():
    n, c, h, w, co = 8, 64, 28, 28, 64
    announce("noalloc warm call: memory unchanged")
    x = spikes((n, c, h, w), 0.05, seed=5).to(DEV)
    wt = _lib.tap_major_weight((torch.randn(co, c, 3, 3, generator=torch.Generator().manual_seed(5)) * 0.1).to(DEV))
    desc = _lib.conv_desc(n, c, h, w, co, h, w, 3, 1, 1, 0, 0)
    y = torch.empty((n, co, h, w), device=DEV)
    _lib.conv2d_forward_noalloc(desc, x, wt, None, 1e-6, y)  # the first call on this GPU may look up and load
    torch.cuda.synchronize()
    y0 = y.clone()
    alloc, (free, total) = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()
    for _ in range(3):
        _lib.conv2d_forward_noalloc(desc, x, wt, None, 1e-6, y)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == alloc
    assert torch.cuda.mem_get_info() == (free, total)
    assert torch.equal(y, y0)


def test_noalloc_rejects_more_than_the_scratch_before_launching():
    # 4096 frames of 256 x 56 x 56 need ~410 MB of bitmap: refused on the host.
    desc = _lib.conv_desc(4096, 256, 56, 56, 64, 56, 56, 3, 1, 1, 0, 0)
    assert _lib.conv2d_workspace_size(desc) > _lib.NOALLOC_SCRATCH_BYTES
    x = torch.empty(1, device=DEV)
    with pytest.raises(_lib.SparseFlowLibError, match="scratch"):
        _lib.conv2d_forward_noalloc(desc, x, x, None, 1e-6, x)
