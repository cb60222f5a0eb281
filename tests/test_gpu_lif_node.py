"""LIFNode on ROCm tensors (the library's multi-step LIF kernel) vs the
node's own torch path on the CPU: spikes and membranes bit-identical (the
kernel follows the torch path's arithmetic operation by operation, with IEEE
division by tau; torch's GPU division by a scalar multiplies by the rounded
reciprocal instead, so the CPU path is the exact reference)."""

import pytest
import torch

from sparseflow_amd import _lib
from sparseflow_amd.neuron import BaseNode, LIFNode
from tests.gpu_helpers import DEV, announce, native_loaded

pytestmark = pytest.mark.gpu


def _torch_steps(node, x_seq):
    # The torch implementation the kernel restates (BaseNode's loop).
    node.reset()
    out = torch.stack([BaseNode.single_step_forward(node, x_seq[t]) for t in range(x_seq.shape[0])])
    return out, node.v


CASES = [
    # (shape, dtype, tau, v_th, v_reset, decay_input)
    ((8, 4, 64, 28, 28), torch.float32, 2.0, 1.0, 0.0, True),
    ((5, 3, 17, 9, 7), torch.float32, 1.5, 0.5, None, True),    # soft reset, odd size (scalar path)
    ((4, 2, 32, 16, 16), torch.float32, 3.0, 0.8, -0.2, False),
    ((6, 2, 48, 10, 10), torch.float16, 2.0, 1.0, 0.0, True),
    ((3, 2, 40, 8, 8), torch.bfloat16, 2.0, 1.0, None, False),
    ((1, 1, 1, 1, 3), torch.float32, 2.0, 1.0, 0.0, True),      # three neurons, one step
]


@pytest.mark.parametrize("case", CASES)
def test_lif_node_kernel_matches_torch_path(case):
    shape, dtype, tau, v_th, v_reset, decay_input = case
    announce(f"lif node {case}")
    g = torch.Generator().manual_seed(len(shape) + shape[0])
    x = (torch.randn(shape, generator=g) * 1.5 + 0.5).to(dtype).to(DEV)
    node = LIFNode(tau=tau, v_threshold=v_th, v_reset=v_reset, decay_input=decay_input, step_mode="m")
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        s_k = node(x)
        v_k = node.v.clone()
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    assert stats["lif_multistep"][0] == 1
    s_t, v_t = _torch_steps(node, x.cpu())
    assert s_k.dtype == dtype and s_k.shape == x.shape
    assert torch.equal(s_k.cpu(), s_t)
    assert torch.equal(v_k.cpu(), v_t)
    assert native_loaded()


def test_lif_node_single_steps_chain_to_multistep():
    x = (torch.randn(6, 2, 16, 12, 12, generator=torch.Generator().manual_seed(3)) * 2).to(DEV)
    announce("lif node chain")
    ms = LIFNode(step_mode="m")
    s_all = ms(x)
    ss = LIFNode(step_mode="s")
    s_steps = torch.stack([ss(x[t]) for t in range(6)])
    assert torch.equal(s_all, s_steps)
    assert torch.equal(ms.v, ss.v)
    # State carried across two multi-step calls.
    ms.reset()
    s_a = ms(x[:2])
    s_b = ms(x[2:])
    assert torch.equal(torch.cat([s_a, s_b]), s_all)


def test_lif_multistep_rejects_bad_arguments():
    x = torch.zeros(2, 8, device=DEV)
    lif = _lib.LifParams(2.0, 1.0, 0.0, 1, 1)
    with pytest.raises(ValueError):
        _lib.lif_multistep(x, 3, lif)
    with pytest.raises(_lib.SparseFlowLibError):
        _lib.lif_multistep(x, 2, _lib.LifParams(0.0, 1.0, 0.0, 1, 1))


def test_lif_residual_fused_equals_add_first():
    g = torch.Generator().manual_seed(7)
    a = (torch.randn(4, 2, 24, 9, 9, generator=g) * 1.5).to(DEV)
    b = (torch.rand(4, 2, 24, 9, 9, generator=g) < 0.3).float().to(DEV)
    announce("lif residual")
    n1, n2 = LIFNode(step_mode="m"), LIFNode(step_mode="m")
    s_fused = n1(a, b)
    s_ref = n2(a + b)
    assert torch.equal(s_fused, s_ref)
    assert torch.equal(n1.v, n2.v)


@pytest.mark.parametrize("shape", [(4, 2, 64, 14, 14), (3, 2, 256, 7, 9), (2, 3, 40, 5, 5), (2, 1, 3, 6, 6)])
def test_lif_spike_map_equals_prescan(shape):
    from sparseflow_amd.Kernels import spike_map

    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * 2).to(DEV)
    announce(f"lif spike map {shape}")
    node = LIFNode(step_mode="m")
    s = node(x)
    T, N, C, H, W = shape
    got = spike_map.lookup(s.flatten(0, 1), 1e-6)
    assert got is not None
    bits_ref, flags_ref = _lib.prescan_pack(s.flatten(0, 1), 1e-6)
    nb = bits_ref.numel()
    assert torch.equal(got[0][:nb], bits_ref)
    assert torch.equal(got[1][:flags_ref.numel()], flags_ref)
    # An in-place change invalidates the map.
    s.mul_(1.0)
    assert spike_map.lookup(s.flatten(0, 1), 1e-6) is None


def test_conv_consumes_handed_spike_map():
    from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward

    g = torch.Generator().manual_seed(9)
    x = (torch.randn(4, 2, 64, 16, 16, generator=g) * 2).to(DEV)
    w = (torch.randn(64, 64, 3, 3, generator=g) * 0.05).to(DEV)
    announce("handed spike map conv")
    s = LIFNode(step_mode="m")(x)
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        y_handed, _, meta = sparse_conv2d_forward(s.flatten(0, 1), w, None, 3, 1, 1, return_backend_meta=True)
        y_own = sparse_conv2d_forward(s.flatten(0, 1).clone(), w, None, 3, 1, 1)[0]
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    assert meta["reason"] == "bitmap_gather_handed_spike_map"
    assert stats["prescan_pack"][0] == 1  # only the clone was packed
    assert torch.equal(y_handed, y_own)
