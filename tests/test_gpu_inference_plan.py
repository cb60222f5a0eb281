"""SparseConv2d's steady-state inference forward (the cached one-call plan).

In inference mode, after a forward that ran the library's one-call path,
later forwards of the same input shape repeat that call directly.  Every
case compares against the module's full forward on the same input, bit for
bit, and checks that the plan is dropped whenever what it was built from
changes.
"""

import pytest
import torch

from oracle import conv as oconv
from sparseflow_amd.Kernels import spike_map
from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d
from tests.gpu_helpers import DEV, announce, close, native_loaded, spikes

pytestmark = pytest.mark.gpu


def _module(c_in=64, c_out=64, k=3, s=1, bias=True, seed=0):
    torch.manual_seed(seed)
    conv = torch.nn.Conv2d(c_in, c_out, k, s, (k - 1) // 2, bias=bias)
    m = SparseConv2d.from_dense(conv).to(DEV)
    m.set_inference_mode(True)
    return m, conv


def _full(m, x):
    """The module's full forward (no plan), same state otherwise."""
    saved = m._plan
    m._plan = None
    try:
        y = m._forward_full(x)
    finally:
        m._plan = saved if m._plan is None else m._plan
    return y


@pytest.mark.parametrize("shape,k,s", [((8, 64, 32, 32), 3, 1), ((4, 64, 28, 28), 3, 1), ((4, 96, 14, 14), 3, 2),
                                       ((6, 128, 16, 16), 1, 1)])
def test_plan_repeats_the_full_forward(shape, k, s):
    announce(f"plan {shape} k{k} s{s}")
    m, conv = _module(shape[1], 64, k, s)
    x0 = spikes(shape, 0.02, seed=1, device=DEV)
    with torch.no_grad():
        m(x0)
        assert m._plan is not None
        for seed in (2, 3):
            x = spikes(shape, 0.03, seed=seed, device=DEV)
            y = m(x)
            assert torch.equal(y, _full(m, x))
            ok, err, _ = close(y, oconv.sparse_conv2d_ref(x.cpu(), conv.weight, conv.bias, s, (k - 1) // 2),
                               atol=1e-4, rtol=1e-4)
            assert ok, f"max abs err {err}"
    assert m.policy.forwards >= 3 and m.fallback_reason == ""
    assert native_loaded()


def test_plan_takes_5d_input_and_returns_5d():
    announce("plan 5d")
    m, _ = _module()
    x = spikes((4, 2, 64, 32, 32), 0.02, seed=4, device=DEV)
    with torch.no_grad():
        y0 = m(x)
        y1 = m(spikes((4, 2, 64, 32, 32), 0.02, seed=5, device=DEV))
        y2 = m(x)
    assert m._plan is not None and m._plan.shape == x.shape
    assert y1.shape == (4, 2, 64, 32, 32) and torch.equal(y0, y2)
    assert torch.equal(y2.flatten(0, 1), _full(m, x.flatten(0, 1)))


def test_plan_follows_in_place_weight_and_bias_updates():
    announce("plan weight/bias updates")
    m, _ = _module()
    x = spikes((4, 64, 32, 32), 0.05, seed=6, device=DEV)
    with torch.no_grad():
        m(x)
        y_old = m(x)
        m.weight.mul_(0.5)
        y_w = m(x)
        m.bias.add_(1.0)
        y_b = m(x)
        m2, _ = _module()
        m2.weight.copy_(m.weight)
        m2.bias.copy_(m.bias)
        y_ref = m2(x)
    assert not torch.equal(y_old, y_w) and not torch.equal(y_w, y_b)
    assert torch.equal(y_b, y_ref)


def test_plan_follows_a_replaced_weight_parameter():
    announce("plan replaced parameter")
    m, _ = _module(bias=False)
    x = spikes((4, 64, 32, 32), 0.05, seed=7, device=DEV)
    with torch.no_grad():
        m(x)
        m(x)
        m.weight = torch.nn.Parameter(torch.randn_like(m.weight) * 0.05)
        y = m(x)
    assert torch.equal(y, _full(m, x))


def test_plan_rebuilt_for_a_new_shape_and_dtype():
    announce("plan new shape/dtype")
    m, _ = _module()
    with torch.no_grad():
        for shape in ((8, 64, 32, 32), (3, 64, 32, 32), (8, 64, 32, 32)):
            x = spikes(shape, 0.02, seed=shape[0], device=DEV)
            m(x)
            y = m(x)
            assert m._plan.shape == x.shape and torch.equal(y, _full(m, x))
        xh = spikes((3, 64, 32, 32), 0.02, seed=8, device=DEV).half()
        yh = m(xh)
        assert yh.dtype == torch.float16 and m._plan.dtype == torch.float16
        assert torch.equal(m(xh), yh)


def test_module_switches_bypass_the_plan():
    announce("plan switches")
    m, _ = _module()
    x = spikes((4, 64, 32, 32), 0.03, seed=9, device=DEV)
    with torch.no_grad():
        y = m(x)
        m(x)
        assert m._plan is not None
        m.backend_mode = "dense"
        yd = m(x)
        assert m.fallback_reason == "dispatch_dense" and m._plan is None
        assert torch.allclose(yd, y, atol=1e-4, rtol=1e-4)
        m.backend_mode = "sparse"
        m(x)
        assert m._plan is not None
        m.threshold = 0.5
        m(x)  # the plan's threshold differs: full forward, new plan
        assert m._plan is not None and m._plan.threshold == 0.5
        m.threshold = 1e-6
        m.return_ms = True
        m(x)
        assert m._plan is None
        m.return_ms = False
        m.set_inference_mode(False)
        m(x)
        assert m._plan is None


def test_handed_spike_map_takes_the_full_forward():
    from sparseflow_amd.neuron import LIFNode as Node

    announce("plan vs handed spike map")
    m, _ = _module()
    g = torch.Generator().manual_seed(10)
    cur = (torch.randn(2, 4, 64, 32, 32, generator=g) * 2).to(DEV)
    with torch.no_grad():
        s = Node(step_mode="m")(cur).flatten(0, 1)
        m(s.clone())
        m(s.clone())  # plan for this shape
        assert m._plan is not None
        assert spike_map.recorded(s)
        y = m(s)  # the map recorded for s: full forward, which reads it
        assert torch.equal(y, m(s.clone()))
