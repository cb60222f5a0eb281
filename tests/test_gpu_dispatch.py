"""Per-layer dispatch on the GPU: the calibration forward times every
SparseConv2d both ways on its real input, the decisions follow the timings,
and the dispatched model computes what it computed before (a dense-dispatched
layer runs F.conv2d, a sparse one the library kernels)."""

import pytest
import torch

import sparseflow_amd as sf
from sparseflow_amd import _lib
from sparseflow_amd.Models import fold_bn_, spiking_resnet50
from sparseflow_amd.neuron import reset_net
from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d
from sparseflow_amd.Utils import dispatch as dp
from tests.gpu_helpers import DEV, announce, native_loaded

pytestmark = pytest.mark.gpu


def _model(T=2, gain=3.0):
    torch.manual_seed(0)
    m = spiking_resnet50(T=T, num_classes=10, width=16)
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, torch.nn.Conv2d):
                mod.weight.mul_(gain)
    return fold_bn_(m).to(DEV)


def test_dispatch_times_every_layer_and_keeps_logits():
    announce("dispatch resnet50 w16")
    m = _model()
    x = torch.randn(2, 3, 64, 64, generator=torch.Generator().manual_seed(1)).to(DEV)
    sf.optimize(m, sample_input=x, verbose=False)
    with torch.no_grad():
        reset_net(m)
        ref = m(x)
    dec = dp.dispatch_model(m, x, repeats=2)
    names = [n for n, mod in m.named_modules() if isinstance(mod, SparseConv2d)]
    assert set(dec) == set(names)
    for d in dec.values():
        assert d.sparse_ms > 0 and d.dense_ms > 0 and d.reason_code in ("timed_faster", "timed_slower")
        assert d.backend == ("sparse" if d.sparse_ms <= dp.SPARSE_MARGIN * d.dense_ms else "dense")
    # Force a mix so both paths run in the dispatched model.
    for i, n in enumerate(names):
        dec[n].backend = "dense" if i % 2 else "sparse"
    dp.apply_decisions(m, dec)
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        with torch.no_grad():
            reset_net(m)
            out = m(x)
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    launched = sum(c for k, (c, _) in stats.items() if k.startswith("conv"))
    sparse_layers = sum(1 for n in names if dec[n].backend == "sparse")
    assert launched >= sparse_layers > 0
    assert all(mod.backend_mode == dec[n].backend for n, mod in m.named_modules() if isinstance(mod, SparseConv2d))
    assert torch.allclose(out, ref, atol=1e-3, rtol=1e-3), (out - ref).abs().max()
    assert native_loaded()


def test_all_dense_dispatch_launches_no_conv_kernel():
    announce("dispatch all dense")
    m = _model()
    x = torch.randn(1, 3, 64, 64, generator=torch.Generator().manual_seed(2)).to(DEV)
    sf.optimize(m, sample_input=x, verbose=False)
    names = [n for n, mod in m.named_modules() if isinstance(mod, SparseConv2d)]
    dec = dp.dispatch_all_layers(names, {n: {"sparse_ms": 2.0, "dense_ms": 1.0} for n in names})
    assert dp.apply_decisions(m, dec)["dense"] == len(names)
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        with torch.no_grad():
            reset_net(m)
            m(x)
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    conv = {k: c for k, (c, _) in stats.items() if c > 0 and k.startswith("conv")}
    assert not conv, conv


def test_runtime_policy_on_device():
    announce("runtime policy")
    conv = torch.nn.Conv2d(32, 16, 3, 1, 1).to(DEV)
    z = SparseConv2d.from_dense(conv, warmup_steps=1, zero_streak_needed=2, calib_every=1)
    z.runtime_policy = True
    x0 = torch.zeros(4, 32, 16, 16, device=DEV)
    for _ in range(3):
        y = z(x0)
    assert z._last_avg_active_ratio == 0.0 and z.policy.forced == "zero"
    xs = (torch.rand(4, 32, 16, 16, generator=torch.Generator().manual_seed(5)) < 0.05).float().to(DEV)
    y = z(xs)  # sticky, as the reference's policy
    assert z.fallback_reason == "force_zero"
    assert torch.equal(y, conv.bias.detach().view(1, -1, 1, 1).expand_as(y))

    d = SparseConv2d.from_dense(conv, warmup_steps=1, calib_every=1)
    d.runtime_policy = True
    x1 = torch.ones(4, 32, 16, 16, device=DEV)
    d(x1)
    d(x1)
    assert d._last_avg_active_ratio == 1.0 and d.policy.forced == "dense"
    y = d(xs)
    assert d.fallback_reason == "force_dense"
    assert torch.allclose(y, conv(xs), atol=1e-4, rtol=1e-4)
