"""Per-layer dispatch policy (host logic): decision gates, the
reference-named helpers, and applying decisions to an optimized model on the
CPU (the calibration measures densities there; timings need the GPU)."""

import copy

import torch

import sparseflow_amd as sf
from sparseflow_amd.Models import fold_bn_, spiking_resnet50
from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d
from sparseflow_amd.Ops.static_zero_conv2d import StaticZeroConv2d
from sparseflow_amd.Utils import dispatch as dp


def test_timed_decision_prefers_faster_with_margin():
    d = dp.make_dispatch_decision("a", {"sparse_ms": 0.10, "dense_ms": 0.50, "density": 0.9})
    assert d.backend == "sparse" and d.reason_code == "timed_faster" and d.confidence == 1.0
    d = dp.make_dispatch_decision("a", {"sparse_ms": 0.50, "dense_ms": 0.10, "density": 0.0})
    assert d.backend == "dense" and d.reason_code == "timed_slower" and d.fallback_reason
    # A near tie (within the margin) stays dense.
    d = dp.make_dispatch_decision("a", {"sparse_ms": 0.99, "dense_ms": 1.0})
    assert d.backend == "dense"


def test_gates_before_timings():
    d = dp.make_dispatch_decision("u", {"supported": False, "sparse_ms": 0.01, "dense_ms": 1.0})
    assert d.backend == "dense" and d.support_status == "unsupported"
    d = dp.make_dispatch_decision("z", {"exact_zero": True, "sparse_ms": 0.01, "dense_ms": 1.0})
    assert d.backend == "staticzero"
    d = dp.make_dispatch_decision("z", {"exact_zero": True, "sparse_ms": 0.01, "dense_ms": 1.0},
                                  allow_static_zero=False)
    assert d.backend == "sparse"
    d = dp.make_dispatch_decision("m", {})
    assert d.backend == "dense" and d.reason_code == "missing_diag"


def test_density_only_decision():
    assert dp.make_dispatch_decision("d", {"density": 0.05}).backend == "sparse"
    d = dp.make_dispatch_decision("d", {"density": 0.5})
    assert d.backend == "dense" and d.diag_source == "density_only"


def test_dispatch_all_layers_and_sets():
    diags = {"a": {"density": 0.01}, "b": {"density": 0.9}, "c": {"exact_zero": True}}
    dec = dp.dispatch_all_layers(["a", "b", "c", "d"], diags, zero_layers={"b"})
    zero, sparse = dp.decisions_to_sets(dec)
    assert zero == {"b", "c"} and sparse == {"a"}
    assert dec["d"].backend == "dense"
    assert set(dec["a"].as_dict()) >= {"layer_name", "backend", "reason", "sparse_ms", "dense_ms"}


def _small_model(v_threshold=1.0):
    torch.manual_seed(0)
    m = spiking_resnet50(T=2, num_classes=10, width=8, v_threshold=v_threshold)
    return fold_bn_(m.eval())


def test_dispatch_model_on_cpu_keeps_logits():
    m = _small_model()
    x = torch.randn(2, 3, 64, 64, generator=torch.Generator().manual_seed(1))
    sf.optimize(m, sample_input=x, verbose=False)
    with torch.no_grad():
        ref = m(x)
    dec = dp.dispatch_model(m, x)
    layers = [n for n, mod in m.named_modules() if isinstance(mod, SparseConv2d)]
    assert set(dec) == set(layers) and layers
    for name, mod in m.named_modules():
        if isinstance(mod, SparseConv2d):
            d = dec[name]
            assert 0.0 <= d.density <= 1.0 and d.sparse_ms < 0  # no timings on the CPU
            assert mod.backend_mode == d.backend and mod.sf_dispatch_decision == d.backend
    with torch.no_grad():
        out = m(x)
    assert torch.equal(out, ref)


def test_static_zero_replacement_when_inputs_are_zero():
    # A threshold no membrane reaches: every spike map is zero, so every
    # layer fed by a neuron sees an exactly-zero input.
    m = _small_model(v_threshold=1e9)
    x = torch.randn(1, 3, 64, 64, generator=torch.Generator().manual_seed(2))
    sf.optimize(m, sample_input=x, verbose=False)
    with torch.no_grad():
        ref = m(x)
    dec = dp.dispatch_model(copy.deepcopy(m), x)          # default: no static zero
    assert not any(d.backend == "staticzero" for d in dec.values())
    dec = dp.dispatch_model(m, x, allow_static_zero=True)
    zero, _ = dp.decisions_to_sets(dec)
    assert zero and zero == set(dec)
    szs = [mod for mod in m.modules() if isinstance(mod, StaticZeroConv2d)]
    assert len(szs) == len(zero) and all(mod.sf_backend_mode == "staticzero" for mod in szs)
    with torch.no_grad():
        out = m(x)
    assert torch.allclose(out, ref, atol=1e-5, rtol=1e-5)


def test_dispatch_all_layers_accepts_targets():
    from sparseflow_amd.Core.analyzer import ReplacementTarget
    import inspect
    params = inspect.signature(ReplacementTarget).parameters
    kw = {k: None for k in params}
    kw.update(conv_name="l.conv", op_type="conv2d_3x3")
    t = ReplacementTarget(**{k: v for k, v in kw.items() if k in params})
    dec = dp.dispatch_all_layers([t, {"name": "p", "op_type": "maxpool2d"}], {"l.conv": {"density": 0.01}})
    assert dec["l.conv"].backend == "sparse" and dec["p"].backend == "dense"
    assert dec["p"].reason_code == "pool_dense_keep"


def test_runtime_policy_state_machine():
    # Ops/sparse_conv2d.py:462-496: warmup seeds the average, a zero streak
    # forces the zero path (sticky for the conv), an average above the dense
    # threshold forces dense.
    m = SparseConv2d(8, 8, 3, 1, 1, warmup_steps=2, zero_streak_needed=2, ema_decay=0.5, dense_threshold=0.85)
    m.runtime_policy = True
    pol = m.policy
    assert pol.wants_ratio(False) and not pol.wants_ratio(True)
    pol.observe(0.9)
    pol.observe(0.9)
    assert pol.warmup_left == 0 and pol.forced is None
    pol.observe(0.9)
    assert pol.forced == "dense" and abs(pol.average - 0.9) < 1e-12
    pol.observe(0.0)            # average 0.45 -> not dense; streak 1
    assert pol.forced is None
    pol.observe(0.0)
    assert pol.forced == "zero"
    pol.observe(0.5)            # sticky for the conv module
    assert pol.forced == "zero"
    pol.forwards = 31
    assert not pol.wants_ratio(False)
    pol.forwards = 32
    assert pol.wants_ratio(False)
    off = SparseConv2d(8, 8, 3, 1, 1)
    assert not off.runtime_policy and not off.policy.wants_ratio(False)
    off.policy.observe(0.0)
    assert off._last_avg_active_ratio == 0.0 and off.policy.forced is None


def test_runtime_policy_linear_zero_choice_clears():
    # The Linear module's zero choice lasts only while inputs stay all-zero
    # (Ops/sparse_linear.py:397-405).
    from sparseflow_amd.Ops.sparse_linear import SparseLinear

    m = SparseLinear(8, 8, warmup_steps=0, zero_streak_needed=1, ema_decay=0.5)
    m.runtime_policy = True
    m.policy.observe(0.0)
    assert m.policy.forced == "zero"
    m.policy.observe(0.2)
    assert m.policy.forced is None


def test_runtime_policy_force_zero_output_on_cpu():
    m = SparseConv2d(4, 6, 3, 1, 1, bias=True)
    m.runtime_policy, m.policy.choice = True, "zero"
    x = torch.randn(2, 3, 4, 5, 5)
    y = m(x)
    assert y.shape == (2, 3, 6, 5, 5) and m.fallback_reason == "force_zero"
    assert torch.equal(y, m.bias.detach().view(1, 1, -1, 1, 1).expand_as(y))


def test_conv1x1_lif_fused_or_pair_rule():
    # Host rule of the fused 1x1 conv + LIF module (no GPU needed): resident
    # weights always fuse; streamed ones fuse only when the fused launch's
    # wavefronts fill at least 3/4 of the GPU (Spiking-ResNet50 shapes at
    # batch 32 on 256 CUs: only layer3.0's conv1 qualifies).
    from sparseflow_amd.Kernels.fused_conv_lif import conv1x1_lif_prefers_fused

    cus = 256
    assert conv1x1_lif_prefers_fused(64, 64, 1, 8, 8, cus)        # resident, tiny
    assert conv1x1_lif_prefers_fused(256, 1024, 32, 14, 14, cus)  # resident (two chunks)
    assert not conv1x1_lif_prefers_fused(1024, 256, 32, 14, 14, cus)  # 512 wavefronts
    assert not conv1x1_lif_prefers_fused(512, 128, 32, 28, 28, cus)   # 832
    assert not conv1x1_lif_prefers_fused(1024, 512, 32, 14, 14, cus)  # 1024
    assert conv1x1_lif_prefers_fused(512, 256, 32, 28, 28, cus)       # 1664 >= 1536
    assert conv1x1_lif_prefers_fused(1024, 256, 128, 14, 14, cus)     # 2048 at batch 128
