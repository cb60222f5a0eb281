"""Python drop-in surface on the CPU: optimize / analyzer / replacer,
SparseConv2d and FusedSparseConvLIF host behaviour, neurons, block rule."""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import sparseflow_amd as sparseflow
from oracle import lif as olif
from sparseflow_amd import _lib
from sparseflow_amd.Core.analyzer import NetworkAnalyzer
from sparseflow_amd.Core.registry import SpikeOpRegistry
from sparseflow_amd.Core.replacer import ModuleReplacer
from sparseflow_amd.Kernels._prescan_common import build_rf_prescan_metadata
from sparseflow_amd.Kernels.conv2d import sparse_conv2d_forward
from sparseflow_amd.neuron import IFNode, LIFNode, reset_net
from sparseflow_amd.Ops import FusedSparseConvLIF, SparseConv2d, StaticZeroConv2d, make_zero_conv_output
from sparseflow_amd.Utils.block_selector import select_block_size, should_replace
from sparseflow_amd.Utils.sparse_helpers import choose_group_size, popcount_buf


class SpikingNet(nn.Module):
    """stem conv (dense input) -> LIF -> 3x3 -> LIF -> {3x3 s2, 1x1} ->
    LIF -> 5x5 (unsupported) ; plus a grouped conv."""

    def __init__(self):
        super().__init__()
        self.stem = nn.Conv2d(3, 16, 3, 1, 1)
        self.bn = nn.BatchNorm2d(16)
        self.lif1 = LIFNode(step_mode="m")
        self.conv2 = nn.Conv2d(16, 16, 3, 1, 1, bias=False)
        self.lif2 = LIFNode(step_mode="m")
        self.down = nn.Conv2d(16, 32, 3, 2, 1)
        self.proj = nn.Conv2d(16, 32, 1, 1, 0)
        self.lif3 = IFNode(step_mode="m")
        self.big = nn.Conv2d(32, 32, 5, 1, 2)
        self.grouped = nn.Conv2d(32, 32, 3, 1, 1, groups=4)

    def forward(self, x):  # x [T, B, 3, H, W]
        T, B = x.shape[0], x.shape[1]
        y = self.bn(self.stem(x.flatten(0, 1))).reshape(T, B, 16, x.shape[3], x.shape[4])
        s = self.lif1(y)
        s = self.lif2(self.conv2(s.flatten(0, 1)).reshape(s.shape))
        f = s.flatten(0, 1)
        z = self.down(f) + F.max_pool2d(self.proj(f), 2)
        z = self.lif3(z.unflatten(0, (T, B)))
        zf = z.flatten(0, 1)
        return self.big(zf) + self.grouped(zf)


def _names(targets):
    return {t.conv_name: t for t in targets}


def test_block_rule_and_group_helpers():
    assert [select_block_size(h) for h in (64, 32, 31, 16, 15, 8, 7, 0)] == [16, 16, 8, 8, 4, 4, None, 16]
    assert select_block_size(56, 7) is None
    assert should_replace(0) and not should_replace(7)
    assert choose_group_size(64) == 16 and choose_group_size(512) == 32 and choose_group_size(2048) == 64
    m = torch.tensor([0, 1, -1, 0x7FFFFFFF, -(1 << 31), 0x0F0F], dtype=torch.int32)
    assert popcount_buf(m, 6).tolist() == [0, 1, 32, 31, 1, 8]


def test_analyzer_fx_path_finds_spike_fed_convs():
    import warnings

    net = SpikingNet().eval()
    x = torch.rand(2, 2, 3, 32, 32)
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # the fx path must succeed without falling back
        targets = NetworkAnalyzer(SpikeOpRegistry.default()).analyze(net, sample_input=x)
    t = _names(targets)
    assert set(t) == {"conv2", "down", "proj"}  # stem fed by input; 5x5 and grouped unsupported
    assert t["conv2"].op_type == "conv2d_3x3" and t["conv2"].spike_name == "lif1"
    assert t["down"].op_type == "conv2d_3x3_s2" and t["proj"].op_type == "conv2d_1x1"
    assert t["conv2"].input_h == 32 and t["conv2"].block_size == 16


def test_analyzer_applies_h_block_rule():
    net = SpikingNet().eval()
    x = torch.rand(1, 1, 3, 14, 14)
    t = _names(NetworkAnalyzer(SpikeOpRegistry.default()).analyze(net, sample_input=x))
    assert t["conv2"].block_size == 4 and t["down"].block_size == 4
    x = torch.rand(1, 1, 3, 6, 6)  # H < 8 everywhere: nothing replaced
    assert NetworkAnalyzer(SpikeOpRegistry.default()).analyze(net, sample_input=x) == []


class Untraceable(nn.Module):
    def __init__(self):
        super().__init__()
        self.lif = LIFNode(step_mode="s")
        self.a = nn.Conv2d(4, 4, 3, 1, 1)
        self.b = nn.Conv2d(4, 4, 1)

    def forward(self, x):
        s = self.lif(x)
        if s.sum() > -1:  # data-dependent control flow defeats torch.fx
            s = self.a(s)
        return self.b(s)


def test_analyzer_runtime_and_module_order_fallbacks():
    net = Untraceable()
    with pytest.warns(UserWarning):
        t = NetworkAnalyzer(SpikeOpRegistry.default()).analyze(net, sample_input=torch.rand(2, 4, 8, 8))
    # Runtime order: `a` follows the spike event; `b` follows `a` (no new spike) and is also paired.
    assert [x.conv_name for x in t] == ["a", "b"]
    with pytest.warns(UserWarning):
        t2 = NetworkAnalyzer(SpikeOpRegistry.default()).analyze(net)
    assert [x.conv_name for x in t2] == ["a", "b"]


def test_optimize_replaces_in_place_and_matches_dense_on_cpu():
    torch.manual_seed(0)
    net = SpikingNet().eval()
    x = (torch.rand(2, 2, 3, 16, 16) > 0.3).float()
    with torch.no_grad():
        reset_net(net)
        ref = net(x)
    out_model = sparseflow.optimize(net, sample_input=x, verbose=False)
    assert out_model is net
    assert isinstance(net.conv2, SparseConv2d) and isinstance(net.down, SparseConv2d)
    assert isinstance(net.proj, SparseConv2d) and isinstance(net.stem, nn.Conv2d)
    assert not isinstance(net.big, SparseConv2d) and not isinstance(net.grouped, SparseConv2d)
    assert net.conv2.sf_spike_source == "lif1" and net.conv2.sf_backend_mode == "sparse"
    assert net.conv2.block_size == 8
    with torch.no_grad():
        reset_net(net)
        got = net(x)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)


def test_replacer_static_zero_and_counts():
    net = SpikingNet().eval()
    x = torch.rand(1, 1, 3, 16, 16)
    targets = NetworkAnalyzer(SpikeOpRegistry.default()).analyze(net, sample_input=x)
    counts = ModuleReplacer(verbose=False).replace(net, targets, static_zero_layers={"proj"},
                                                   block_sizes={"conv2": 4})
    assert counts == (3, 2, 1, 0)
    assert isinstance(net.proj, StaticZeroConv2d) and net.proj.sf_backend_family == "exact_zero"
    assert net.conv2.block_size == 4


def test_static_zero_outputs_bias():
    conv = nn.Conv2d(8, 5, 3, 2, 1)
    sz = StaticZeroConv2d.from_conv(conv)
    y4 = sz(torch.zeros(3, 8, 9, 9))
    torch.testing.assert_close(y4, F.conv2d(torch.zeros(3, 8, 9, 9), conv.weight, conv.bias, 2, 1))
    y5 = sz(torch.zeros(2, 3, 8, 9, 9))
    assert y5.shape == (2, 3, 5, 5, 5)
    y5.add_(1.0)  # write-safe: the template is not aliased
    torch.testing.assert_close(sz(torch.zeros(3, 8, 9, 9)), y4)
    z = make_zero_conv_output(2, 4, 3, 3, None, "cpu")
    assert z.abs().sum() == 0


def test_sparse_conv2d_module_host_path():
    conv = nn.Conv2d(16, 24, 3, 2, 1)
    sp = SparseConv2d.from_dense(conv, block_size=8)
    x = (torch.rand(3, 2, 16, 12, 12) > 0.9).float()
    y = sp(x)
    torch.testing.assert_close(y.flatten(0, 1), conv(x.flatten(0, 1)))
    assert sp.fallback_reason == "module_dense_path"
    with pytest.raises(ValueError):
        sp(torch.rand(2, 16, 12))
    assert "block_size=8" in sp.extra_repr()
    sp.set_inference_mode(True)
    assert not sp.collect_diag and not sp.profile_runtime


def test_sparse_conv2d_forward_host_tensors_fall_back_dense():
    x = torch.rand(2, 8, 10, 10)
    w = torch.randn(4, 8, 3, 3)
    out = sparse_conv2d_forward(x, w, None, 3, 1, 1, return_avg_active_ratio=True, return_tile_stats=True,
                                return_backend_meta=True)
    assert len(out) == 5
    assert out[4]["backend"] == "dense_fallback" and out[4]["reason"] == "host_tensor"
    torch.testing.assert_close(out[0], F.conv2d(x, w, None, 1, 1))


def test_prescan_requires_device_tensor():
    x = torch.rand(1, 8, 8, 16)
    with pytest.raises(_lib.SparseFlowLibError):
        build_rf_prescan_metadata(x, (8, 8), 3, 1, 1, (8, 8), 16, 1, 1e-6)
    with pytest.raises(NotImplementedError):
        build_rf_prescan_metadata(torch.rand(1, 8, 8, 8, 4), (8, 8, 8), 3, 1, 1, (8, 8, 8), 16, 1, 1e-6)


def test_lif_node_matches_oracle_and_modes():
    I = torch.randn(7, 3, 5) * 1.2
    for v_reset, decay in [(0.0, True), (None, True), (0.0, False), (-0.3, True)]:
        node = LIFNode(tau=1.7, v_threshold=0.9, v_reset=v_reset, decay_input=decay, step_mode="m")
        s = node(I)
        v0 = None if v_reset is None else np.full((3, 5), v_reset, np.float32)
        s_ref, v_ref, _ = olif.lif_multistep(I.numpy(), 1.7, 0.9, v_reset, decay, v0=v0)
        assert (s.numpy() > 0.5).tolist() == s_ref.tolist()
        np.testing.assert_allclose(node.v.numpy(), v_ref, rtol=0, atol=0)
        node.reset()
        single = LIFNode(tau=1.7, v_threshold=0.9, v_reset=v_reset, decay_input=decay, step_mode="s")
        s_single = torch.stack([single(I[t]) for t in range(7)])
        assert torch.equal(s_single, s)


def test_fused_conv_lif_module_host_path_matches_oracle():
    conv = nn.Conv2d(8, 12, 3, 1, 1)
    lif = LIFNode(tau=2.0, v_threshold=1.0, v_reset=None, decay_input=False)
    mod = FusedSparseConvLIF.from_conv_and_lif(conv, lif)
    assert mod.v_reset is None and not mod.decay_input
    x = (torch.rand(5, 2, 8, 7, 7) > 0.7).float()
    with torch.no_grad():
        s = mod(x)
        I = np.stack([F.conv2d(x[t], conv.weight, conv.bias, 1, 1).numpy() for t in range(5)])
    s_ref, v_ref, _ = olif.lif_multistep(I, 2.0, 1.0, None, False)
    assert (s.numpy() > 0.5).tolist() == s_ref.tolist()
    np.testing.assert_allclose(mod.v.numpy(), v_ref, rtol=0, atol=0)
    reset_net(mod)
    assert mod.v is None


def test_package_exposes_reference_layout():
    import sparseflow_amd.Core as C
    import sparseflow_amd.Kernels.conv2d as K
    import sparseflow_amd.Kernels.fused_conv_lif as KF
    import sparseflow_amd.Ops as O
    import sparseflow_amd.Utils.config as cfg

    assert callable(sparseflow.optimize) and sparseflow.__version__
    assert hasattr(C, "NetworkAnalyzer") and hasattr(C, "ModuleReplacer") and hasattr(C, "SpikeOpRegistry")
    assert hasattr(K, "sparse_conv2d_forward") and hasattr(K, "_select_tile_sizes")
    assert hasattr(KF, "sparse_fused_conv_lif_forward")
    assert hasattr(O, "SparseConv2d") and hasattr(O, "FusedSparseConvLIF")
    assert cfg.PRESCAN_ACTIVITY_EPS == 1e-6 and cfg.ENABLE_RUNTIME_FALLBACK_POLICY is False


# Key names of the reference's exact-zero diagnostics (Ops/static_zero_conv2d.py
# get_diag and make_synthetic_zero_diag): the schema its harness reads.
_STATIC_ZERO_DIAG_KEYS = {"backend_family", "zero_reason", "diag_path", "fallback_reason", "has_bias",
                          "out_channels", "forward_count", "template_cache_size", "sparse_path_executed",
                          "sparse_total_ms"}
_SYNTHETIC_ZERO_DIAG_KEYS = {"active_group_ratio", "tile_zero_ratio", "total_group_count", "nonzero_group_count",
                             "tile_zero_count", "total_tile_count", "effective_k_ratio", "sparse_compute_ms",
                             "sparse_total_ms", "zero_tiles", "sparse_tiles", "denseish_tiles", "stage1_zero_tiles",
                             "stage2_tiles", "prescan_mode", "_synthetic", "_diag_path", "backend_family",
                             "zero_reason"}


def test_static_zero_conv_matches_dense_conv_of_zeros_for_every_geometry():
    from sparseflow_amd.Ops.static_zero_conv2d import make_synthetic_zero_diag

    for k, s, p, d, bias in [(3, 1, 1, 1, True), (3, 2, 1, 1, False), (1, 1, 0, 1, True), (5, 3, 2, 2, True),
                             ((3, 1), (2, 1), (0, 1), (1, 1), True)]:
        conv = nn.Conv2d(4, 6, k, s, p, d, bias=bias)
        sz = StaticZeroConv2d.from_conv(conv, zero_reason="probe")
        sz.collect_diag = True
        x = torch.zeros(2, 3, 4, 11, 13)
        y = sz(x)
        ref = conv(x.flatten(0, 1)).reshape(2, 3, *conv(x[0]).shape[1:])
        torch.testing.assert_close(y, ref, rtol=0, atol=0)
        assert y.dtype == x.dtype
        diag = sz.get_diag()
        assert set(diag) == _STATIC_ZERO_DIAG_KEYS and sz._last_diag == diag
        assert diag["forward_count"] == 1 and diag["has_bias"] == bias and diag["zero_reason"] == "probe"
    assert sz(torch.zeros(2, 4, 7, 7, dtype=torch.float16)).dtype == torch.float16
    with pytest.raises(ValueError):
        sz(torch.zeros(4, 7, 7))
    syn = make_synthetic_zero_diag("layer1.0.conv2", total_group_count=8.0, total_tile_count=12.0)
    assert set(syn) - {"layer_name"} == _SYNTHETIC_ZERO_DIAG_KEYS
    assert syn["zero_tiles"] == syn["stage1_zero_tiles"] == 12 and syn["tile_zero_ratio"] == 1.0
    assert make_synthetic_zero_diag()["zero_tiles"] == -1


def test_static_zero_linear_and_reporting_mixin():
    from sparseflow_amd.Ops import StaticZeroLinear
    from sparseflow_amd.Ops.sparse_attention import SparseAttention
    from sparseflow_amd.Ops.sparse_bmm import SparseBMM, SparseMatmul
    from sparseflow_amd.Ops.sparse_linear import SparseLinear

    lin = nn.Linear(5, 3)
    z = StaticZeroLinear.from_linear(lin)
    torch.testing.assert_close(z(torch.zeros(2, 4, 5)), lin(torch.zeros(2, 4, 5)), rtol=0, atol=0)
    assert z.get_diag()["forward_count"] == 1 and z.get_diag()["out_features"] == 3
    mods = [SparseConv2d(4, 4, 3, 1, 1), SparseLinear(4, 4), SparseAttention(2, 4), SparseBMM(), SparseMatmul(),
            FusedSparseConvLIF(4, 4, 3, padding=1)]
    for m in mods:
        assert m._last_sparse_ms == 0.0 and m._last_diag == {} and m.support_status == "supported"
        m.collect_diag = True
        m.profile_runtime = True
        m.set_inference_mode(True)
        assert m._inference_mode and not m.collect_diag and not m.profile_runtime
    assert mods[3].diag_path == "bmm" and mods[4].score_family == "matmul"
