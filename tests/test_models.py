"""Spiking-ResNet50 model (host side): BN folding is exact up to rounding,
optimize() finds every eligible conv through torch.fx, and the replaced
model computes the same logits on the CPU (where SparseConv2d runs the
reference's F.conv2d path)."""

import copy

import torch

import sparseflow_amd as sf
from sparseflow_amd.Models import fold_bn_, spiking_resnet50
from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d


def _model(T=2, classes=10, seed=0):
    torch.manual_seed(seed)
    m = spiking_resnet50(T=T, num_classes=classes)
    # Non-trivial BN statistics so folding has something to fold.
    g = torch.Generator().manual_seed(seed + 1)
    for mod in m.modules():
        if isinstance(mod, torch.nn.BatchNorm2d):
            mod.running_mean.copy_(torch.randn(mod.num_features, generator=g) * 0.1)
            mod.running_var.copy_(torch.rand(mod.num_features, generator=g) + 0.5)
    return m.eval()


def test_fold_bn_matches_unfolded():
    m = _model()
    x = torch.randn(1, 3, 64, 64, generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        ref = m(x)
        folded = fold_bn_(copy.deepcopy(m))
        out = folded(x)
    assert not any(isinstance(mod, torch.nn.BatchNorm2d) for mod in folded.modules())
    assert torch.allclose(out, ref, atol=1e-4, rtol=1e-4)


def test_optimize_finds_resnet50_targets_by_fx():
    m = fold_bn_(_model())
    x = torch.randn(1, 3, 224, 224)
    sf.optimize(m, sample_input=x, verbose=False)
    sparse = {n for n, mod in m.named_modules() if isinstance(mod, SparseConv2d)}
    dense = {n for n, mod in m.named_modules() if isinstance(mod, torch.nn.Conv2d) and not isinstance(mod, SparseConv2d)}
    # 16 blocks x 3 convs + layer1's 1x1 s1 downsample = 49 candidates; the
    # stem (image input), the 1x1 stride-2 downsamples and layer4's 7x7 maps
    # (H < 8, block rule) stay dense.
    assert len(sparse) == 42
    assert dense == {"conv1", "layer2.0.downsample.0", "layer3.0.downsample.0", "layer4.0.conv3",
                     "layer4.0.downsample.0", "layer4.1.conv1", "layer4.1.conv2", "layer4.1.conv3",
                     "layer4.2.conv1", "layer4.2.conv2", "layer4.2.conv3"}
    assert "layer1.0.downsample.0" in sparse and "layer4.0.conv2" in sparse  # 14x14 input, stride 2


def test_optimized_model_same_logits_on_cpu():
    m = fold_bn_(_model(seed=3))
    x = torch.randn(2, 3, 64, 64, generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        ref = m(x)
        sf.optimize(m, sample_input=x, verbose=False)
        out = m(x)
    assert torch.equal(out, ref)


def test_fused_pairs_follow_dispatch_swaps_and_dense_decisions():
    # fuse_conv_lif_ builds SparseConv1x1LIF pairs; a later dispatch pass that
    # swaps a block's conv by name makes its pair stale (the block then runs
    # the unfused modules), and a dense decision on the pair's conv turns the
    # fused kernel off.
    from types import SimpleNamespace

    from sparseflow_amd.Models import fuse_conv_lif_
    from sparseflow_amd.Models.spiking_resnet import SpikingBottleneck
    from sparseflow_amd.Ops.static_zero_conv2d import StaticZeroConv2d

    m = fold_bn_(_model(seed=5))
    x = torch.randn(1, 3, 64, 64, generator=torch.Generator().manual_seed(6))
    with torch.no_grad():
        sf.optimize(m, sample_input=x, verbose=False)
        assert fuse_conv_lif_(m) >= 8
        blk = next(b for b in m.modules() if isinstance(b, SpikingBottleneck) and b.conv1_lif is not None)
        pair = blk.conv1_lif
        calls = []
        pair.register_forward_hook(lambda *a: calls.append(1))
        blk.conv1 = StaticZeroConv2d.from_conv(blk.conv1)
        from sparseflow_amd.neuron import reset_net
        reset_net(m)
        m(x)
        assert calls == []          # stale pair not used
    cuda_like = SimpleNamespace(dim=lambda: 5, is_cuda=True, dtype=torch.float32,
                                shape=(2, 1, pair.conv.in_channels, 16, 16))
    assert pair.conv.in_channels <= 256  # resident weights: fused whatever the batch
    assert pair.runs_fused(cuda_like)
    pair.conv.backend_mode = "dense"
    assert not pair.runs_fused(cuda_like)


def test_calibrated_thresholds_give_the_target_density_per_layer():
    # Every neuron layer is calibrated in network order on its own input
    # currents: on the calibration input each layer then fires at ~1%.
    from sparseflow_amd.Models import calibrate_lif_thresholds_
    from sparseflow_amd.neuron import LIFNode, reset_net

    m = fold_bn_(_model(T=4, seed=7))
    x = torch.randn(1, 3, 64, 64, generator=torch.Generator().manual_seed(8))
    rec = calibrate_lif_thresholds_(m, x, target_density=0.01, sample=1 << 15)
    names = [n for n, mod in m.named_modules() if isinstance(mod, LIFNode)]
    assert list(rec) == names and len(names) == 49
    ths = [mod.v_threshold for mod in m.modules() if isinstance(mod, LIFNode)]
    assert len(set(ths)) > 40 and all(t > 0 for t in ths)
    dens = {}
    hooks = [mod.register_forward_hook(lambda _m, _i, o, n=n: dens.__setitem__(n, float(o.float().mean())))
             for n, mod in m.named_modules() if isinstance(mod, LIFNode)]
    with torch.no_grad():
        reset_net(m)
        m(x)
    for h in hooks:
        h.remove()
    for n, d in dens.items():
        assert 0.005 < d < 0.02, f"{n}: density {d}"
