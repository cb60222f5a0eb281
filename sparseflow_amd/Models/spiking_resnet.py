"""Multi-step Spiking-ResNet (bottleneck 3-4-6-3 = ResNet-50) for the
end-to-end images/s workload.

The reference benchmarks spikingjelly's `spiking_resnet50` with multi-step
LIF neurons, BN folded into the convolutions and random weights
(Benchmark/bench_4test.py:166-197, 696-726, 845-877); spikingjelly is not
installed here, so the network is restated with this package's LIFNode:

  stem   conv 7x7/2 (3 -> 64) + BN + LIF + max-pool 3x3/2
  layers bottleneck blocks: conv1x1 + BN + LIF, conv3x3 (stride s) + BN +
         LIF, conv1x1 (x4) + BN, + identity or downsample (conv1x1/s + BN),
         LIF
  head   global average pool, fc, mean over the T steps

Activations are [T, N, C, H, W]; every conv/BN runs on the T*N frames at
once.  The input image is direct-encoded (the same frame at every step, as
the reference's `raw_repeat`, Benchmark/bench_4test.py:303-304), so the stem
conv + BN run once on the N images and their output is repeated over T
(conv(repeat(x)) == repeat(conv(x))).
"""

from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn as nn

from ..Ops.spike_pool import SpikeMaxPool2d

from ..neuron import LIFNode


def _seq(conv: nn.Module, bn: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """conv + BN over the T*N frames of a [T, N, C, H, W] tensor."""
    T, N = x.shape[0], x.shape[1]
    y = bn(conv(x.flatten(0, 1)))
    return y.reshape(T, N, y.shape[1], y.shape[2], y.shape[3])


def _lif(**kw) -> LIFNode:
    return LIFNode(step_mode="m", **kw)


class SpikingBottleneck(nn.Module):
    expansion = 4

    def __init__(self, inplanes: int, planes: int, stride: int = 1, downsample: Optional[nn.Sequential] = None,
                 neuron: Optional[dict] = None):
        super().__init__()
        neuron = neuron or {}
        self.conv1 = nn.Conv2d(inplanes, planes, 1, bias=False)
        self.bn1 = nn.BatchNorm2d(planes)
        self.sn1 = _lif(**neuron)
        self.conv2 = nn.Conv2d(planes, planes, 3, stride, 1, bias=False)
        self.bn2 = nn.BatchNorm2d(planes)
        self.sn2 = _lif(**neuron)
        self.conv3 = nn.Conv2d(planes, planes * self.expansion, 1, bias=False)
        self.bn3 = nn.BatchNorm2d(planes * self.expansion)
        self.downsample = downsample
        self.sn3 = _lif(**neuron)
        # Set by fuse_conv_lif_: conv1 + sn1 and conv3 + (residual) + sn3 as
        # single fused modules.
        self.conv1_lif: Optional[nn.Module] = None
        self.conv3_lif: Optional[nn.Module] = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # A fused pair is used only while it still wraps this block's conv: a
        # dispatch pass that swapped the conv by name (for a static-zero one)
        # makes the pair stale, and the unfused modules then run.
        if self.conv1_lif is not None and self.conv1_lif.conv is self.conv1:
            out = self.conv1_lif(x)
        else:
            out = self.sn1(_seq(self.conv1, self.bn1, x))
        out = self.sn2(_seq(self.conv2, self.bn2, out))
        identity = x if self.downsample is None else _seq(self.downsample[0], self.downsample[1], x)
        if self.conv3_lif is not None and self.conv3_lif.conv is self.conv3:
            return self.conv3_lif(out, identity)
        out = _seq(self.conv3, self.bn3, out)
        return self.sn3(out, identity)  # LIF(out + identity), the add fused into the neuron pass


class SpikingResNet(nn.Module):
    def __init__(self, layers: List[int], T: int = 16, num_classes: int = 1000, neuron: Optional[dict] = None,
                 width: int = 64):
        super().__init__()
        self.T = int(T)
        self.neuron = dict(neuron or {})
        self.inplanes = width
        self.conv1 = nn.Conv2d(3, width, 7, 2, 3, bias=False)
        self.bn1 = nn.BatchNorm2d(width)
        self.sn1 = _lif(**self.neuron)
        # nn.MaxPool2d that pools handed spike maps on the GPU (Ops.spike_pool).
        self.maxpool = SpikeMaxPool2d(3, 2, 1)
        self.layer1 = self._make_layer(width, layers[0], 1)
        self.layer2 = self._make_layer(width * 2, layers[1], 2)
        self.layer3 = self._make_layer(width * 4, layers[2], 2)
        self.layer4 = self._make_layer(width * 8, layers[3], 2)
        self.avgpool = nn.AdaptiveAvgPool2d(1)
        self.fc = nn.Linear(width * 8 * SpikingBottleneck.expansion, num_classes)
        for m in self.modules():
            if isinstance(m, nn.Conv2d):
                nn.init.kaiming_normal_(m.weight, mode="fan_out", nonlinearity="relu")
            elif isinstance(m, nn.BatchNorm2d):
                nn.init.ones_(m.weight)
                nn.init.zeros_(m.bias)

    def _make_layer(self, planes: int, blocks: int, stride: int) -> nn.Sequential:
        downsample = None
        if stride != 1 or self.inplanes != planes * SpikingBottleneck.expansion:
            downsample = nn.Sequential(
                nn.Conv2d(self.inplanes, planes * SpikingBottleneck.expansion, 1, stride, bias=False),
                nn.BatchNorm2d(planes * SpikingBottleneck.expansion),
            )
        layers = [SpikingBottleneck(self.inplanes, planes, stride, downsample, self.neuron)]
        self.inplanes = planes * SpikingBottleneck.expansion
        layers += [SpikingBottleneck(self.inplanes, planes, 1, None, self.neuron) for _ in range(1, blocks)]
        return nn.Sequential(*layers)

    def forward(self, img: torch.Tensor) -> torch.Tensor:
        """img [N, 3, H, W] -> logits [N, num_classes] (mean over T steps)."""
        stem = self.bn1(self.conv1(img))
        x = stem.unsqueeze(0).expand(self.T, -1, -1, -1, -1).contiguous()
        x = self.sn1(x)
        T, N = x.shape[0], x.shape[1]
        x = self.maxpool(x.flatten(0, 1))
        x = x.reshape(T, N, x.shape[1], x.shape[2], x.shape[3])
        x = self.layer4(self.layer3(self.layer2(self.layer1(x))))
        x = self.avgpool(x.flatten(0, 1)).flatten(1)
        x = self.fc(x)
        return x.reshape(T, N, x.shape[1]).mean(0)


def spiking_resnet50(T: int = 16, num_classes: int = 1000, tau: float = 2.0, v_threshold: float = 1.0,
                     v_reset: Optional[float] = 0.0, width: int = 64) -> SpikingResNet:
    """Spiking ResNet-50 with multi-step LIF (tau 2, v_th 1, hard reset to 0
    by default, as BASELINE config 3)."""
    return SpikingResNet([3, 4, 6, 3], T=T, num_classes=num_classes, width=width,
                         neuron={"tau": tau, "v_threshold": v_threshold, "v_reset": v_reset})


def fold_bn_(model: nn.Module) -> nn.Module:
    """Fold every BatchNorm2d into the Conv2d it follows (eval semantics,
    torch.nn.utils.fusion.fuse_conv_bn_eval, as the reference's benchmark
    does before timing), in place; the BN modules become Identity."""
    from torch.nn.utils.fusion import fuse_conv_bn_eval

    model.eval()
    pairs = []
    for mod in model.modules():
        if isinstance(mod, SpikingBottleneck):
            pairs += [(mod, "conv1", mod, "bn1"), (mod, "conv2", mod, "bn2"), (mod, "conv3", mod, "bn3")]
            if mod.downsample is not None:
                pairs.append((mod.downsample, "0", mod.downsample, "1"))
        elif isinstance(mod, SpikingResNet):
            pairs.append((mod, "conv1", mod, "bn1"))
    for cparent, cname, bparent, bname in pairs:
        conv, bn = getattr(cparent, cname), getattr(bparent, bname)
        if isinstance(bn, nn.BatchNorm2d):
            setattr(cparent, cname, fuse_conv_bn_eval(conv, bn))
            setattr(bparent, bname, nn.Identity())
    return model


def fuse_conv_lif_(model: nn.Module) -> int:
    """After optimize() and BN folding: run every bottleneck's 1x1 conv +
    LIF pair (conv1 -> sn1, and conv3 -> + identity -> sn3) as one fused
    kernel (Ops.sparse_fused_conv_lif.SparseConv1x1LIF), so the fp32 currents
    of those layers never round-trip through HBM.  Spikes equal the unfused
    model's up to threshold ties (the fused membrane update rounds
    differently).  Returns the number of fused pairs; in place."""
    from ..Ops.sparse_fused_conv_lif import SparseConv1x1LIF

    n = 0
    for mod in model.modules():
        if not isinstance(mod, SpikingBottleneck):
            continue
        if isinstance(mod.bn1, nn.Identity) and SparseConv1x1LIF.eligible(mod.conv1, mod.sn1):
            mod.conv1_lif = SparseConv1x1LIF(mod.conv1, mod.sn1)
            n += 1
        if isinstance(mod.bn3, nn.Identity) and SparseConv1x1LIF.eligible(mod.conv3, mod.sn3):
            mod.conv3_lif = SparseConv1x1LIF(mod.conv3, mod.sn3)
            n += 1
    return n


def _lif_density(I: torch.Tensor, node: LIFNode, v_th: float) -> float:
    """Spike density of `node`'s LIF dynamics on currents I [T, K] with
    threshold v_th (the membrane starts at v_reset, 0 for soft reset)."""
    vr = 0.0 if node.v_reset is None else float(node.v_reset)
    v = torch.full_like(I[0], vr)
    fired = torch.zeros((), dtype=torch.float64, device=I.device)
    for t in range(I.shape[0]):
        h = v + (I[t] - (v - vr)) / node.tau if node.decay_input else v - (v - vr) / node.tau + I[t]
        s = h >= v_th
        fired += s.sum()
        v = torch.where(s, torch.full_like(h, vr), h) if node.v_reset is not None else h - s.float() * v_th
    return float(fired) / I.numel()


def calibrate_lif_thresholds_(model: nn.Module, img: torch.Tensor, target_density: float = 0.01,
                              sample: int = 1 << 20, iters: int = 28, seed: int = 0) -> dict:
    """Set every LIFNode's v_threshold so that its spike density on `img` is
    `target_density`, in place; returns {layer name: (v_threshold, density)}.

    Random-initialised spiking networks are nearly silent past the first
    neuron layer at v_threshold = 1 (the density dies out layer by layer), so
    the sparse kernels would only ever see all-zero input.  The reference's
    own harness varies the thresholds to vary sparsity
    (Benchmark/run-resnet50.sh:16-64, v_threshold in {1.0, 0.75, 0.5, 0.25});
    this calibrates each layer instead: one forward in network order, a
    pre-hook on each neuron layer bisects the threshold on its input currents
    (x, plus the residual where one is added) over a fixed random sample of
    `sample` neurons, so every layer is calibrated on the spikes of the
    already calibrated layers before it.  The LIF dynamics are elementwise,
    so a neuron sample gives the layer's density to ~1/sqrt(sample)."""
    names = {m: n for n, m in model.named_modules() if isinstance(m, LIFNode)}
    gen = torch.Generator(device=img.device).manual_seed(seed)
    result = {}

    def pre(mod, args):
        cur = args[0].float()
        if len(args) > 1 and args[1] is not None:
            cur = cur + args[1].float()
        flat = cur.reshape(cur.shape[0], -1)
        if flat.shape[1] > sample:
            idx = torch.randint(0, flat.shape[1], (sample,), generator=gen, device=flat.device)
            flat = flat[:, idx]
        lo, hi = 0.0, float(flat.abs().max()) + 1.0
        for _ in range(iters):
            mid = 0.5 * (lo + hi)
            if _lif_density(flat, mod, mid) > target_density:
                lo = mid
            else:
                hi = mid
        mod.v_threshold = hi
        result[names[mod]] = (hi, _lif_density(flat, mod, hi))

    hooks = [m.register_forward_pre_hook(pre) for m in names]
    try:
        with torch.no_grad():
            from ..neuron import reset_net
            reset_net(model)
            model(img)
            reset_net(model)
    finally:
        for h in hooks:
            h.remove()
    return result

