"""Spiking-ResNet50 end to end on the GPU: the optimized model (SparseConv2d
on every eligible conv, library LIF kernel in every neuron layer) against
the same model with dense F.conv2d (MIOpen) convolutions.  Spikes of every
neuron layer agree except at threshold ties (fp32 rounding of two different
conv summation orders), and the logits agree."""

import copy

import pytest
import torch

import sparseflow_amd as sf
from sparseflow_amd.Models import fold_bn_, spiking_resnet50
from sparseflow_amd.neuron import LIFNode, reset_net
from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d
from tests.gpu_helpers import DEV, announce, native_loaded

pytestmark = pytest.mark.gpu


def _record(model):
    outs, hooks = {}, []
    for name, mod in model.named_modules():
        if isinstance(mod, LIFNode):
            hooks.append(mod.register_forward_hook(lambda _m, _i, o, n=name: outs.__setitem__(n, o.detach().clone())))
    return outs, hooks


@pytest.mark.parametrize("T,N,H,gain", [(2, 2, 64, 3.0), (4, 1, 112, 3.0)])
def test_resnet50_optimized_matches_dense(T, N, H, gain):
    announce(f"resnet50 e2e T={T} N={N} H={H}")
    torch.manual_seed(0)
    dense = spiking_resnet50(T=T, num_classes=10)
    with torch.no_grad():
        for mod in dense.modules():  # livelier spikes than the plain init
            if isinstance(mod, torch.nn.Conv2d):
                mod.weight.mul_(gain)
    dense = fold_bn_(dense).to(DEV)
    opt = copy.deepcopy(dense)
    x = torch.randn(N, 3, H, H, generator=torch.Generator().manual_seed(1)).to(DEV)
    sf.optimize(opt, sample_input=x, verbose=False)
    assert sum(isinstance(m, SparseConv2d) for m in opt.modules()) > 0
    rec_d, hd = _record(dense)
    rec_o, ho = _record(opt)
    with torch.no_grad():
        for m in (dense, opt):
            reset_net(m)
        ref = dense(x)
        out = opt(x)
    torch.cuda.synchronize()
    for h in hd + ho:
        h.remove()
    active = 0.0
    for name, s_ref in rec_d.items():
        s = rec_o[name]
        assert s.shape == s_ref.shape
        agree = (s == s_ref).float().mean().item()
        assert agree > 0.999, f"{name}: spikes agree on {agree:.5f}"
        active = max(active, s_ref.float().mean().item())
    assert active > 0.01  # the network actually spikes
    assert torch.allclose(out, ref, atol=1e-3, rtol=1e-3), (out - ref).abs().max()
    assert native_loaded()
