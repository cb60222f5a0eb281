"""Spikformer end to end on the GPU: the optimized model (SparseConv2d in the
patch embedding, SparseAttentionBlock with SparseLinear projections and the
fused spike-attention kernel, SparseLinear MLP and head) against the same model
with dense torch layers.  Every neuron layer's spikes agree except at
threshold ties (fp32 rounding of different summation orders, which can
cascade to a few downstream neurons), and the logits agree."""

import copy

import pytest
import torch

import sparseflow_amd as sf
from sparseflow_amd import _lib
from sparseflow_amd.Models import spikformer_cifar_4_384, spikformer_cifar_tiny
from sparseflow_amd.neuron import LIFNode, reset_net
from sparseflow_amd.Ops import SparseAttentionBlock, SparseConv2d, SparseLinear
from tests.gpu_helpers import DEV, announce, native_loaded

pytestmark = pytest.mark.gpu


def _lively(m, conv_gain=5.0, linear_gain=25.0):
    """Scale the random weights so every stage spikes (10-50% rates), and
    round the Linear weights to bf16 values: the matrix-core Linear then
    computes exact products (its bf16 hi + lo split of W is otherwise exact
    to ~2^-17, which moves a few threshold ties per layer and, through four
    blocks of 30-50% activity, the logits by more than summation order
    does)."""
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, torch.nn.Conv2d):
                mod.weight.mul_(conv_gain)
            elif isinstance(mod, torch.nn.Linear):
                mod.weight.mul_(linear_gain)
                mod.weight.copy_(mod.weight.to(torch.bfloat16).float())
    return m.eval()


def _record(model):
    outs, hooks = {}, []
    for name, mod in model.named_modules():
        if isinstance(mod, LIFNode):
            hooks.append(mod.register_forward_hook(lambda _m, _i, o, n=name: outs.__setitem__(n, o.detach().clone())))
    return outs, hooks


@pytest.mark.parametrize("builder,T,B", [(spikformer_cifar_tiny, 2, 2), (spikformer_cifar_4_384, 4, 2)])
def test_spikformer_optimized_matches_dense(builder, T, B):
    announce(f"spikformer {builder.__name__} T={T} B={B}")
    torch.manual_seed(0)
    dense = _lively(builder(T=T)).to(DEV)
    opt = copy.deepcopy(dense)
    x = torch.randn(B, 3, 32, 32, generator=torch.Generator().manual_seed(1)).to(DEV)
    sf.optimize(opt, sample_input=x, verbose=False)
    kinds = {type(m) for m in opt.modules()}
    assert {SparseConv2d, SparseLinear, SparseAttentionBlock} <= kinds
    with torch.no_grad():
        reset_net(dense)
        rec_d, hooks_d = _record(dense)
        ref = dense(x)
        for h in hooks_d:
            h.remove()
        reset_net(opt)
        rec, hooks = _record(opt)
        _lib.timing_reset()
        _lib.timing_enable(True)
        out = opt(x)
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
        _lib.timing_enable(False)
        for h in hooks:
            h.remove()
    launched = {k for k, (c, _) in stats.items() if c > 0}
    assert {"linear_mfma", "spike_attention"} <= launched, launched
    rates = {n: s.float().mean().item() for n, s in rec.items()}
    assert min(rates.values()) > 0.01, rates
    for name, s_ref in rec_d.items():
        agree = (rec[name] == s_ref).float().mean().item()
        assert agree > 0.99, f"{name}: spikes agree on {agree:.5f}"
    diff = (out - ref).abs().max().item()
    scale = ref.abs().max().item()
    assert diff <= 0.05 * max(scale, 1.0), (diff, scale)
    assert native_loaded()
