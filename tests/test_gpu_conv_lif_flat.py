"""Fused 1x1 conv + multi-step LIF (+ residual) with spike-map output
(sf_conv1x1_lif_sparse through Kernels.fused_conv_lif.sparse_conv1x1_lif_multistep),
and the Spiking-ResNet50 fusion built on it.

Bar: spikes equal the float64 closed form except at threshold ties
(|H_ref - v_th| <= 1e-5, a neuron dropped from its first legitimate flip),
membranes within 1e-4; the output spike map equals the prescan of the
spikes bit for bit with all flags zero."""

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import lif as olif
from oracle import prescan as opre
from sparseflow_amd import _lib
from sparseflow_amd.Kernels import spike_map
from sparseflow_amd.Kernels.fused_conv_lif import sparse_conv1x1_lif_multistep
from tests.gpu_helpers import DEV, announce, bits_numpy, native_loaded, spikes

pytestmark = pytest.mark.gpu

CASES = [
    # (T, N, C, H, W, Co, density, tau, v_th, v_reset, decay_input, bias, residual, gain)
    (4, 2, 64, 14, 14, 64, 0.1, 2.0, 1.0, 0.0, True, True, True, 3.0),
    (3, 2, 256, 7, 9, 128, 0.05, 2.0, 1.0, 0.0, True, False, True, 4.0),
    (2, 3, 96, 5, 13, 68, 0.2, 1.5, 0.5, None, True, True, False, 2.0),    # soft reset, ragged C_out
    (3, 2, 300, 6, 6, 32, 0.1, 2.0, 1.0, 0.0, False, True, True, 3.0),    # streamed weight chunks
    (2, 2, 40, 8, 8, 260, 0.2, 3.0, 0.8, -0.2, True, True, True, 3.0),    # v_reset != 0, 5 output groups
    (16, 2, 64, 56, 56, 256, 0.02, 2.0, 1.0, 0.0, True, False, True, 5.0),  # layer1 conv3 shape (fewer frames)
]


def _ref(x, w, b, res, tau, v_th, v_reset, decay_input, v0=None):
    T = x.shape[0]
    I = np.stack([oconv.sparse_conv2d_ref(x[t], w, b, 1, 0).numpy() for t in range(T)])
    if res is not None:
        I = I + res.double().numpy()
    return olif.lif_multistep(I, tau, v_th, v_reset, decay_input,
                              v0=None if v0 is None else v0.double().numpy(), dtype=np.float64)


def _check(spk, v, s_ref, v_ref, h_ref, v_th):
    bad, comparable = olif.compare_spikes(spk.cpu().numpy() > 0.5, s_ref, h_ref, v_th)
    assert bad == 0, f"{bad} spike mismatches away from threshold ties"
    alive = comparable[-1] & ~(((spk.cpu().numpy() > 0.5) != s_ref)[-1])
    err = np.abs(v.double().cpu().numpy() - v_ref)[alive]
    assert (err <= 1e-4 + 1e-4 * np.abs(v_ref[alive])).all(), f"max membrane err {err.max()}"
    assert alive.mean() > 0.99


@pytest.mark.parametrize("case", CASES)
def test_conv1x1_lif_matches_closed_form(case):
    T, N, C, H, W, Co, p, tau, v_th, v_reset, dec, has_b, has_r, gain = case
    announce(f"conv1x1 lif {case}")
    g = torch.Generator().manual_seed(C + Co)
    x = spikes((T, N, C, H, W), p, seed=T * 7 + C)
    w = torch.randn(Co, C, 1, 1, generator=g) * gain / C ** 0.5
    b = torch.randn(Co, generator=g) * 0.1 if has_b else None
    r = spikes((T, N, Co, H, W), 0.3, seed=Co) if has_r else None
    spike_map.clear()
    spk, v = sparse_conv1x1_lif_multistep(x.to(DEV), w.to(DEV), None if b is None else b.to(DEV), tau=tau,
                                          v_threshold=v_th, v_reset=v_reset, decay_input=dec,
                                          residual=None if r is None else r.to(DEV))
    torch.cuda.synchronize()
    s_ref, v_ref, h_ref = _ref(x, w, b, r, tau, v_th, v_reset, dec)
    _check(spk, v, s_ref, v_ref, h_ref, v_th)
    assert 0.0 < float(spk.float().mean()) < 1.0
    # The output spike map is the prescan of the spikes.
    handed = spike_map.lookup(spk.view(T * N, Co, H, W), 1e-6)
    assert handed is not None
    cwp = opre.words_per_pixel(Co)
    want = opre.bitmap(spk.view(T * N, Co, H, W).cpu().numpy(), 1e-6)
    assert np.array_equal(bits_numpy(handed[0], T * N, H * W, cwp), want)
    nfl = int(_lib.lib().sf_prescan_flags_bytes(T * N, Co, H, W)) // 4
    assert int(handed[1][:nfl].abs().sum()) == 0
    assert native_loaded()


def test_conv1x1_lif_value_input_v_init_and_handed_map():
    T, N, C, H, W, Co = 3, 2, 64, 10, 10, 64
    g = torch.Generator().manual_seed(5)
    x = spikes((T, N, C, H, W), 0.1, seed=6)
    x[1, 0, :, 3] = x[1, 0, :, 3] * 2.0          # non-binary chunk: the value path
    w = torch.randn(Co, C, 1, 1, generator=g) * 0.6
    v0 = torch.rand(N, Co, H, W, generator=g) * 0.5
    announce("conv1x1 lif value path + v_init")
    spike_map.clear()
    spk, v = sparse_conv1x1_lif_multistep(x.to(DEV), w.to(DEV), None, v_init=v0.to(DEV))
    s_ref, v_ref, h_ref = _ref(x, w, None, None, 2.0, 1.0, 0.0, True, v0=v0)
    _check(spk, v, s_ref, v_ref, h_ref, 1.0)
    # Chained: the spikes' handed map feeds a second fused layer, which must
    # give what it gives from a fresh prescan.
    w2 = torch.randn(32, Co, 1, 1, generator=g) * 0.8
    s2a, v2a = sparse_conv1x1_lif_multistep(spk, w2.to(DEV), None)
    s2b, v2b = sparse_conv1x1_lif_multistep(spk.clone(), w2.to(DEV), None)
    assert torch.equal(s2a, s2b) and torch.equal(v2a, v2b)


def test_resnet50_fused_matches_unfused():
    import copy

    import sparseflow_amd as sf
    from sparseflow_amd.Models import fold_bn_, fuse_conv_lif_, spiking_resnet50
    from sparseflow_amd.neuron import LIFNode, reset_net

    announce("resnet50 fused conv-LIF")
    torch.manual_seed(0)
    m = spiking_resnet50(T=2, num_classes=10)
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, torch.nn.Conv2d):
                mod.weight.mul_(3.0)
    m = fold_bn_(m).to(DEV)
    x = torch.randn(2, 3, 64, 64, generator=torch.Generator().manual_seed(1)).to(DEV)
    sf.optimize(m, sample_input=x, verbose=False)
    fused = copy.deepcopy(m)
    n_fused = fuse_conv_lif_(fused)
    assert n_fused >= 8

    def record(model):
        outs, hooks = {}, []
        for name, mod in model.named_modules():
            if isinstance(mod, LIFNode):
                hooks.append(mod.register_forward_hook(
                    lambda _m, _i, o, n=name: outs.__setitem__(n, o.detach().clone())))
        return outs, hooks

    with torch.no_grad():
        reset_net(m)
        ref = m(x)
        reset_net(fused)
        rec, hooks = record(fused)
        _lib.timing_reset()
        _lib.timing_enable(True)
        out = fused(x)
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
        _lib.timing_enable(False)
        for h in hooks:
            h.remove()
    # One fused launch per pair whose weights the kernel keeps resident; the
    # pairs with more input channels run as conv + neuron (at batch 2 none of
    # them has the samples to fill the GPU).
    from sparseflow_amd.Kernels.fused_conv_lif import CONV1X1_LIF_RESIDENT_CIN
    from sparseflow_amd.Ops.sparse_fused_conv_lif import SparseConv1x1LIF

    pairs = [mod for mod in fused.modules() if isinstance(mod, SparseConv1x1LIF)]
    assert len(pairs) == n_fused
    n_resident = sum(1 for mod in pairs if mod.conv.in_channels <= CONV1X1_LIF_RESIDENT_CIN)
    assert 0 < n_resident < n_fused
    assert stats["conv_lif_flat"][0] == n_resident
    assert torch.allclose(out, ref, atol=1e-2, rtol=1e-2), (out - ref).abs().max()
    assert any(float(s.float().mean()) > 0.01 for s in rec.values())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hw", [(12, 12), (7, 9)])
def test_conv1x1_lif_half_types_match_f32(dtype, hw):
    # Binary spikes and residual are exact in f16 / bf16 and the sum is f32,
    # so the spikes and the membrane equal the f32 run (vector-store path for
    # H*W % 4 == 0, per-channel stores otherwise).
    T, N, C, Co = 3, 2, 64, 128
    H, W = hw
    announce(f"conv1x1 lif {dtype} {hw}")
    g = torch.Generator().manual_seed(11)
    x = spikes((T, N, C, H, W), 0.15, seed=12)
    r = spikes((T, N, Co, H, W), 0.3, seed=13)
    w = torch.randn(Co, C, 1, 1, generator=g) * 0.5
    b = torch.randn(Co, generator=g) * 0.1
    spike_map.clear()
    s32, v32 = sparse_conv1x1_lif_multistep(x.to(DEV), w.to(DEV), b.to(DEV), residual=r.to(DEV))
    spike_map.clear()
    s16, v16 = sparse_conv1x1_lif_multistep(x.to(DEV, dtype), w.to(DEV), b.to(DEV), residual=r.to(DEV, dtype))
    torch.cuda.synchronize()
    assert s16.dtype == dtype
    assert torch.equal(s16.float(), s32) and torch.equal(v16, v32)
    assert 0.0 < float(s32.mean()) < 1.0


def test_conv1x1_lif_binary_residual_from_its_spike_map(monkeypatch):
    # A residual that is a registered spike tensor is read from its bitmap
    # (sf_conv1x1_lif_sparse_binres); the results equal the values path.
    T, N, C, H, W, Co = 3, 2, 64, 12, 12, 128
    announce("conv1x1 lif binary residual from its spike map")
    g = torch.Generator().manual_seed(21)
    x = spikes((T, N, C, H, W), 0.2, seed=22)
    w1 = torch.randn(Co, C, 1, 1, generator=g) * 0.6
    w2 = torch.randn(Co, C, 1, 1, generator=g) * 0.6
    b2 = torch.randn(Co, generator=g) * 0.1
    spike_map.clear()
    res, _ = sparse_conv1x1_lif_multistep(x.to(DEV), w1.to(DEV), None)   # registered spikes
    assert spike_map.lookup(res.view(T * N, Co, H, W), 1e-6) is not None
    assert 0.0 < float(res.mean()) < 1.0
    used = []
    real = _lib.conv1x1_lif_sparse

    def spy(*args, **kw):
        used.append(kw.get("res_bits") is not None)
        return real(*args, **kw)

    monkeypatch.setattr(_lib, "conv1x1_lif_sparse", spy)
    s_b, v_b = sparse_conv1x1_lif_multistep(x.to(DEV), w2.to(DEV), b2.to(DEV), residual=res)
    s_v, v_v = sparse_conv1x1_lif_multistep(x.to(DEV), w2.to(DEV), b2.to(DEV), residual=res.clone())
    torch.cuda.synchronize()
    assert used == [True, False]
    assert torch.equal(s_b, s_v) and torch.equal(v_b, v_v)
    s_ref, v_ref, h_ref = _ref(x, w2, b2, res.cpu(), 2.0, 1.0, 0.0, True)
    _check(s_b, v_b, s_ref, v_ref, h_ref, 1.0)


def _fused_pair(C, Co, v_reset, seed):
    from sparseflow_amd.neuron import LIFNode
    from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d
    from sparseflow_amd.Ops.sparse_fused_conv_lif import SparseConv1x1LIF

    g = torch.Generator().manual_seed(seed)
    conv = torch.nn.Conv2d(C, Co, 1, bias=True)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(Co, C, 1, 1, generator=g) * 0.7)
        conv.bias.copy_(torch.randn(Co, generator=g) * 0.1)
    sc = SparseConv2d.from_dense(conv).to(DEV)
    lif = LIFNode(step_mode="m", v_reset=v_reset)
    return SparseConv1x1LIF(sc, lif), sc, LIFNode(step_mode="m", v_reset=v_reset)


@pytest.mark.parametrize("v_reset", [0.0, -0.3])
def test_conv1x1_lif_module_batch_change_without_reset(v_reset):
    # Batch 2 then batch 4 with no reset_net in between: the fused module must
    # start the second call from a fresh membrane (as the unfused LIFNode
    # does on a new shape), not read the batch-2 membrane past its end.
    T, C, Co, H, W = 3, 64, 64, 8, 8
    announce(f"conv1x1 lif module batch 2 -> 4, v_reset={v_reset}")
    fused, conv, lif_ref = _fused_pair(C, Co, v_reset, seed=31)
    for N, seed in ((2, 32), (4, 33), (4, 34)):
        x = spikes((T, N, C, H, W), 0.2, seed=seed).to(DEV)
        spike_map.clear()
        s_f = fused(x)
        y = conv(x.flatten(0, 1)).reshape(T, N, Co, H, W)
        s_u = lif_ref(y)
        torch.cuda.synchronize()
        assert tuple(fused.lif.v.shape) == (N, Co, H, W)
        mism = float((s_f != s_u).float().mean())
        assert mism < 1e-3, f"N={N}: {mism} of spikes differ from the unfused pair"
        assert torch.allclose(fused.lif.v, lif_ref.v, atol=1e-4, rtol=1e-4)
        assert 0.0 < float(s_f.mean()) < 1.0


def test_conv1x1_lif_rejects_mismatched_v_init():
    T, N, C, H, W, Co = 2, 2, 32, 6, 6, 32
    x = spikes((T, N, C, H, W), 0.2, seed=41).to(DEV)
    w = torch.randn(Co, C, 1, 1).to(DEV)
    with pytest.raises(ValueError):
        sparse_conv1x1_lif_multistep(x, w, None, v_init=torch.zeros(N - 1, Co, H, W, device=DEV))
    with pytest.raises(ValueError):
        sparse_conv1x1_lif_multistep(x, w, None, v_init=torch.zeros(N, Co, H + 1, W, device=DEV))


def test_conv1x1_lif_module_honours_dense_dispatch():
    # A dispatch decision that puts the conv on the dense path runs the conv
    # and the neuron one after the other: no fused launch.
    T, N, C, Co, H, W = 2, 2, 64, 64, 8, 8
    announce("conv1x1 lif module with a dense dispatch decision")
    fused, conv, lif_ref = _fused_pair(C, Co, 0.0, seed=51)
    conv.backend_mode = "dense"
    x = spikes((T, N, C, H, W), 0.2, seed=52).to(DEV)
    _lib.timing_reset()
    _lib.timing_enable(True)
    s_f = fused(x)
    torch.cuda.synchronize()
    stats = _lib.timing_collect()
    _lib.timing_enable(False)
    assert stats.get("conv_lif_flat", (0,))[0] == 0
    s_u = lif_ref(conv(x.flatten(0, 1)).reshape(T, N, Co, H, W))
    assert torch.equal(s_f, s_u)


def test_conv1x1_lif_module_streamed_weights_run_as_pair():
    # C_in above the fused kernel's resident limit: the module runs the conv
    # over all frames and then the neuron (no fused launch), and its spikes
    # and membrane match the closed form.
    from sparseflow_amd.Kernels.fused_conv_lif import CONV1X1_LIF_RESIDENT_CIN

    T, N, C, Co, H, W = 3, 2, 512, 128, 7, 9
    assert C > CONV1X1_LIF_RESIDENT_CIN
    announce("conv1x1 lif module with streamed weights (C_in 512)")
    fused, conv, lif_ref = _fused_pair(C, Co, 0.0, seed=61)
    with torch.no_grad():
        conv.weight.mul_(4.0 / C ** 0.5)
    x = spikes((T, N, C, H, W), 0.05, seed=62).to(DEV)
    spike_map.clear()
    _lib.timing_reset()
    _lib.timing_enable(True)
    s_f = fused(x)
    torch.cuda.synchronize()
    stats = _lib.timing_collect()
    _lib.timing_enable(False)
    assert stats.get("conv_lif_flat", (0,))[0] == 0
    s_ref, v_ref, h_ref = _ref(x.cpu(), conv.weight.detach().cpu(), conv.bias.detach().cpu(), None,
                               2.0, 1.0, 0.0, True)
    _check(s_f, fused.lif.v, s_ref, v_ref, h_ref, 1.0)
    assert 0.0 < float(s_f.mean()) < 1.0

