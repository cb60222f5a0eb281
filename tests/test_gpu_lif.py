"""Fused conv + multi-step LIF on the GPU vs the oracle.

Spikes must match exactly except at threshold ties (|H_ref - V_th| <= 1e-5
with H_ref from float64 currents); a neuron whose spike flips at a tie is
excluded from later steps.  Membranes of comparable neurons match within
1e-4 abs + 1e-4 rel.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import conv as oconv, lif as olif
from sparseflow_amd.Kernels.fused_conv_lif import sparse_fused_conv_lif_forward, sparse_fused_conv_lif_multistep
from sparseflow_amd.neuron import LIFNode
from sparseflow_amd.Ops.sparse_fused_conv_lif import FusedSparseConvLIF
from tests.gpu_helpers import DEV, announce, native_loaded, spikes

pytestmark = pytest.mark.gpu


def _currents(x, w, b, k):
    p = (k - 1) // 2
    return np.stack([oconv.conv2d_ref(x[t], w, b, 1, p).numpy() for t in range(x.shape[0])])


def _check(spk, v, x, w, b, k, tau, v_th, v_reset, decay_input, v0=None):
    I = _currents(x, w, b, k)
    s_ref, v_ref, h_ref = olif.lif_multistep(I, tau, v_th, v_reset, decay_input,
                                             v0=None if v0 is None else v0.double().numpy(), dtype=np.float64)
    bad, comparable = olif.compare_spikes(spk.cpu().numpy() > 0.5, s_ref, h_ref, v_th)
    assert bad == 0, f"{bad} spike mismatches away from threshold ties"
    alive = comparable[-1] & ~(((spk.cpu().numpy() > 0.5) != s_ref)[-1])
    vg = v.double().cpu().numpy()
    err = np.abs(vg - v_ref)[alive]
    assert (err <= 1e-4 + 1e-4 * np.abs(v_ref[alive])).all(), f"max membrane err {err.max()}"
    assert alive.mean() > 0.99


LIF_CASES = [
    # (T, N, C, H, W, Co, k, density, tau, v_th, v_reset, decay_input, bias, weight gain)
    (4, 2, 64, 16, 16, 64, 3, 0.05, 2.0, 1.0, 0.0, True, True, 1.0),
    (6, 3, 32, 12, 10, 96, 3, 0.1, 1.5, 0.5, 0.0, False, False, 1.0),
    (5, 2, 48, 9, 9, 64, 3, 0.1, 2.0, 1.0, None, True, True, 1.0),     # soft reset
    (3, 2, 64, 10, 10, 130, 3, 0.05, 3.0, 0.8, -0.2, True, True, 4.0),  # ragged C_out, v_reset != 0
    (4, 2, 128, 14, 14, 64, 1, 0.05, 2.0, 1.0, 0.0, True, True, 3.0),   # 1x1
]


@pytest.mark.parametrize("case", LIF_CASES)
def test_fused_lif_matches_oracle(case):
    T, N, C, H, W, Co, k, dens, tau, v_th, v_reset, decay_input, has_b, gain = case
    announce(f"lif {case}")
    x = spikes((T, N, C, H, W), dens, seed=T * 100 + C)
    g = torch.Generator().manual_seed(C)
    w = torch.randn(Co, C, k, k, generator=g) * (4.0 / (C * k * k)) ** 0.5 * gain
    b = torch.randn(Co, generator=g) * 0.2 if has_b else None
    spk, v, _ = sparse_fused_conv_lif_multistep(x.to(DEV), w.to(DEV), None if b is None else b.to(DEV), tau=tau,
                                                v_threshold=v_th, v_reset=v_reset, decay_input=decay_input,
                                                kernel_size=k)
    torch.cuda.synchronize()
    assert spk.shape == (T, N, Co, H, W) and v.shape == (N, Co, H, W)
    assert spk.float().mean() > 0.0  # the case exercises firing
    _check(spk, v, x, w, b, k, tau, v_th, v_reset, decay_input)
    assert native_loaded()


def test_fused_lif_v_init_and_single_step_chain():
    T, N, C, H, W, Co = 4, 2, 32, 8, 8, 64
    x = spikes((T, N, C, H, W), 0.15, seed=7)
    w = torch.randn(Co, C, 3, 3, generator=torch.Generator().manual_seed(1)) * 0.3
    v0 = torch.rand(N, Co, H, W, generator=torch.Generator().manual_seed(2)) * 0.9
    announce("lif v_init chain")
    spk, v, _ = sparse_fused_conv_lif_multistep(x.to(DEV), w.to(DEV), None, v_init=v0.to(DEV))
    _check(spk, v, x, w, None, 3, 2.0, 1.0, 0.0, True, v0=v0)
    # The single-step drop-in chained T times gives the same result bitwise.
    vs = v0.to(DEV)
    for t in range(T):
        s_t, vs, _ = sparse_fused_conv_lif_forward(x[t].to(DEV), vs, w.to(DEV), None)
        assert torch.equal(s_t, spk[t])
    assert torch.equal(vs, v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_lif_half_input(dtype):
    # 12x12 planes and full 32-channel slices: the four-pixel vector spike
    # stores in f16 / bf16.
    x = spikes((3, 2, 64, 12, 12), 0.05, seed=5)
    w = torch.randn(64, 64, 3, 3, generator=torch.Generator().manual_seed(4)) * 0.25
    announce(f"lif {dtype}")
    spk, v, _ = sparse_fused_conv_lif_multistep(x.to(DEV, dtype), w.to(DEV), None)
    assert spk.dtype == dtype and v.dtype == torch.float32
    _check(spk.float(), v, x, w, None, 3, 2.0, 1.0, 0.0, True)


def test_fused_lif_golden_fixture():
    from tests.golden import load_golden

    g = load_golden("lif_golden.npz")
    tau, v_th, v_reset = (float(t) for t in g["params"])
    announce("golden lif")
    spk, v, _ = sparse_fused_conv_lif_multistep(torch.from_numpy(g["x"]).to(DEV), torch.from_numpy(g["w"]).to(DEV),
                                                torch.from_numpy(g["b"]).to(DEV), tau=tau, v_threshold=v_th,
                                                v_reset=v_reset)
    bad, _ = olif.compare_spikes(spk.cpu().numpy() > 0.5, g["spikes"], g["h"], v_th)
    assert bad == 0


def test_module_multistep_and_state():
    conv = nn.Conv2d(32, 64, 3, 1, 1, bias=True)
    lif = LIFNode(tau=2.0, v_threshold=1.0, v_reset=0.0)
    mod = FusedSparseConvLIF.from_conv_and_lif(conv, lif).to(DEV)
    x = spikes((6, 2, 32, 10, 10), 0.2, seed=3).to(DEV)
    announce("lif module")
    with torch.no_grad():
        s_all = mod(x)
        v_all = mod.v.clone()
        mod.reset()
        s_a = mod(x[:3])
        s_b = mod(x[3:])           # state carried from the first call
        assert torch.equal(torch.cat([s_a, s_b]), s_all)
        assert torch.equal(mod.v, v_all)
        mod.reset()
        s_steps = torch.stack([mod(x[t]) for t in range(6)])  # 4-D single-step calls
        assert torch.equal(s_steps, s_all)
    # Host module (reference CPU path) agrees up to threshold ties.
    mod_cpu = FusedSparseConvLIF.from_conv_and_lif(conv, lif)
    with torch.no_grad():
        s_cpu = mod_cpu(x.cpu())
    assert (s_cpu != s_all.cpu()).float().mean() < 1e-3


def test_config4_full_size_sampled():
    """BASELINE config 4 at full size; exact oracle trajectories at sampled
    neurons (size-independent check)."""
    T, N, C, H, W, Co = 8, 64, 128, 28, 28, 128
    x = spikes((T, N, C, H, W), 0.005, seed=44)
    w = torch.randn(Co, C, 3, 3, generator=torch.Generator().manual_seed(45)) * (2.0 / (C * 9)) ** 0.5 * 6
    announce("config4 full size")
    spk, v, _ = sparse_fused_conv_lif_multistep(x.to(DEV), w.to(DEV), None)
    torch.cuda.synchronize()
    spk_c, v_c = spk.cpu().numpy(), v.cpu().numpy()
    assert spk_c.mean() > 0
    xn, wn = x.numpy(), w.numpy()
    rng = np.random.default_rng(0)
    for _ in range(64):
        n, co, oh, ow = (int(rng.integers(N)), int(rng.integers(Co)), int(rng.integers(H)), int(rng.integers(W)))
        I = np.array([[oconv.conv2d_at(xn[t], wn, None, 1, 1, n, co, oh, ow)] for t in range(T)])
        s_ref, v_ref, h_ref = olif.lif_multistep(I, dtype=np.float64)
        bad, comparable = olif.compare_spikes(spk_c[:, n, co, oh, ow][:, None] > 0.5, s_ref, h_ref, 1.0)
        assert bad == 0
        if comparable[-1, 0]:
            assert abs(v_c[n, co, oh, ow] - v_ref[0]) <= 1e-4 + 1e-4 * abs(v_ref[0])


def _lif_kernels(fn):
    from sparseflow_amd import _lib

    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        out = fn()
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return out, {k: c for k, (c, _) in stats.items() if c > 0}


PX_LIF_CASES = [
    # (T, N, C, H, W, Co, density, v_reset, decay_input, gain): 3x3 with C_out % 4 == 0 runs the pixel-tile kernel
    (4, 2, 64, 16, 16, 64, 0.05, 0.0, True, 1.0),     # two chunks
    (3, 3, 128, 14, 14, 128, 0.03, 0.0, True, 3.0),   # config-4 channel counts: four chunks resident
    (3, 2, 160, 9, 9, 64, 0.1, 0.0, False, 1.0),      # five chunks: streamed through two LDS buffers
    (5, 2, 33, 7, 11, 36, 0.1, None, True, 2.0),      # soft reset, ragged channel group, odd plane
    (2, 1, 1, 5, 5, 4, 0.5, -0.3, True, 6.0),         # one input channel
    (3, 2, 96, 11, 9, 40, 0.05, 0.0, True, 2.0),      # second 64-channel super-chunk of one word, ragged group
    (2, 3, 100, 12, 12, 32, 0.08, None, False, 2.0),  # last word partial, soft reset, vector spike stores
]


@pytest.mark.parametrize("case", PX_LIF_CASES)
def test_fused_lif_pixel_kernel(case):
    T, N, C, H, W, Co, dens, v_reset, decay_input, gain = case
    announce(f"lif px3 {case}")
    x = spikes((T, N, C, H, W), dens, seed=T * 10 + C)
    g = torch.Generator().manual_seed(C + Co)
    w = torch.randn(Co, C, 3, 3, generator=g) * (4.0 / (C * 9)) ** 0.5 * gain
    b = torch.randn(Co, generator=g) * 0.2
    (spk, v, _), kernels = _lif_kernels(lambda: sparse_fused_conv_lif_multistep(
        x.to(DEV), w.to(DEV), b.to(DEV), tau=2.0, v_threshold=1.0, v_reset=v_reset, decay_input=decay_input))
    assert "conv_lif_px3" in kernels and "conv_lif" not in kernels, kernels
    assert spk.float().mean() > 0.0
    _check(spk, v, x, w, b, 3, 2.0, 1.0, v_reset, decay_input)


def test_fused_lif_pixel_kernel_value_path():
    # Non-binary inputs in one sample's step: that tile multiplies by x.
    T, N, C, H, W, Co = 3, 2, 64, 10, 10, 64
    x = spikes((T, N, C, H, W), 0.1, seed=17)
    x[1, 0, :, 2:4] = x[1, 0, :, 2:4] * torch.rand(C, 2, W, generator=torch.Generator().manual_seed(18)) * 2
    w = torch.randn(Co, C, 3, 3, generator=torch.Generator().manual_seed(19)) * 0.3
    announce("lif px3 value path")
    (spk, v, _), kernels = _lif_kernels(lambda: sparse_fused_conv_lif_multistep(x.to(DEV), w.to(DEV), None))
    assert "conv_lif_px3" in kernels
    _check(spk, v, x, w, None, 3, 2.0, 1.0, 0.0, True)


def _random_lif_cases(n, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(n):
        T = int(torch.randint(1, 6, (1,), generator=g))
        N = int(torch.randint(1, 4, (1,), generator=g))
        C = int(torch.randint(1, 200, (1,), generator=g))
        Co = 4 * int(torch.randint(1, 30, (1,), generator=g))
        H = int(torch.randint(1, 20, (1,), generator=g))
        W = int(torch.randint(1, 24, (1,), generator=g))
        dens = [0.02, 0.1][int(torch.randint(0, 2, (1,), generator=g))]
        v_reset = [0.0, None, -0.3][int(torch.randint(0, 3, (1,), generator=g))]
        decay = bool(torch.randint(0, 2, (1,), generator=g))
        out.append((T, N, C, H, W, Co, dens, v_reset, decay))
    return out


@pytest.mark.parametrize("case", _random_lif_cases(24, 77))
def test_fused_lif_pixel_kernel_random_shapes(case):
    # Random geometry through the 3x3 fused conv-LIF (resident 64-channel
    # super-chunks for C_in <= 128, streamed 32-channel chunks beyond; ragged
    # channel groups; planes smaller than a tile; one wavefront per workgroup
    # for the smallest launches) against the float64 closed form.
    T, N, C, H, W, Co, dens, v_reset, decay_input = case
    announce(f"lif px3 random {case}")
    x = spikes((T, N, C, H, W), dens, seed=C * 3 + W)
    g = torch.Generator().manual_seed(C + Co + H)
    w = torch.randn(Co, C, 3, 3, generator=g) * (4.0 / (C * 9)) ** 0.5 * 3.0
    b = torch.randn(Co, generator=g) * 0.2
    (spk, v, _), kernels = _lif_kernels(lambda: sparse_fused_conv_lif_multistep(
        x.to(DEV), w.to(DEV), b.to(DEV), tau=2.0, v_threshold=1.0, v_reset=v_reset, decay_input=decay_input))
    assert "conv_lif_px3" in kernels, kernels
    _check(spk, v, x, w, b, 3, 2.0, 1.0, v_reset, decay_input)
