"""Pin the CPU oracle before trusting it (CPU only).

Each restatement in oracle/ is checked against something it was not derived
from: an independent brute-force loop, the torch library routine the
reference itself calls, or a closed form.  A plausible slip (wrong pool
padding, off-by-one tile edge, dropped group, wrong compare precision,
transposed weight, wrong LIF association) fails at least one test here.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute, conv as oconv, lif as olif, prescan as op

RNG = np.random.default_rng(1234)


def _spikes(shape, p, rng=RNG):
    return (rng.random(shape) < p).astype(np.float32)


# ---------------------------------------------------------------------------
# Prescan restatement vs brute force
# ---------------------------------------------------------------------------

GEOMS = [
    # (N, C, H, W, k, s, p, th, tw, gs)
    (2, 5, 7, 9, 3, 1, 1, 4, 4, 2),
    (1, 33, 10, 10, 3, 1, 1, 8, 8, 16),
    (2, 20, 9, 11, 3, 2, 1, 3, 4, 4),
    (1, 7, 6, 5, 1, 1, 0, 4, 2, 4),
    (1, 12, 13, 8, 3, 1, 1, 8, 16, 4),  # tile larger than the map
    (3, 3, 5, 5, 3, 2, 1, 2, 2, 1),
]


@pytest.mark.parametrize("geom", GEOMS)
@pytest.mark.parametrize("density", [0.0, 0.03, 0.3, 1.0])
def test_prescan_cascade_matches_brute_force(geom, density):
    N, C, H, W, k, s, p, th, tw, gs = geom
    x = _spikes((N, C, H, W), density)
    ng = -(-C // gs)
    ag, tc, _ = op.prescan_2d(x, k, s, p, th, tw, gs, ng, 1e-6)
    ag_b, tc_b = brute.prescan_tiles(x.tolist(), k, s, p, th, tw, gs, 1e-6)
    assert ag.tolist() == ag_b
    assert tc.tolist() == tc_b


def test_prescan_values_near_threshold_and_nan():
    # Non-binary magnitudes around the fp16 threshold boundary and a NaN.
    vals = np.array([0.0, 1e-6, 1.0133e-6, 1.04e-6, 1.05e-6, -2e-6, 3.0, np.nan], np.float32)
    x = RNG.choice(vals, size=(2, 6, 6, 7)).astype(np.float32)
    for (k, s, p) in [(3, 1, 1), (3, 2, 1), (1, 1, 0)]:
        ag, tc, _ = op.prescan_2d(x, k, s, p, 2, 3, 2, 3, 1e-6)
        ag_b, tc_b = brute.prescan_tiles(x.tolist(), k, s, p, 2, 3, 2, 1e-6)
        assert ag.tolist() == ag_b
        assert tc.tolist() == tc_b


def test_bit31_group_wraps_negative():
    C = 32 * 16  # 32 groups of 16
    x = np.zeros((1, C, 8, 8), np.float32)
    x[0, C - 1, 3, 3] = 1.0
    ag, tc, _ = op.prescan_2d(x, 3, 1, 1, 8, 8, 16, 32, 1e-6)
    assert ag.tolist() == [-(1 << 31)]
    assert tc.tolist() == [1]


# ---------------------------------------------------------------------------
# Pooling and comparison semantics vs the torch routines the reference calls
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("k,s,p", [(3, 1, 1), (3, 2, 1), (2, 2, 0)])
def test_rf_pool_matches_torch_max_pool2d(k, s, p):
    a = RNG.standard_normal((2, 3, 11, 9)).astype(np.float32)
    a[0, 1, 2, 2] = np.nan
    got = op._max_pool(a, k, k, s, s, p, p)
    ref = F.max_pool2d(torch.from_numpy(a), kernel_size=k, stride=s, padding=p).numpy()
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("bh,bw", [(8, 8), (8, 16), (4, 4), (3, 5)])
def test_tile_pool_ceil_mode_matches_torch(bh, bw):
    a = RNG.standard_normal((2, 4, 13, 29)).astype(np.float32)
    got = op._max_pool(a, bh, bw, bh, bw, 0, 0, ceil_mode=True)
    ref = F.max_pool2d(torch.from_numpy(a), kernel_size=(bh, bw), stride=(bh, bw), ceil_mode=True).numpy()
    np.testing.assert_array_equal(got, ref)


def test_fp16_compare_matches_torch_half_tensor_vs_python_float():
    # The reference compares an fp16 tensor with a Python float
    # (Kernels/_prescan_common.py:188); torch does it in fp16.
    mags = np.concatenate([
        np.linspace(0.9e-6, 1.2e-6, 4001, dtype=np.float32),
        np.array([0, 2.0 ** -25, 2.0 ** -24, 1.0, 65504.0, 7e4], np.float32),
    ])
    for thr in [1e-6, 0.0, 5e-7, 1e-3, 0.5]:
        ref = (torch.from_numpy(mags).half() > thr).numpy()
        got = op.active_elements(mags, thr)
        np.testing.assert_array_equal(got, ref)


def test_group_size_rule_table():
    table = {1: 16, 64: 16, 128: 16, 129: 32, 256: 32, 512: 32, 1024: 32, 1025: 64, 2048: 64, 4096: 128}
    for c, gs in table.items():
        assert op.choose_group_size(c) == gs
        assert -(-c // gs) <= 32


def test_block_rule_table():
    assert [op.select_block_size(h) for h in (224, 56, 32, 31, 28, 16, 15, 14, 8, 7, 1)] == \
        [16, 16, 16, 8, 8, 8, 4, 4, 4, None, None]


def test_tile_sizes_rule():
    assert op.select_tile_sizes(56, 56) == (8, 16)
    assert op.select_tile_sizes(28, 28) == (8, 8)
    assert op.select_tile_sizes(56, 55) == (8, 8)  # 3080 < 3136


def test_bitmap_layout_roundtrip():
    x = _spikes((2, 70, 5, 6), 0.2)
    bits = op.bitmap(x, 1e-6)
    assert bits.shape == (2, 30, 4)  # ceil(70/32)=3 -> padded to 4 words
    unpacked = np.zeros((2, 128, 30), np.float32)
    for c in range(128):
        unpacked[:, c] = (bits[:, :, c // 32] >> np.uint32(c % 32)) & 1
    np.testing.assert_array_equal(unpacked[:, :70], x.reshape(2, 70, 30))
    assert not unpacked[:, 70:].any()


def test_channel_lists_agree_with_group_size_one_masks():
    x = _spikes((2, 40, 9, 9), 0.02)
    mask, count, lists = op.tile_channel_lists(x, 3, 1, 1, 4, 4, 1e-6)
    _, _, act = op.prescan_2d(x, 3, 1, 1, 4, 4, 1, 40, 1e-6)
    act = act.reshape(-1, 40)
    for t in range(act.shape[0]):
        assert lists[t].tolist() == [c for c in range(40) if act[t, c]]
        assert count[t] == len(lists[t])
        assert sum(bin(int(w)).count("1") for w in mask[t]) == count[t]


# ---------------------------------------------------------------------------
# Conv reference
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("k,s,p", [(3, 1, 1), (3, 2, 1), (1, 1, 0)])
def test_conv_ref_matches_brute_force(k, s, p):
    x = _spikes((2, 3, 5, 6), 0.3) * RNG.standard_normal((2, 3, 5, 6)).astype(np.float32)
    w = RNG.standard_normal((4, 3, k, k)).astype(np.float32)
    b = RNG.standard_normal(4).astype(np.float32)
    y = oconv.conv2d_ref(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b), s, p).numpy()
    yb = np.array(brute.conv2d(x.tolist(), w.tolist(), b.tolist(), s, p))
    np.testing.assert_allclose(y, yb, rtol=1e-12, atol=1e-12)
    n, co, oh, ow = 1, 2, y.shape[2] - 1, 0
    assert math.isclose(oconv.conv2d_at(x, w, b, s, p, n, co, oh, ow), y[n, co, oh, ow], rel_tol=1e-12)


def test_conv_of_binary_spikes_is_a_sum_of_weight_taps():
    x = np.zeros((1, 2, 4, 4), np.float32)
    x[0, 0, 1, 1] = 1.0
    x[0, 1, 2, 3] = 1.0
    w = RNG.standard_normal((3, 2, 3, 3)).astype(np.float32)
    y = oconv.conv2d_ref(torch.from_numpy(x), torch.from_numpy(w), None, 1, 1).numpy()
    # Output (co, 1, 2) sees (ci=0,(1,1)) at tap (1,0) and (ci=1,(2,3)) at tap (2,2).
    w64 = w.astype(np.float64)
    np.testing.assert_allclose(y[0, :, 1, 2], w64[:, 0, 1, 0] + w64[:, 1, 2, 2], rtol=0, atol=1e-15)


def test_masked_input_drops_subthreshold_values():
    x = torch.tensor([[[[1.0, 1e-7, -3e-6, 1.03e-6]]]])
    m = oconv.masked_input(x, 1e-6)
    assert m.flatten().tolist() == pytest.approx([1.0, 0.0, -3e-6, 0.0])


# ---------------------------------------------------------------------------
# LIF reference
# ---------------------------------------------------------------------------

def test_lif_constant_current_closed_form():
    # Decay-input LIF with V_r = 0 and constant I: V_t = I * (1 - (1 - 1/tau)^t)
    # until the first spike.
    tau, I = 2.0, 0.9
    I_seq = np.full((6, 1), I, np.float64)
    spk, V, H = olif.lif_multistep(I_seq, tau=tau, v_th=1.0, v_reset=0.0, dtype=np.float64)
    expect = [I * (1 - (1 - 1 / tau) ** (t + 1)) for t in range(6)]
    np.testing.assert_allclose(H[:, 0], expect, rtol=1e-12)
    assert not spk.any()


def test_lif_hard_and_soft_reset_and_no_decay():
    I_seq = np.array([[1.5], [0.6], [0.9]], np.float64)
    spk, V, H = olif.lif_multistep(I_seq, tau=2.0, v_th=1.0, v_reset=0.0, dtype=np.float64)
    # H1 = 0.75 (no spike), H2 = 0.75 + (0.6-0.75)/2 = 0.675, H3 = 0.675 + (0.9-0.675)/2 = 0.7875
    np.testing.assert_allclose(H[:, 0], [0.75, 0.675, 0.7875])
    spk, V, H = olif.lif_multistep(np.array([[3.0], [0.0]]), tau=1.0, v_th=1.0, v_reset=None, dtype=np.float64)
    # tau=1: H = I; soft reset keeps the excess above threshold.
    assert spk[:, 0].tolist() == [True, False]
    np.testing.assert_allclose(H[:, 0], [3.0, 0.0])
    spk, V, H = olif.lif_multistep(np.array([[0.5], [0.5]]), tau=2.0, v_th=1.0, v_reset=0.0,
                                   decay_input=False, dtype=np.float64)
    # H1 = 0 - 0 + 0.5; H2 = 0.5 - 0.25 + 0.5 = 0.75
    np.testing.assert_allclose(H[:, 0], [0.5, 0.75])


# Hand-derived trajectories in which the post-reset membrane decides the next
# step (tau = 2, V_0 = 0 unless given).  Each row: (kwargs, I sequence,
# expected spikes, expected H, expected V_T).
#   hard, v_reset=-0.2: H1 = (3 - (0 + 0.2)) / 2 = 1.4 -> spike, V1 = -0.2;
#                       H2 = -0.2 + (0 - 0) / 2 = -0.2, V_T = -0.2
#   soft:               H1 = 3 / 2 = 1.5 -> spike, V1 = 0.5;
#                       H2 = 0.5 + (0 - 0.5) / 2 = 0.25, V_T = 0.25
#   hard, no decay_input, v_reset=0.1:
#                       H1 = 0 - (0 - 0.1) / 2 + 1.2 = 1.25 -> spike, V1 = 0.1;
#                       H2 = 0.1 - 0 + 0.3 = 0.4, V_T = 0.4
#   soft, no decay_input: H1 = 1.5 -> spike, V1 = 0.5;
#                       H2 = 0.5 - 0.25 + 0.2 = 0.45, V_T = 0.45
#   hard, v_reset=0, V_0 = 0.6: H1 = 0.6 + (1.6 - 0.6) / 2 = 1.1 -> spike,
#                       V1 = 0; H2 = 0 + (1.0 - 0) / 2 = 0.5, V_T = 0.5
#   hard, v_reset=0.5, two spikes: H1 = (4 - (0 - 0.5)) / 2 = 2.25, V1 = 0.5;
#                       H2 = 0.5 + (2 - 0) / 2 = 1.5, V2 = 0.5;
#                       H3 = 0.5 + (0 - 0) / 2 = 0.5, V_T = 0.5
LIF_RESET_CASES = [
    (dict(v_reset=-0.2), [3.0, 0.0], [True, False], [1.4, -0.2], -0.2, None),
    (dict(v_reset=None), [3.0, 0.0], [True, False], [1.5, 0.25], 0.25, None),
    (dict(v_reset=0.1, decay_input=False), [1.2, 0.3], [True, False], [1.25, 0.4], 0.4, None),
    (dict(v_reset=None, decay_input=False), [1.5, 0.2], [True, False], [1.5, 0.45], 0.45, None),
    (dict(v_reset=0.0), [1.6, 1.0], [True, False], [1.1, 0.5], 0.5, 0.6),
    (dict(v_reset=0.5), [4.0, 2.0, 0.0], [True, True, False], [2.25, 1.5, 0.5], 0.5, None),
]


def _lif_case_failures(step_fn):
    """Run every reset case through a multistep loop over `step_fn` (the
    oracle's lif_step or a planted mistake); return the failing cases."""
    failures = []
    for kw, I, s_exp, h_exp, v_exp, v0 in LIF_RESET_CASES:
        V = np.full((1,), 0.0 if v0 is None else v0, np.float64)
        S_all, H_all = [], []
        for i in I:
            S, V, H = step_fn(np.array([i]), V, 2.0, 1.0, kw["v_reset"], kw.get("decay_input", True), np.float64)
            S_all.append(bool(S[0]))
            H_all.append(float(H[0]))
        if S_all != s_exp or not np.allclose(H_all, h_exp, rtol=0, atol=1e-12) or abs(V[0] - v_exp) > 1e-12:
            failures.append((kw, I))
    return failures


def test_lif_reset_trajectories_closed_form():
    assert _lif_case_failures(olif.lif_step) == []
    for kw, I, s_exp, h_exp, v_exp, v0 in LIF_RESET_CASES:
        v0a = None if v0 is None else np.array([v0])
        spk, V, H = olif.lif_multistep(np.array(I)[:, None], tau=2.0, v_th=1.0, v_reset=kw["v_reset"],
                                       decay_input=kw.get("decay_input", True), v0=v0a, dtype=np.float64)
        assert spk[:, 0].tolist() == s_exp
        np.testing.assert_allclose(H[:, 0], h_exp, rtol=0, atol=1e-12)
        assert abs(float(V[0]) - v_exp) <= 1e-12


def _mutant(kind):
    """lif_step with one planted reset mistake (CPU only)."""
    def step(I, V, tau, v_th, v_reset, decay_input=True, dtype=np.float64):
        I = np.asarray(I, dtype=dtype)
        V = np.asarray(V, dtype=dtype)
        vr = 0.0 if v_reset is None else v_reset
        H = V + (I - (V - vr)) / tau if decay_input else (V - (V - vr) / tau) + I
        S = H >= v_th
        if kind == "hard_reset_to_zero":
            Vn = H - S * v_th if v_reset is None else np.where(S, 0.0, H)
        elif kind == "no_hard_reset":
            Vn = H - S * v_th if v_reset is None else H
        elif kind == "always_soft_reset":
            Vn = H - S * v_th
        elif kind == "soft_reset_to_zero":
            Vn = np.where(S, 0.0, H)
        else:
            raise ValueError(kind)
        return S, Vn.astype(dtype), H
    return step


@pytest.mark.parametrize("kind", ["hard_reset_to_zero", "no_hard_reset", "always_soft_reset",
                                  "soft_reset_to_zero"])
def test_lif_reset_cases_catch_planted_mistakes(kind):
    assert _lif_case_failures(_mutant(kind)), f"mutation {kind} passes the closed-form reset cases"


def test_compare_spikes_tie_rule():
    ref = np.array([[True], [False]])
    H = np.array([[1.0 + 1e-7], [0.2]])
    test = np.array([[False], [True]])
    bad, comparable = olif.compare_spikes(test, ref, H, 1.0)
    assert bad == 0  # first flip is a tie; the neuron then drops out
    assert comparable.tolist() == [[True], [False]]
