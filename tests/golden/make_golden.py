"""Write the golden fixtures in this directory from the CPU oracle.

Every prescan case is cross-checked against the independent brute-force
form (oracle/brute.py) before it is written, so a fixture only exists if
the two restatements agree.  Run from the repo root:

    python -m tests.golden.make_golden
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import brute, conv as oconv, lif as olif, prescan as op
from tests.golden import GOLDEN_DIR

PRESCAN_CASES = [
    # (N, C, H, W, k, s, p, bh, bw, gs, density)
    (2, 64, 12, 12, 3, 1, 1, 8, 8, 16, 0.01),
    (1, 40, 9, 11, 3, 2, 1, 8, 8, 16, 0.05),
    (2, 48, 10, 10, 1, 1, 0, 8, 16, 16, 0.02),
    (1, 160, 8, 8, 3, 1, 1, 8, 8, 32, 0.01),
    (1, 16, 17, 9, 3, 1, 1, 4, 4, 16, 0.0),
]


def make_prescan(rng):
    out = {"count": np.int32(len(PRESCAN_CASES))}
    for i, (N, C, H, W, k, s, p, bh, bw, gs, dens) in enumerate(PRESCAN_CASES):
        x = (rng.random((N, C, H, W)) < dens).astype(np.float32)
        if i == 1:  # a few non-binary magnitudes near the fp16 threshold
            x[0, 0, 0, :4] = [1e-7, 1.04e-6, 1.05e-6, -0.25]
        ng = -(-C // gs)
        ag, tc, _ = op.prescan_2d(x, k, s, p, bh, bw, gs, ng, 1e-6)
        ag_b, tc_b = brute.prescan_tiles(x.tolist(), k, s, p, bh, bw, gs, 1e-6)
        assert ag.tolist() == ag_b and tc.tolist() == tc_b, f"oracle/brute disagree on case {i}"
        out[f"x{i}"] = x
        out[f"geom{i}"] = np.array([k, s, p, bh, bw, gs, ng], np.int32)
        out[f"ag{i}"] = ag
        out[f"tc{i}"] = tc
        out[f"bits{i}"] = op.bitmap(x, 1e-6)
    np.savez_compressed(GOLDEN_DIR / "prescan_golden.npz", **out)


CONV_CASES = [
    # (N, C, H, W, Cout, k, s, density, bias)
    (2, 8, 6, 7, 5, 3, 1, 0.1, True),
    (1, 20, 9, 9, 12, 3, 2, 0.05, False),
    (2, 33, 5, 5, 70, 1, 1, 0.2, True),
]


def make_conv(rng):
    out = {"count": np.int32(len(CONV_CASES))}
    for i, (N, C, H, W, Co, k, s, dens, has_b) in enumerate(CONV_CASES):
        p = (k - 1) // 2
        x = (rng.random((N, C, H, W)) < dens).astype(np.float32)
        w = (rng.standard_normal((Co, C, k, k)) * 0.2).astype(np.float32)
        b = (rng.standard_normal(Co) * 0.1).astype(np.float32) if has_b else None
        y = oconv.conv2d_ref(torch.from_numpy(x), torch.from_numpy(w), None if b is None else torch.from_numpy(b),
                             s, p).numpy()
        yb = np.array(brute.conv2d(x.tolist(), w.tolist(), None if b is None else b.tolist(), s, p))
        np.testing.assert_allclose(y, yb, rtol=1e-12, atol=1e-12)
        out[f"x{i}"] = x
        out[f"w{i}"] = w
        out[f"b{i}"] = b if b is not None else np.zeros(0, np.float32)
        out[f"geom{i}"] = np.array([k, s, p], np.int32)
        out[f"y{i}"] = y
    np.savez_compressed(GOLDEN_DIR / "conv_golden.npz", **out)


def make_lif(rng):
    T, N, C, H, W, Co = 4, 2, 16, 6, 6, 8
    x = (rng.random((T, N, C, H, W)) < 0.2).astype(np.float32)
    w = (rng.standard_normal((Co, C, 3, 3)) * 0.5).astype(np.float32)
    b = (rng.standard_normal(Co) * 0.2).astype(np.float32)
    I = np.stack([oconv.conv2d_ref(torch.from_numpy(x[t]), torch.from_numpy(w), torch.from_numpy(b), 1, 1).numpy()
                  for t in range(T)])
    spk, V, H_seq = olif.lif_multistep(I, tau=2.0, v_th=1.0, v_reset=0.0, decay_input=True, dtype=np.float64)
    np.savez_compressed(GOLDEN_DIR / "lif_golden.npz", x=x, w=w, b=b, spikes=spk, v=V, h=H_seq,
                        params=np.array([2.0, 1.0, 0.0], np.float64))


def main():
    rng = np.random.default_rng(20261201)
    make_prescan(rng)
    make_conv(rng)
    make_lif(rng)
    print("golden fixtures written to", GOLDEN_DIR)


if __name__ == "__main__":
    main()
