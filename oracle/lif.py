"""Multi-step LIF reference (test infrastructure only).

Closed form of the reference module's LIF step (Ops/sparse_fused_conv_lif.py:
283-292, spikingjelly LIFNode semantics):
  decay_input:      H = V + (I - (V - Vr)) / tau
  not decay_input:  H = V - (V - Vr) / tau + I
  S = [H >= V_th]
  hard reset:       V' = S ? V_reset : H
  soft reset:       V' = H - S * V_th        (Vr = 0 in the decay)
  V_0 = 0 (Ops/sparse_fused_conv_lif.py:202-203)
"""

from __future__ import annotations

from typing import Optional

import numpy as np


def lif_step(I, V, tau, v_th, v_reset: Optional[float], decay_input=True, dtype=np.float32):
    I = np.asarray(I, dtype=dtype)
    V = np.asarray(V, dtype=dtype)
    t = dtype(tau)
    vr = dtype(0.0 if v_reset is None else v_reset)
    if decay_input:
        H = V + (I - (V - vr)) / t
    else:
        H = (V - (V - vr) / t) + I
    S = H >= dtype(v_th)
    if v_reset is None:
        Vn = H - S.astype(dtype) * dtype(v_th)
    else:
        Vn = np.where(S, dtype(v_reset), H).astype(dtype)
    return S, Vn.astype(dtype), H


def lif_multistep(I_seq, tau=2.0, v_th=1.0, v_reset: Optional[float] = 0.0, decay_input=True, v0=None,
                  dtype=np.float32):
    """I_seq [T, ...] -> (spikes bool [T, ...], V_T, H [T, ...])."""
    I_seq = np.asarray(I_seq)
    V = np.zeros(I_seq.shape[1:], dtype=dtype) if v0 is None else np.asarray(v0, dtype=dtype)
    spikes, Hs = [], []
    for t in range(I_seq.shape[0]):
        S, V, H = lif_step(I_seq[t], V, tau, v_th, v_reset, decay_input, dtype)
        spikes.append(S)
        Hs.append(H)
    return np.stack(spikes), V, np.stack(Hs)


def compare_spikes(spk_test, spk_ref, H_ref, v_th, tie_tol=1e-5):
    """Tie-aware spike comparison.  Returns (mismatches outside ties,
    mask [T, ...] of (t, neuron) entries still comparable: a neuron drops out
    from the first step where its spike legitimately flipped at a tie)."""
    spk_test = np.asarray(spk_test).astype(bool)
    spk_ref = np.asarray(spk_ref).astype(bool)
    tie = np.abs(np.asarray(H_ref, dtype=np.float64) - v_th) <= tie_tol
    T = spk_ref.shape[0]
    alive = np.ones(spk_ref.shape[1:], dtype=bool)
    comparable = np.zeros_like(spk_ref, dtype=bool)
    bad = 0
    for t in range(T):
        comparable[t] = alive
        diff = spk_test[t] != spk_ref[t]
        bad += int((diff & alive & ~tie[t]).sum())
        alive &= ~(diff & tie[t])
    return bad, comparable
