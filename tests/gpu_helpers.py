"""Shared helpers for the GPU parity tests."""

from __future__ import annotations

import numpy as np
import torch

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def announce(msg: str) -> None:
    """Name the case before a GPU step (visible even if the step faults)."""
    print(f"[gpu-case] {msg}", flush=True)


def spikes(shape, p, seed=0, dtype=torch.float32, device=None) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(shape, generator=g) < p).to(dtype)
    return x if device is None else x.to(device)


def clustered_spikes(shape, block=16, p_block=0.03, p_inner=0.3, seed=0) -> torch.Tensor:
    """Spatially clustered spikes: random block x block tiles active with
    p_block, Bernoulli(p_inner) inside (BASELINE config 2 generator)."""
    g = torch.Generator().manual_seed(seed)
    *lead, H, W = shape
    gh, gw = -(-H // block), -(-W // block)
    gate = (torch.rand(*lead, gh, gw, generator=g) < p_block).float()
    gate = gate.repeat_interleave(block, -2).repeat_interleave(block, -1)[..., :H, :W]
    inner = (torch.rand(shape, generator=g) < p_inner).float()
    return gate * inner


def bits_numpy(bits: torch.Tensor, n: int, hw: int, cwp: int) -> np.ndarray:
    return bits[: n * hw * cwp].cpu().numpy().view(np.uint32).reshape(n, hw, cwp)


def native_loaded() -> bool:
    with open("/proc/self/maps") as f:
        return "libsparseflow_hip.so" in f.read()


def close(y: torch.Tensor, ref: torch.Tensor, atol: float, rtol: float):
    """(ok, max_abs_err, worst_excess) with |y - ref| <= atol + rtol*|ref|."""
    y64 = y.detach().double().cpu()
    r64 = ref.detach().double().cpu()
    err = (y64 - r64).abs()
    excess = err - (atol + rtol * r64.abs())
    return bool((excess <= 0).all()), float(err.max()) if err.numel() else 0.0, float(excess.max()) if err.numel() else 0.0
