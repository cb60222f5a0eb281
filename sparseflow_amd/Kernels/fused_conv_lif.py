"""Fused sparse conv + LIF on MI355X (drop-in for Kernels/fused_conv_lif.py).

The reference's fused path launches one Triton kernel per timestep and
round-trips the membrane through HBM (Kernels/fused_conv_lif.py:310-484,
Ops/sparse_fused_conv_lif.py:191-197); it is also unimportable as shipped
(Kernels/fused_conv_lif.py:22).  Here one HIP launch runs all T steps: the
membrane stays in VGPRs, spikes are written once per step and the final
membrane once.

LIF arithmetic follows the module's torch path operation for operation
(Ops/sparse_fused_conv_lif.py:283-292), including decay_input=False and
soft reset (v_reset=None), which the reference kernel ignores
(Kernels/fused_conv_lif.py:451-452).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .. import _lib
from ..Utils.config import PRESCAN_ACTIVITY_EPS, SPARSE_DENSE_RATIO_THRESHOLD
from .conv2d import _build_two_stage_metadata, _select_tile_sizes, choose_group_size, popcount_buf

__all__ = [
    "sparse_fused_conv_lif_forward",
    "sparse_fused_conv_lif_multistep",
    "lif_params",
]

FALLBACK_RATIO = SPARSE_DENSE_RATIO_THRESHOLD

# The fused 1x1 conv + LIF kernel keeps the weights of up to two 128-channel
# input chunks resident in LDS.  Beyond that it streams every chunk again at
# every time step through two 64 KB buffers (one 8-wavefront workgroup per
# CU), and its parallelism is one wavefront per (sample, 64-pixel tile, 64
# output channels) carrying all T steps.
CONV1X1_LIF_RESIDENT_CIN = 256
CONV1X1_LIF_STREAMED_WAVES_PER_CU = 8
# With streamed weights the fused kernel is kept when its wavefronts fill at
# least this share of the GPU's workgroup slots; below it the conv over all
# T*N frames followed by the neuron pass is faster, although it writes and
# reads the currents (Spiking-ResNet50, T=16, batch 32, 1% spikes: 1024->256
# at 14x14 fills 25%: 687 us fused, 335 us as the pair; 512->128 at 28x28
# fills 41%: 380 / 314 us; 1024->512 at 14x14 fills 50%: 646 / 548 us;
# 512->256 at 28x28 fills 81%: 402 / 491 us).
CONV1X1_LIF_MIN_FILL = 0.75

_num_cus: dict = {}


def _cus(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _num_cus:
        _num_cus[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _num_cus[idx]


def conv1x1_lif_prefers_fused(c_in: int, c_out: int, n: int, h: int, w: int, num_cus: int) -> bool:
    """Whether the fused 1x1 conv + LIF kernel is the faster form for n
    samples of C_in x h x w (the alternative: the sparse conv over all frames,
    then the neuron layer): always with resident weights, with streamed ones
    when its wavefronts fill at least CONV1X1_LIF_MIN_FILL of the GPU."""
    if c_in <= CONV1X1_LIF_RESIDENT_CIN:
        return True
    waves = n * -(-(h * w) // 64) * -(-c_out // 64)
    return waves >= CONV1X1_LIF_MIN_FILL * CONV1X1_LIF_STREAMED_WAVES_PER_CU * num_cus


def lif_params(tau, v_threshold, v_reset, decay_input) -> _lib.LifParams:
    hard = v_reset is not None
    return _lib.LifParams(float(tau), float(v_threshold), float(v_reset) if hard else 0.0,
                          1 if hard else 0, 1 if decay_input else 0)


def _torch_lif_step(conv: torch.Tensor, v_prev: torch.Tensor, tau, v_threshold, v_reset, decay_input):
    """One LIF step on host tensors, the module's fallback semantics
    (Ops/sparse_fused_conv_lif.py:283-292)."""
    vr = 0.0 if v_reset is None else float(v_reset)
    if decay_input:
        v_tmp = v_prev + (conv - (v_prev - vr)) / tau
    else:
        v_tmp = v_prev - (v_prev - vr) / tau + conv
    spike = (v_tmp >= v_threshold).to(v_tmp.dtype)
    if v_reset is None:
        v_next = v_tmp - spike * v_threshold
    else:
        v_next = torch.where(spike.bool(), torch.full_like(v_tmp, float(v_reset)), v_tmp)
    return spike, v_next


def _check_pattern(kernel_size, stride, padding):
    if (kernel_size, stride, padding) not in ((3, 1, 1), (1, 1, 0)):
        raise _lib.UnsupportedError("fused conv-LIF supports 3x3 s1 p1 and 1x1 s1 p0")


def sparse_fused_conv_lif_multistep(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    tau: float = 2.0,
    v_threshold: float = 1.0,
    v_reset: Optional[float] = 0.0,
    decay_input: bool = True,
    kernel_size: int = 3,
    threshold: float = PRESCAN_ACTIVITY_EPS,
    v_init: Optional[torch.Tensor] = None,
    w_tap: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    return_ms: bool = False,
):
    """x [T, N, C, H, W] -> (spikes [T, N, C_out, H, W] in x.dtype,
    v_T [N, C_out, H, W] f32, ms).  One kernel launch for all T steps."""
    if x.dim() != 5:
        raise ValueError(f"expected [T, N, C, H, W], got {tuple(x.shape)}")
    padding = 1 if kernel_size == 3 else 0
    _check_pattern(kernel_size, 1, padding)
    T, N, C, H, W = (int(v) for v in x.shape)
    C_OUT = int(weight.shape[0])
    H_OUT = H + 2 * padding - kernel_size + 1
    W_OUT = W + 2 * padding - kernel_size + 1
    if not x.is_cuda:
        v = torch.zeros((N, C_OUT, H_OUT, W_OUT), dtype=torch.float32) if v_init is None else v_init.float()
        outs = []
        for t in range(T):
            conv = F.conv2d(x[t], weight, bias, stride=1, padding=padding).float()
            s, v = _torch_lif_step(conv, v, tau, v_threshold, v_reset, decay_input)
            outs.append(s.to(x.dtype))
        return torch.stack(outs, 0), v, 0.0

    x = x.contiguous()
    wt = w_tap if w_tap is not None else _lib.tap_major_weight(weight)
    b = None if bias is None else bias.detach().to(torch.float32).contiguous()
    vi = None if v_init is None else v_init.detach().to(torch.float32).contiguous()
    if vi is not None and (tuple(vi.shape) != (N, C_OUT, H_OUT, W_OUT) or vi.device != x.device):
        raise ValueError(f"v_init shape {tuple(vi.shape)} on {vi.device} != {(N, C_OUT, H_OUT, W_OUT)} on {x.device}")
    code = _lib.dtype_code(x.dtype)
    desc = _lib.conv_desc(N, C, H, W, C_OUT, H_OUT, W_OUT, kernel_size, 1, padding, code, code)
    need = _lib.conv_lif_workspace_size(desc, T)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    spikes = torch.empty((T, N, C_OUT, H_OUT, W_OUT), dtype=x.dtype, device=x.device)
    v_out = torch.empty((N, C_OUT, H_OUT, W_OUT), dtype=torch.float32, device=x.device)
    ms = 0.0
    if return_ms:
        se, ee = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        se.record()
    _lib.conv_lif_forward(desc, T, x, wt, b, lif_params(tau, v_threshold, v_reset, decay_input),
                          threshold, vi, spikes, v_out, workspace)
    if return_ms:
        ee.record()
        torch.cuda.synchronize(x.device)
        ms = se.elapsed_time(ee)
    return spikes, v_out, ms


def sparse_fused_conv_lif_forward(
    x,
    v_prev,
    weight,
    bias,
    tau=2.0,
    v_threshold=1.0,
    v_reset=0.0,
    decay_input=True,
    block_size=None,
    kernel_size=3,
    threshold=1e-6,
    w_cl=None,
    ag_mask_buf=None,
    return_ms=False,
    fallback_ratio=FALLBACK_RATIO,
    return_avg_active_ratio=False,
    **legacy_kwargs,
):
    """Single LIF step, same signature and returns as
    Kernels/fused_conv_lif.py:310-329: (spike, v_next, ms[, ratio])."""
    N, C, H, W = (int(v) for v in x.shape)
    padding = 1 if kernel_size == 3 else 0
    _check_pattern(kernel_size, 1, padding)
    H_OUT = H + 2 * padding - kernel_size + 1
    W_OUT = W + 2 * padding - kernel_size + 1
    ratio = None
    if x.is_cuda and (ag_mask_buf is not None or return_avg_active_ratio):
        BH, BW = _select_tile_sizes(H_OUT, W_OUT)
        GH, GW = -(-H_OUT // BH), -(-W_OUT // BW)
        n_tiles = N * GH * GW
        if ag_mask_buf is None or ag_mask_buf.numel() < n_tiles:
            ag_mask_buf = torch.empty(max(n_tiles, 1), dtype=torch.int32, device=x.device)
        tile_class = torch.empty(max(n_tiles, 1), dtype=torch.int32, device=x.device)
        _, ng, _, _ = _build_two_stage_metadata(x.contiguous(), N, C, H, W, H_OUT, W_OUT, BH, BW, GH, GW,
                                                kernel_size, 1, padding, threshold, ag_mask_buf, tile_class)
        if return_avg_active_ratio:
            ratio = popcount_buf(ag_mask_buf, n_tiles).float().mean().item() / max(ng, 1)
    w_tap = w_cl if (w_cl is not None and w_cl.dtype == torch.float32 and w_cl.dim() == 2) else None
    spikes, v_next, ms = sparse_fused_conv_lif_multistep(
        x.unsqueeze(0), weight, bias, tau=tau, v_threshold=v_threshold, v_reset=v_reset,
        decay_input=decay_input, kernel_size=kernel_size, threshold=threshold, v_init=v_prev,
        w_tap=w_tap, return_ms=return_ms)
    spike = spikes[0]
    if return_avg_active_ratio:
        return spike, v_next, ms, (1.0 if ratio is None else ratio)
    return spike, v_next, ms


def sparse_conv1x1_lif_multistep(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    tau: float = 2.0,
    v_threshold: float = 1.0,
    v_reset: Optional[float] = 0.0,
    decay_input: bool = True,
    residual: Optional[torch.Tensor] = None,
    threshold: float = PRESCAN_ACTIVITY_EPS,
    v_init: Optional[torch.Tensor] = None,
    w_tap: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    emit_spike_map: bool = True,
    map_requests: Optional["spike_map.LayoutRequests"] = None,
):
    """Fused 1x1 conv + multi-step LIF (+ residual) on device tensors:
    x [T, N, C, H, W] -> (spikes [T, N, C_out, H, W] in x.dtype, v_T
    [N, C_out, H, W] f32), LIF(conv(x_t) + residual_t) at every step.

    The input's spike map is taken from the neuron layer that produced x
    when it handed one over (else x is prescanned into `workspace`); the
    output's spike map is attached to the spikes for the next sparse conv.
    One launch (sf_conv1x1_lif_sparse); the currents never reach HBM.
    The membrane starts at v_init, or 0.  `map_requests` (the neuron's
    LayoutRequests) picks the output map's layout and records it with the
    map."""
    from . import spike_map

    if x.dim() != 5 or not x.is_cuda:
        raise ValueError("sparse_conv1x1_lif_multistep takes a [T, N, C, H, W] device tensor")
    T, N, C, H, W = (int(v) for v in x.shape)
    C_OUT = int(weight.shape[0])
    if tuple(weight.shape[1:]) != (C, 1, 1):
        raise ValueError(f"weight {tuple(weight.shape)} is not a 1x1 kernel over {C} channels")
    x = x.contiguous()
    x4 = x.view(T * N, C, H, W)
    if residual is not None:
        if tuple(residual.shape) != (T, N, C_OUT, H, W):
            raise ValueError(f"residual shape {tuple(residual.shape)} != {(T, N, C_OUT, H, W)}")
        residual = residual.to(x.dtype).contiguous()
    code = _lib.dtype_code(x.dtype)
    desc = _lib.conv_desc(N, C, H, W, C_OUT, H, W, 1, 1, 0, code, code)
    # A residual that is itself a registered spike tensor (the spikes entering
    # a bottleneck) is read from its bitmap: 1/32 of its fp32 bytes.
    # The flat kernel reads pixel-major words (input map and residual map).
    pm = spike_map.PIXEL_MAJOR
    res_bits = None
    if residual is not None:
        rmap = spike_map.lookup(residual.view(T * N, C_OUT, H, W), threshold, want=pm,
                                consumer=("conv1x1_lif_residual", weight.data_ptr()))
        if rmap is not None:
            res_bits = rmap[0]
    handed = spike_map.lookup(x4, threshold, want=pm, consumer=("conv1x1_lif", weight.data_ptr()))
    if handed is not None:
        bits, flags = handed[0], handed[1]
    else:
        bits, flags = _lib.prescan_pack(x4, threshold)
    wt = w_tap if w_tap is not None else _lib.tap_major_weight(weight)
    b = None if bias is None else bias.detach().to(torch.float32).contiguous()
    # V_0 = v_init, else 0 (as sparse_fused_conv_lif_multistep).  The C ABI
    # takes a bare pointer, so a membrane of another shape is refused here.
    vi = None if v_init is None else v_init.detach().to(torch.float32).contiguous()
    if vi is not None and (tuple(vi.shape) != (N, C_OUT, H, W) or vi.device != x.device):
        raise ValueError(f"v_init shape {tuple(vi.shape)} on {vi.device} != {(N, C_OUT, H, W)} on {x.device}")
    spikes = torch.empty((T, N, C_OUT, H, W), dtype=x.dtype, device=x.device)
    v_out = torch.empty((N, C_OUT, H, W), dtype=torch.float32, device=x.device)
    out_bits = out_flags = None
    # Word planes only where asked for and without a residual map (the
    # kernel reads a residual map in the output map's pixel-major layout).
    out_layout = pm
    if map_requests is not None and res_bits is None:
        out_layout = map_requests.layout
    if emit_spike_map:
        L = _lib.lib()
        frames = T * N
        out_bits = torch.empty(max(int(L.sf_prescan_bitmap_bytes(frames, C_OUT, H, W)) // 4, 1), dtype=torch.int32,
                               device=x.device)
        out_flags = torch.empty(max(int(L.sf_prescan_flags_bytes(frames, C_OUT, H, W)) // 4, 1), dtype=torch.int32,
                                device=x.device)
    _lib.conv1x1_lif_sparse(desc, T, bits, flags, x, wt, b, residual, lif_params(tau, v_threshold, v_reset,
                                                                                 decay_input),
                            vi, spikes, v_out, out_bits, out_flags, res_bits=res_bits, out_layout=out_layout)
    if emit_spike_map:
        spike_map.attach(spikes, T * N, C_OUT, H, W, out_bits, out_flags, out_layout, map_requests)
    return spikes, v_out
