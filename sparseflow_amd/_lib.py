"""ctypes binding of libsparseflow_hip.so (the C ABI in include/sparseflow.h).

This is the only module that talks to the native library.  Device tensors
cross the boundary as raw pointers; the current torch stream is passed as the
hipStream_t so library launches order with surrounding torch work.

If the library is missing, every device entry point raises
SparseFlowLibError: there is no silent fallback for ROCm tensors.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p
from pathlib import Path
from typing import Optional, Tuple

import torch

LIB_PATH = Path(__file__).resolve().parent / "libsparseflow_hip.so"

SF_OK = 0
SF_ERR_INVALID = 1
SF_ERR_UNSUPPORTED = 2
SF_ERR_WORKSPACE = 3
SF_ERR_HIP = 4

SF_F32, SF_F16, SF_BF16 = 0, 1, 2
SF_BITMAP_PIXEL_MAJOR, SF_BITMAP_PLANES = 0, 1
_DTYPE_CODE = {torch.float32: SF_F32, torch.float16: SF_F16, torch.bfloat16: SF_BF16}

# Every exported symbol of include/sparseflow.h with its ctypes signature.
_P = c_void_p
EXPORTS = {
    "sf_version": (c_int, []),
    "sf_last_error": (ctypes.c_char_p, []),
    "sf_activity_cutoff": (c_float, [c_float]),
    "sf_bitmap_words_per_pixel": (c_int, [c_int32]),
    "sf_prescan_chunk_pixels": (c_int32, [c_int64, c_int32, c_int32, c_int32]),
    "sf_prescan_bitmap_bytes": (c_size_t, [c_int64, c_int32, c_int32, c_int32]),
    "sf_prescan_flags_bytes": (c_size_t, [c_int64, c_int32, c_int32, c_int32]),
    "sf_conv2d_workspace_size": (c_size_t, [_P]),
    "sf_conv_lif_workspace_size": (c_size_t, [_P, c_int32]),
    "sf_prescan_pack": (c_int, [_P, c_int32, c_int64, c_int32, c_int32, c_int32, c_float, _P, _P, _P]),
    "sf_prescan_tiles": (
        c_int,
        [_P, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
         c_int32, c_int32, c_int32, _P, _P, _P, _P, _P, _P],
    ),
    "sf_conv2d_sparse": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P]),
    "sf_conv2d_bitmap_layout": (c_int, [_P]),
    "sf_conv2d_sparse_layout": (c_int, [_P, _P, c_int32, _P, _P, _P, _P, _P, _P]),
    "sf_conv2d_forward": (c_int, [_P, _P, _P, _P, c_float, _P, c_size_t, _P, _P]),
    "sf_conv2d_forward_noalloc": (c_int, [_P, _P, _P, _P, c_float, _P, _P]),
    "sf_conv_lif_forward": (c_int, [_P, c_int32, _P, _P, _P, _P, c_float, _P, _P, _P, _P, c_size_t, _P]),
    "sf_conv1x1_lif_sparse": (c_int, [_P, c_int32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "sf_conv1x1_lif_sparse_binres": (c_int, [_P, c_int32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "sf_conv1x1_lif_sparse_layout": (c_int, [_P, c_int32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int32,
                                             _P]),
    "sf_lif_multistep": (c_int, [_P, _P, c_int32, c_int32, c_int64, c_int32, c_int64, _P, _P, _P, c_int32, _P, _P, _P,
                                 _P]),
    "sf_lif_multistep_layout": (c_int, [_P, _P, c_int32, c_int32, c_int64, c_int32, c_int64, _P, _P, _P, c_int32, _P,
                                        _P, _P, c_int32, _P]),
    "sf_spike_maxpool2d": (c_int, [_P, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, _P, c_int32,
                                   _P, _P]),
    "sf_linear_bitmap_bytes": (c_size_t, [c_int64, c_int32]),
    "sf_linear_flags_bytes": (c_size_t, [c_int64]),
    "sf_linear_workspace_size": (c_size_t, [c_int64, c_int32]),
    "sf_linear_prescan": (c_int, [_P, c_int32, c_int64, c_int32, c_float, _P, _P, _P]),
    "sf_linear_sparse": (c_int, [_P, _P, _P, c_int32, c_int64, c_int32, _P, _P, c_int32, _P, c_int32, _P]),
    "sf_linear_forward": (c_int, [_P, c_int32, c_int64, c_int32, _P, _P, c_int32, c_float, _P, c_size_t, _P, c_int32,
                                  _P]),
    "sf_linear_mfma": (c_int, [_P, c_int32, c_int64, c_int32, _P, _P, c_int32, _P, c_int32, c_float, _P, c_int32,
                               _P]),
    "sf_linear_mfma_bits": (c_int, [_P, _P, _P, c_int32, c_int64, c_int32, _P, _P, c_int32, _P, c_int32, c_float, _P,
                                    c_int32, _P]),
    "sf_bmm_supported": (c_int, [c_int32, c_int32]),
    "sf_bmm_sparse": (c_int, [_P, _P, c_int32, c_int64, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_float,
                              c_float, _P, c_int32, _P]),
    "sf_bmm_mfma_supported": (c_int, [c_int32, c_int32]),
    "sf_bmm_mfma": (c_int, [_P, _P, c_int32, c_int64, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_float,
                            c_float, _P, c_int32, _P]),
    "sf_spike_attention_supported": (c_int, [c_int32, c_int32]),
    "sf_spike_attention": (c_int, [_P, _P, _P, c_int32, c_int64, c_int32, c_int32, c_int32, _P, c_float, c_float, _P,
                                   _P, c_int32, _P]),
    "sf_timing_enable": (c_int, [c_int32]),
    "sf_timing_collect": (c_int, []),
    "sf_timing_query": (c_int64, [ctypes.c_char_p, ctypes.POINTER(c_double)]),
    "sf_timing_reset": (None, []),
}


class SparseFlowLibError(RuntimeError):
    """The native library is missing or a library call failed."""


class UnsupportedError(SparseFlowLibError):
    """The kernels do not implement this shape/pattern (SF_ERR_UNSUPPORTED)."""


class ConvDesc(ctypes.Structure):
    _fields_ = [
        ("n", c_int64),
        ("c_in", c_int32), ("h_in", c_int32), ("w_in", c_int32),
        ("c_out", c_int32), ("h_out", c_int32), ("w_out", c_int32),
        ("kernel", c_int32), ("stride", c_int32), ("pad", c_int32),
        ("in_dtype", c_int32), ("out_dtype", c_int32),
    ]


class LifParams(ctypes.Structure):
    _fields_ = [
        ("tau", c_float), ("v_threshold", c_float), ("v_reset", c_float),
        ("hard_reset", c_int32), ("decay_input", c_int32),
    ]


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def _load() -> ctypes.CDLL:
    global _lib, _load_error
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            _load_error = (
                f"{LIB_PATH.name} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python sparseflow_amd/_build.py`"
            )
            raise SparseFlowLibError(_load_error)
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in EXPORTS.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def lib() -> ctypes.CDLL:
    """The loaded library; raises SparseFlowLibError when it is not built."""
    loaded = _lib
    return loaded if loaded is not None else _load()


def available() -> bool:
    try:
        _load()
        return True
    except (SparseFlowLibError, OSError):
        return False


def _check(rc: int, what: str) -> None:
    if rc == SF_OK:
        return
    msg = lib().sf_last_error().decode(errors="replace")
    if rc == SF_ERR_UNSUPPORTED:
        raise UnsupportedError(f"{what}: {msg}")
    raise SparseFlowLibError(f"{what} failed (status {rc}): {msg}")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else c_void_p(t.data_ptr())


_current_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def raw_stream(index: int) -> int:
    """Handle (hipStream_t as an int) of torch's current stream on device
    `index`, without building a torch Stream object."""
    if _current_raw_stream is not None:
        return int(_current_raw_stream(index))
    return int(torch.cuda.current_stream(index).cuda_stream)


def _stream(device: torch.device):
    index = device.index
    return c_void_p(raw_stream(torch.cuda.current_device() if index is None else index))


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise UnsupportedError(f"dtype {dtype} is not supported (float32/float16/bfloat16)") from None


def _require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise SparseFlowLibError(f"{name} must be a ROCm device tensor")


# ---------------------------------------------------------------------------
# Host utilities
# ---------------------------------------------------------------------------

def version() -> int:
    return int(lib().sf_version())


def activity_cutoff(threshold: float) -> float:
    return float(lib().sf_activity_cutoff(float(threshold)))


def words_per_pixel(c: int) -> int:
    return int(lib().sf_bitmap_words_per_pixel(int(c)))


def chunk_pixels(n: int, c: int, h: int, w: int) -> int:
    return int(lib().sf_prescan_chunk_pixels(int(n), int(c), int(h), int(w)))


def conv_desc(n, c_in, h_in, w_in, c_out, h_out, w_out, k, s, p, in_dtype, out_dtype) -> ConvDesc:
    return ConvDesc(int(n), int(c_in), int(h_in), int(w_in), int(c_out), int(h_out), int(w_out),
                    int(k), int(s), int(p), int(in_dtype), int(out_dtype))


def conv2d_workspace_size(desc: ConvDesc) -> int:
    return int(lib().sf_conv2d_workspace_size(ctypes.byref(desc)))


def conv_lif_workspace_size(desc: ConvDesc, T: int) -> int:
    return int(lib().sf_conv_lif_workspace_size(ctypes.byref(desc), int(T)))


def tap_major_weight(weight: torch.Tensor) -> torch.Tensor:
    """[C_out, C_in, k, k] -> f32 [C_in*k*k, C_out], row (ci*k + kh)*k + kw."""
    c_out, c_in, kh, kw = weight.shape
    return weight.detach().to(torch.float32).permute(1, 2, 3, 0).reshape(c_in * kh * kw, c_out).contiguous()


# ---------------------------------------------------------------------------
# Stage 1
# ---------------------------------------------------------------------------

def prescan_pack(x: torch.Tensor, threshold: float,
                 bits: Optional[torch.Tensor] = None,
                 flags: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [n, c, h, w] (contiguous) -> (bits uint32 [n, h*w, cwp], flags uint32)."""
    _require_device(x, "x")
    if x.dim() != 4:
        raise ValueError(f"prescan_pack expects a 4-D NCHW tensor, got {tuple(x.shape)}")
    x = x.contiguous()
    n, c, h, w = (int(v) for v in x.shape)
    L = lib()
    nbits = int(L.sf_prescan_bitmap_bytes(n, c, h, w)) // 4
    nflags = int(L.sf_prescan_flags_bytes(n, c, h, w)) // 4
    if bits is None:
        bits = torch.empty(max(nbits, 1), dtype=torch.int32, device=x.device)
    if flags is None:
        flags = torch.empty(max(nflags, 1), dtype=torch.int32, device=x.device)
    if bits.numel() < nbits or flags.numel() < nflags:
        raise ValueError("bits/flags buffers are too small")
    rc = L.sf_prescan_pack(_ptr(x), dtype_code(x.dtype), n, c, h, w, float(threshold),
                           _ptr(bits), _ptr(flags), _stream(x.device))
    _check(rc, "sf_prescan_pack")
    return bits, flags


def prescan_tiles(bits: torch.Tensor, n: int, c: int, h_in: int, w_in: int, h_out: int, w_out: int,
                  kernel: int, stride: int, pad: int, tile_h: int, tile_w: int, group_size: int = 16,
                  ch_mask: Optional[torch.Tensor] = None, ch_count: Optional[torch.Tensor] = None,
                  ch_list: Optional[torch.Tensor] = None, ag_mask: Optional[torch.Tensor] = None,
                  tile_class: Optional[torch.Tensor] = None) -> None:
    """Fill whichever per-tile outputs are given (see sf_prescan_tiles)."""
    _require_device(bits, "bits")
    rc = lib().sf_prescan_tiles(
        _ptr(bits), int(n), int(c), int(h_in), int(w_in), int(h_out), int(w_out), int(kernel),
        int(stride), int(pad), int(tile_h), int(tile_w), int(group_size),
        _ptr(ch_mask), _ptr(ch_count), _ptr(ch_list), _ptr(ag_mask), _ptr(tile_class), _stream(bits.device))
    _check(rc, "sf_prescan_tiles")


# ---------------------------------------------------------------------------
# Stage 2 / fused
# ---------------------------------------------------------------------------

def conv2d_sparse(desc: ConvDesc, bits: torch.Tensor, flags: torch.Tensor, x: torch.Tensor,
                  wt: torch.Tensor, bias: Optional[torch.Tensor], y: torch.Tensor,
                  layout: int = SF_BITMAP_PIXEL_MAJOR) -> torch.Tensor:
    """Stage 2 over a bitmap in `layout` (word planes raise UnsupportedError
    for shapes whose Stage-2 kernel reads pixel-major words)."""
    if layout == SF_BITMAP_PIXEL_MAJOR:
        rc = lib().sf_conv2d_sparse(ctypes.byref(desc), _ptr(bits), _ptr(flags), _ptr(x), _ptr(wt),
                                    _ptr(bias), _ptr(y), _stream(x.device))
        _check(rc, "sf_conv2d_sparse")
        return y
    rc = lib().sf_conv2d_sparse_layout(ctypes.byref(desc), _ptr(bits), int(layout), _ptr(flags), _ptr(x), _ptr(wt),
                                       _ptr(bias), _ptr(y), _stream(x.device))
    _check(rc, "sf_conv2d_sparse_layout")
    return y


def conv2d_bitmap_layout(desc: ConvDesc) -> int:
    """The bitmap layout the shape's Stage-2 kernel reads fastest."""
    rc = int(lib().sf_conv2d_bitmap_layout(ctypes.byref(desc)))
    if rc < 0:
        _check(-rc, "sf_conv2d_bitmap_layout")
    return rc


def conv2d_forward(desc: ConvDesc, x: torch.Tensor, wt: torch.Tensor, bias: Optional[torch.Tensor],
                   threshold: float, workspace: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    rc = lib().sf_conv2d_forward(ctypes.byref(desc), _ptr(x), _ptr(wt), _ptr(bias), float(threshold),
                                 _ptr(workspace), workspace.numel() * workspace.element_size(),
                                 _ptr(y), _stream(x.device))
    _check(rc, "sf_conv2d_forward")
    return y


NOALLOC_SCRATCH_BYTES = 64 << 20  # SF_NOALLOC_SCRATCH_BYTES


def conv2d_forward_noalloc(desc: ConvDesc, x: torch.Tensor, wt: torch.Tensor, bias: Optional[torch.Tensor],
                           threshold: float, y: torch.Tensor) -> torch.Tensor:
    """sf_conv2d_forward with the bitmap in the library's per-GPU scratch
    area: nothing is allocated (calls overlapping on one GPU race)."""
    rc = lib().sf_conv2d_forward_noalloc(ctypes.byref(desc), _ptr(x), _ptr(wt), _ptr(bias), float(threshold),
                                         _ptr(y), _stream(x.device))
    _check(rc, "sf_conv2d_forward_noalloc")
    return y


def conv_lif_forward(desc: ConvDesc, T: int, x: torch.Tensor, wt: torch.Tensor, bias: Optional[torch.Tensor],
                     lif: LifParams, threshold: float, v_init: Optional[torch.Tensor],
                     spikes: torch.Tensor, v_out: torch.Tensor, workspace: torch.Tensor) -> None:
    rc = lib().sf_conv_lif_forward(
        ctypes.byref(desc), int(T), _ptr(x), _ptr(wt), _ptr(bias), ctypes.byref(lif), float(threshold),
        _ptr(v_init), _ptr(spikes), _ptr(v_out), _ptr(workspace),
        workspace.numel() * workspace.element_size(), _stream(x.device))
    _check(rc, "sf_conv_lif_forward")


def lif_multistep(x: torch.Tensor, T: int, lif: LifParams, v_init: Optional[torch.Tensor] = None,
                  spikes: Optional[torch.Tensor] = None, v_out: Optional[torch.Tensor] = None,
                  out_dtype: Optional[torch.dtype] = None, x2: Optional[torch.Tensor] = None,
                  spike_map: bool = False, map_layout: int = SF_BITMAP_PIXEL_MAJOR):
    """x [T, ...] currents (+ x2, same shape) -> (spikes [T, ...] in out_dtype
    (default x's), v [...] f32, map) where map is None or, with spike_map=True
    on a [T, N, C, H, W] input, (bits, flags) of the T*N output frames in
    `map_layout` (the prescan's pixel-major words, or word planes)."""
    _require_device(x, "x")
    x = x.contiguous()
    if x.shape[0] != T:
        raise ValueError(f"x has {x.shape[0]} steps, expected T={T}")
    if x2 is not None:
        if x2.shape != x.shape or x2.dtype != x.dtype:
            raise ValueError("x2 must match x in shape and dtype")
        _require_device(x2, "x2")
        x2 = x2.contiguous()
    if x.dim() == 5:
        n, c, hw = int(x.shape[1]), int(x.shape[2]), int(x.shape[3]) * int(x.shape[4])
    else:
        n, c, hw = 1, 1, x.numel() // T
        spike_map = False
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if spikes is None:
        spikes = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    if v_out is None:
        v_out = torch.empty(x.shape[1:], dtype=torch.float32, device=x.device)
    if v_init is not None:
        _require_device(v_init, "v_init")
        if v_init.dtype != torch.float32 or v_init.numel() != n * c * hw:
            raise ValueError("v_init must be float32 with one value per neuron")
        v_init = v_init.contiguous()
    bits = flags = None
    if spike_map:
        L = lib()
        frames = T * n
        bits = torch.empty(max(int(L.sf_prescan_bitmap_bytes(frames, c, 1, hw)) // 4, 1), dtype=torch.int32,
                           device=x.device)
        flags = torch.empty(max(int(L.sf_prescan_flags_bytes(frames, c, 1, hw)) // 4, 1), dtype=torch.int32,
                            device=x.device)
    rc = lib().sf_lif_multistep_layout(_ptr(x), _ptr(x2), dtype_code(x.dtype), int(T), n, c, hw, ctypes.byref(lif),
                                       _ptr(v_init), _ptr(spikes), dtype_code(out_dtype), _ptr(v_out), _ptr(bits),
                                       _ptr(flags), int(map_layout), _stream(x.device))
    _check(rc, "sf_lif_multistep_layout")
    return spikes, v_out, (None if bits is None else (bits, flags))


def spike_maxpool2d(bits: torch.Tensor, n: int, c: int, h: int, w: int, k: int, stride: int, padding: int,
                    dtype: torch.dtype, device: torch.device):
    """Max pooling of n frames of binary spikes [c, h, w] given by their spike
    map `bits` (sf_spike_maxpool2d): (y [n, c, h_out, w_out] in dtype, (out
    bits, zeroed flags)) -- the pooled spikes and their own spike map."""
    h_out = (h + 2 * padding - k) // stride + 1
    w_out = (w + 2 * padding - k) // stride + 1
    y = torch.empty((n, c, h_out, w_out), dtype=dtype, device=device)
    out_bits = torch.empty(n * h_out * w_out * int(lib().sf_bitmap_words_per_pixel(c)), dtype=torch.int32,
                           device=device)
    flags = torch.zeros((int(lib().sf_prescan_flags_bytes(n, c, h_out, w_out)) + 3) // 4, dtype=torch.int32,
                        device=device)
    rc = lib().sf_spike_maxpool2d(_ptr(bits), int(n), int(c), int(h), int(w), int(k), int(stride), int(padding),
                                  _ptr(y), dtype_code(dtype), _ptr(out_bits), _stream(device))
    _check(rc, "sf_spike_maxpool2d")
    return y, (out_bits, flags)


def conv1x1_lif_sparse(desc: ConvDesc, T: int, bits: torch.Tensor, flags: torch.Tensor, x: torch.Tensor,
                       wt: torch.Tensor, bias: Optional[torch.Tensor], x2: Optional[torch.Tensor], lif: LifParams,
                       v_init: Optional[torch.Tensor], spikes: torch.Tensor, v_out: torch.Tensor,
                       out_bits: Optional[torch.Tensor], out_flags: Optional[torch.Tensor],
                       res_bits: Optional[torch.Tensor] = None, out_layout: int = SF_BITMAP_PIXEL_MAJOR) -> None:
    """res_bits: a binary residual's pixel-major spike map, read instead of
    x2 (sf_conv1x1_lif_sparse_binres); out_layout: the output map's layout
    (word planes only without res_bits)."""
    if res_bits is not None:
        if out_layout != SF_BITMAP_PIXEL_MAJOR:
            raise UnsupportedError("a binary residual's map is read with a pixel-major output map")
        rc = lib().sf_conv1x1_lif_sparse_binres(ctypes.byref(desc), int(T), _ptr(bits), _ptr(flags), _ptr(x),
                                                _ptr(wt), _ptr(bias), _ptr(res_bits), ctypes.byref(lif),
                                                _ptr(v_init), _ptr(spikes), _ptr(v_out), _ptr(out_bits),
                                                _ptr(out_flags), _stream(x.device))
        _check(rc, "sf_conv1x1_lif_sparse_binres")
        return
    rc = lib().sf_conv1x1_lif_sparse_layout(ctypes.byref(desc), int(T), _ptr(bits), _ptr(flags), _ptr(x), _ptr(wt),
                                            _ptr(bias), _ptr(x2), ctypes.byref(lif), _ptr(v_init), _ptr(spikes),
                                            _ptr(v_out), _ptr(out_bits), _ptr(out_flags), int(out_layout),
                                            _stream(x.device))
    _check(rc, "sf_conv1x1_lif_sparse_layout")


# ---------------------------------------------------------------------------
# Sparse linear / batched matmul
# ---------------------------------------------------------------------------

def linear_prescan(x2d: torch.Tensor, threshold: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [m, k] (contiguous) -> (bits int32 [m * words], flags int32) of the
    row prescan (sf_linear_prescan)."""
    _require_device(x2d, "x")
    m, k = (int(v) for v in x2d.shape)
    L = lib()
    bits = torch.empty(max(int(L.sf_linear_bitmap_bytes(m, k)) // 4, 1), dtype=torch.int32, device=x2d.device)
    flags = torch.empty(max(int(L.sf_linear_flags_bytes(m)) // 4, 1), dtype=torch.int32, device=x2d.device)
    rc = L.sf_linear_prescan(_ptr(x2d), dtype_code(x2d.dtype), m, k, float(threshold), _ptr(bits), _ptr(flags),
                             _stream(x2d.device))
    _check(rc, "sf_linear_prescan")
    return bits, flags


def linear_workspace_size(m: int, k: int) -> int:
    return int(lib().sf_linear_workspace_size(int(m), int(k)))


def linear_forward(x2d: torch.Tensor, wt: torch.Tensor, bias: Optional[torch.Tensor], threshold: float,
                   y: torch.Tensor, workspace: torch.Tensor) -> torch.Tensor:
    """y [m, c_out] = x [m, k] @ wt [k, c_out] (f32) + bias (sf_linear_forward)."""
    _require_device(x2d, "x")
    m, k = (int(v) for v in x2d.shape)
    rc = lib().sf_linear_forward(_ptr(x2d), dtype_code(x2d.dtype), m, k, _ptr(wt), _ptr(bias), int(wt.shape[1]),
                                 float(threshold), _ptr(workspace), workspace.numel() * workspace.element_size(),
                                 _ptr(y), dtype_code(y.dtype), _stream(x2d.device))
    _check(rc, "sf_linear_forward")
    return y


def linear_sparse(bits: torch.Tensor, flags: torch.Tensor, x2d: torch.Tensor, wt: torch.Tensor,
                  bias: Optional[torch.Tensor], y: torch.Tensor) -> torch.Tensor:
    m, k = (int(v) for v in x2d.shape)
    rc = lib().sf_linear_sparse(_ptr(bits), _ptr(flags), _ptr(x2d), dtype_code(x2d.dtype), m, k, _ptr(wt),
                                _ptr(bias), int(wt.shape[1]), _ptr(y), dtype_code(y.dtype), _stream(x2d.device))
    _check(rc, "sf_linear_sparse")
    return y


def linear_mfma(x2d: torch.Tensor, w_hi: torch.Tensor, w_lo: torch.Tensor, bias: Optional[torch.Tensor],
                y: torch.Tensor, threshold: float = 1e-6) -> torch.Tensor:
    """y [m, c_out] = x [m, k] @ (w_hi + w_lo)^T + bias on the matrix cores
    (sf_linear_mfma); w_hi / w_lo bf16 [c_out, kp] (kp = k rounded up to 32)."""
    _require_device(x2d, "x")
    m, k = (int(v) for v in x2d.shape)
    c_out, kp = (int(v) for v in w_hi.shape)
    rc = lib().sf_linear_mfma(_ptr(x2d), dtype_code(x2d.dtype), m, k, _ptr(w_hi), _ptr(w_lo), kp, _ptr(bias), c_out,
                              float(threshold), _ptr(y), dtype_code(y.dtype), _stream(x2d.device))
    _check(rc, "sf_linear_mfma")
    return y


def linear_mfma_bits(bits: torch.Tensor, flags: torch.Tensor, x2d: torch.Tensor, w_hi: torch.Tensor,
                     w_lo: torch.Tensor, bias: Optional[torch.Tensor], y: torch.Tensor,
                     threshold: float = 1e-6) -> torch.Tensor:
    """linear_mfma over linear_prescan's (bits, flags) of the same x and
    threshold (sf_linear_mfma_bits): spike row blocks read the bitmap."""
    _require_device(x2d, "x")
    m, k = (int(v) for v in x2d.shape)
    c_out, kp = (int(v) for v in w_hi.shape)
    rc = lib().sf_linear_mfma_bits(_ptr(bits), _ptr(flags), _ptr(x2d), dtype_code(x2d.dtype), m, k, _ptr(w_hi),
                                   _ptr(w_lo), kp, _ptr(bias), c_out, float(threshold), _ptr(y), dtype_code(y.dtype),
                                   _stream(x2d.device))
    _check(rc, "sf_linear_mfma_bits")
    return y


def bmm_supported(k: int, n: int) -> bool:
    return bool(lib().sf_bmm_supported(int(k), int(n)))


def bmm_mfma_supported(k: int, n: int) -> bool:
    return bool(lib().sf_bmm_mfma_supported(int(k), int(n)))


def bmm_sparse(a: torch.Tensor, b: torch.Tensor, threshold: float, c: torch.Tensor, alpha: float = 1.0,
               mfma: bool = False) -> torch.Tensor:
    """c [B, m, n] = alpha * (a [B, m, k] (contiguous) @ b [B, k, n] (any
    strides, same dtype as a)) (sf_bmm_sparse, or sf_bmm_mfma)."""
    _require_device(a, "a")
    _require_device(b, "b")
    bt, m, k = (int(v) for v in a.shape)
    n = int(b.shape[2])
    fn = lib().sf_bmm_mfma if mfma else lib().sf_bmm_sparse
    rc = fn(_ptr(a), _ptr(b), dtype_code(a.dtype), bt, m, k, n, int(b.stride(0)), int(b.stride(1)),
                             int(b.stride(2)), float(threshold), float(alpha), _ptr(c), dtype_code(c.dtype),
                             _stream(a.device))
    _check(rc, "sf_bmm_mfma" if mfma else "sf_bmm_sparse")
    return c


def spike_attention_supported(s: int, d: int) -> bool:
    return bool(lib().sf_spike_attention_supported(int(s), int(d)))


def spike_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, threshold: float,
                    y: torch.Tensor) -> torch.Tensor:
    """q, k, v, y [TB, S, H, D] views (any strides, d contiguous, q/k/v with
    the same strides): y = (q @ k^T * scale) @ v per (tb, h) (sf_spike_attention)."""
    _require_device(q, "q")
    tb, s, h, d = (int(t) for t in q.shape)
    if k.stride() != q.stride() or v.stride() != q.stride() or q.stride(3) != 1 or y.stride(3) != 1:
        raise ValueError("q, k, v must share strides and every operand must have a contiguous last dim")
    qs = (ctypes.c_int64 * 3)(q.stride(0), q.stride(1), q.stride(2))
    ys = (ctypes.c_int64 * 3)(y.stride(0), y.stride(1), y.stride(2))
    rc = lib().sf_spike_attention(_ptr(q), _ptr(k), _ptr(v), dtype_code(q.dtype), tb, s, h, d, qs, float(scale),
                                  float(threshold), _ptr(y), ys, dtype_code(y.dtype), _stream(q.device))
    _check(rc, "sf_spike_attention")
    return y


# ---------------------------------------------------------------------------
# Per-kernel timing (bench instrumentation)
# ---------------------------------------------------------------------------

KERNEL_NAMES = ("prescan_pack", "prescan_tiles", "conv_gather", "conv_lif", "conv_rows", "conv_rows_kc", "conv_flat", "conv_px3", "conv_lif_px3",
                "lif_multistep", "prescan_rows", "linear_flat", "bmm_sparse", "spike_attention",
                "linear_mfma", "bmm_mfma", "conv_lif_flat", "conv_mfma", "conv_rows_fused", "conv_dense_mfma")


def timing_enable(on: bool) -> None:
    lib().sf_timing_enable(1 if on else 0)


def timing_reset() -> None:
    lib().sf_timing_reset()


def timing_collect() -> dict:
    """Synchronise recorded launches; return {kernel: (launches, total_ms)}."""
    _check(lib().sf_timing_collect(), "sf_timing_collect")
    out = {}
    for name in KERNEL_NAMES:
        ms = c_double(0.0)
        cnt = int(lib().sf_timing_query(name.encode(), ctypes.byref(ms)))
        out[name] = (cnt, float(ms.value))
    return out
