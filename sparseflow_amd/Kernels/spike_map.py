"""Spike maps handed from a neuron layer to the next sparse convolution.

A LIF layer that runs on the GPU can write, next to its spikes, their
bitmap in the exact layout the prescan (`sf_prescan_pack`) would produce
from them.  The map is remembered here, keyed by the spike tensor's memory
(device index and address);
`sparse_conv2d_forward` asks for it and, when the input is still that very
tensor (alive, not modified in place since: same version counter), skips its
prescan pass over x.  This is the bit-packed inter-layer spike format: the
convolution reads 1 bit per spike instead of the fp32 spike tensor.  The
reference has no counterpart (its layers hand over dense fp16/fp32 NCHW
spikes, Kernels/conv2d.py:986).

Only exact binary spike tensors are registered, so the map equals the
prescan's output for any activity threshold below 0.5.
"""

from __future__ import annotations

import collections
import weakref
from typing import Optional, Tuple

import torch

_MAX_ENTRIES = 8
_entries: "collections.OrderedDict[Tuple[int, int], _Entry]" = collections.OrderedDict()


def _key(t: torch.Tensor) -> Tuple[int, int]:
    return (t.get_device(), t.data_ptr())


class _Entry:
    __slots__ = ("ref", "version", "shape", "bits", "flags")

    def __init__(self, spikes: torch.Tensor, shape, bits: torch.Tensor, flags: torch.Tensor):
        self.ref = weakref.ref(spikes)
        self.version = spikes._version
        self.shape = tuple(int(v) for v in shape)
        self.bits = bits
        self.flags = flags


def attach(spikes: torch.Tensor, frames: int, c: int, h: int, w: int, bits: torch.Tensor, flags: torch.Tensor) -> None:
    """Remember (bits, flags) as the prescan output of `spikes` viewed as
    [frames, c, h, w]."""
    key = _key(spikes)
    _entries.pop(key, None)
    _entries[key] = _Entry(spikes, (frames, c, h, w), bits, flags)
    while len(_entries) > _MAX_ENTRIES:
        _entries.popitem(last=False)


def lookup(x: torch.Tensor, threshold: float) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """(bits, flags) of `x` [frames, c, h, w] if a neuron layer wrote them for
    exactly this memory and it is unchanged since; else None."""
    if not (0.0 <= threshold < 0.5) or not x.is_cuda or not x.is_contiguous():
        return None
    key = _key(x)
    e = _entries.get(key)
    if e is None:
        return None
    src = e.ref()
    if src is None or src._version != e.version or x._version != e.version or tuple(x.shape) != e.shape:
        _entries.pop(key, None)
        return None
    return e.bits, e.flags


def recorded(x: torch.Tensor) -> bool:
    """Whether a map is recorded for x's memory (valid or not): a cheap
    pre-check before `lookup`."""
    return bool(_entries) and _key(x) in _entries


def clear() -> None:
    _entries.clear()
