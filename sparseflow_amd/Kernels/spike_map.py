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

Layout.  A map's words are pixel-major ([frame][pixel][word], the prescan's
layout) or word planes ([frame][word][pixel]); which one a consumer's
kernel reads fastest depends on the consumer (the 3x3 pixel-tile and row
kernels load one word of 64 neighbouring pixels at a time: planes; the 1x1
kernels and spike pooling read pixel-major words).  The producer cannot
see its consumers, so each producer keeps a `LayoutRequests`: a consumer
that looks a map up notes there the layout it reads best, and from the next
forward on the producer writes planes when every consumer noted planes.
(The first forward takes whatever layout the map has, or no map.)
"""

from __future__ import annotations

import collections
import weakref
from typing import Hashable, Optional, Tuple

import torch

PIXEL_MAJOR, PLANES = 0, 1  # sf_bitmap_layout

_MAX_ENTRIES = 8
_entries: "collections.OrderedDict[Tuple[int, int], _Entry]" = collections.OrderedDict()


class LayoutRequests:
    """The map layouts a producer's consumers read fastest, by consumer."""

    __slots__ = ("_wants",)
    _MAX = 16

    def __init__(self):
        self._wants: "collections.OrderedDict[Hashable, int]" = collections.OrderedDict()

    def note(self, consumer: Hashable, layout: int) -> None:
        if self._wants.get(consumer) == layout:
            return
        self._wants.pop(consumer, None)
        self._wants[consumer] = int(layout)
        while len(self._wants) > self._MAX:
            self._wants.popitem(last=False)

    @property
    def layout(self) -> int:
        """Word planes when at least one consumer asked and all asked for
        them; pixel-major words otherwise."""
        if self._wants and all(v == PLANES for v in self._wants.values()):
            return PLANES
        return PIXEL_MAJOR

    def clear(self) -> None:
        self._wants.clear()


def _key(t: torch.Tensor) -> Tuple[int, int]:
    return (t.get_device(), t.data_ptr())


class _Entry:
    __slots__ = ("ref", "version", "shape", "bits", "flags", "layout", "requests")

    def __init__(self, spikes: torch.Tensor, shape, bits: torch.Tensor, flags: torch.Tensor, layout: int,
                 requests: Optional[LayoutRequests]):
        self.ref = weakref.ref(spikes)
        self.version = spikes._version
        self.shape = tuple(int(v) for v in shape)
        self.bits = bits
        self.flags = flags
        self.layout = int(layout)
        self.requests = requests


def attach(spikes: torch.Tensor, frames: int, c: int, h: int, w: int, bits: torch.Tensor, flags: torch.Tensor,
           layout: int = PIXEL_MAJOR, requests: Optional[LayoutRequests] = None) -> None:
    """Remember (bits, flags) as the prescan output of `spikes` viewed as
    [frames, c, h, w], its words in `layout`; `requests` is the producer's
    record that consumers note their preferred layout in."""
    key = _key(spikes)
    _entries.pop(key, None)
    _entries[key] = _Entry(spikes, (frames, c, h, w), bits, flags, layout, requests)
    while len(_entries) > _MAX_ENTRIES:
        _entries.popitem(last=False)


def lookup(x: torch.Tensor, threshold: float, accept: Tuple[int, ...] = (PIXEL_MAJOR,),
           want: Optional[int] = None, consumer: Hashable = None
           ) -> Optional[Tuple[torch.Tensor, torch.Tensor, int]]:
    """(bits, flags, layout) of `x` [frames, c, h, w] if a neuron layer wrote
    them for exactly this memory, it is unchanged since, and the words are
    in one of the `accept`ed layouts; else None.  `want` (with a
    `consumer` key) is noted with the map's producer as the layout this
    consumer reads fastest."""
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
    if want is not None and e.requests is not None:
        e.requests.note(consumer, want)
    # With one word per pixel (c <= 32) the two layouts are the same words.
    if e.layout not in accept and e.shape[1] > 32:
        return None
    return e.bits, e.flags, e.layout


def recorded(x: torch.Tensor) -> bool:
    """Whether a map is recorded for x's memory (valid or not): a cheap
    pre-check before `lookup`."""
    return bool(_entries) and _key(x) in _entries


def clear() -> None:
    _entries.clear()
