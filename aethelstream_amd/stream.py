"""Streamed NF4 layer stack on one GPU.

Host-side mirror of flowcast's VRAM double buffer
(flowcast/src/vram_double_buffer.rs:196-301, ready.rs:16-51) over the C ABI:
layers live in pinned host memory (``PinnedBuffer``, the counterpart of
ramflow's PinnedBuffer, ramflow/src/allocator/pinned.rs:306), are copied into
a two-slot device buffer on a copy stream (``VramDoubleBuffer.advance``) and
consumed on the compute stream after waiting on the slot's ready event.

A layer is one contiguous blob: for each matrix, its packed nibbles, uint8
double-quant absmax codes and fp32 scales, each segment 256-byte aligned
(``LayerLayout``), so one hipMemcpyAsync moves a whole layer.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Sequence, Tuple

import torch

from . import _lib
from .nf4 import BLOCK_SIZE, DQ_GROUP, Nf4Weight

ALIGN = 256


def _align(x: int) -> int:
    return (x + ALIGN - 1) // ALIGN * ALIGN


class PinnedBuffer:
    """Pinned host memory (hipHostMalloc) with a CPU uint8 tensor view."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _lib.check(_lib.load().nf4s_host_alloc(self.nbytes, ctypes.byref(p)))
        self.ptr = p.value
        arr = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)
        self.tensor = torch.frombuffer(arr, dtype=torch.uint8)

    def close(self) -> None:
        if self.ptr:
            self.tensor = None
            _lib.check(_lib.load().nf4s_host_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class Nf4View:
    """A device NF4 weight addressed by raw pointers (e.g. inside a slot)."""

    shape: list
    desc: _lib.Nf4sTensor

    def descriptor(self) -> _lib.Nf4sTensor:
        return self.desc


class LayerLayout:
    """Byte layout of one double-quantized layer blob."""

    def __init__(self, shapes: Sequence[Tuple[str, int, int]], block_size: int = BLOCK_SIZE,
                 dq_group: int = DQ_GROUP):
        self.shapes = list(shapes)
        self.block_size = block_size
        self.dq_group = dq_group
        # (name, rows, cols, off_packed, n_packed, off_q, nblocks, off_scale, ngroups)
        self.segments = []
        off = 0
        for name, r, c in self.shapes:
            n = r * c
            npk = (n + 1) // 2
            nb = (n + block_size - 1) // block_size
            ng = (nb + dq_group - 1) // dq_group
            op = off
            oq = _align(op + npk)
            os_ = _align(oq + nb)
            off = _align(os_ + 4 * ng)
            self.segments.append((name, r, c, op, npk, oq, nb, os_, ng))
        self.nbytes = off

    def pack_into(self, host: torch.Tensor, weights: Sequence[Nf4Weight]) -> None:
        """Copy double-quantized device weights into a CPU uint8 view."""
        if len(weights) != len(self.segments):
            raise ValueError("one weight per layout segment")
        for seg, w in zip(self.segments, weights):
            _, r, c, op, npk, oq, nb, os_, ng = seg
            if not w.double_quant or list(w.shape) != [r, c]:
                raise ValueError("layer blobs hold double-quantized weights of the layout's shapes")
            host[op:op + npk].copy_(w.packed.view(torch.uint8))
            host[oq:oq + nb].copy_(w.absmax_q.view(torch.uint8))
            host[os_:os_ + 4 * ng].copy_(w.absmax_scale.view(torch.uint8))

    def views(self, dev_ptr: int) -> List[Nf4View]:
        """Descriptors of the layer's matrices inside a device copy of the blob."""
        out = []
        for _, r, c, op, npk, oq, nb, os_, ng in self.segments:
            d = _lib.Nf4sTensor(packed=dev_ptr + op, packed_len=npk, absmax=None,
                                absmax_q=dev_ptr + oq, absmax_scale=dev_ptr + os_,
                                absmax_len=nb, scale_len=ng, block_size=self.block_size,
                                dq_group=self.dq_group)
            out.append(Nf4View(shape=[r, c], desc=d))
        return out


class VramDoubleBuffer:
    """flowcast/src/vram_double_buffer.rs:215-301 on the device."""

    def __init__(self, slot_bytes: int):
        h = ctypes.c_void_p()
        _lib.check(_lib.load().nf4s_dbuf_create(int(slot_bytes), ctypes.byref(h)))
        self.handle = h.value

    def slot_capacity(self) -> int:
        return int(_lib.load().nf4s_dbuf_capacity(self.handle))

    def advance(self, layer_idx: int, src_ptr: int, nbytes: int) -> Tuple[int, int]:
        """Copy `nbytes` at pinned host `src_ptr` into the staging slot on the
        copy stream and swap slots; returns (device pointer, ready event)."""
        dp, ev = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(_lib.load().nf4s_dbuf_advance(self.handle, layer_idx, src_ptr, int(nbytes),
                                                 ctypes.byref(dp), ctypes.byref(ev)))
        return dp.value, ev.value

    def release(self, dev_ptr: int, stream: torch.cuda.Stream) -> None:
        """Everything enqueued so far on `stream` is the last use of the slot
        at `dev_ptr`; its refill (two advances later) waits for that."""
        _lib.check(_lib.load().nf4s_dbuf_release(self.handle, dev_ptr, stream.cuda_stream))

    def close(self) -> None:
        if self.handle:
            _lib.check(_lib.load().nf4s_dbuf_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def stream_wait_event(stream: torch.cuda.Stream, event: int) -> None:
    """The consumer's wait before reading a slot (flowcast/src/ready.rs:43-51)."""
    _lib.check(_lib.load().nf4s_stream_wait_event(stream.cuda_stream, event))


def run_stack(layers: Sequence[PinnedBuffer], layout: LayerLayout, dbuf: VramDoubleBuffer,
              compute, stream: torch.cuda.Stream) -> None:
    """Streams every layer through the double buffer.  The copy of layer l+1
    is enqueued before layer l's kernels, so H2D and compute overlap; the copy
    of layer l+2 into layer l's slot waits for layer l's release.
    ``compute(l, views)`` enqueues layer l's kernels on the current stream."""
    n = len(layers)
    if n == 0:
        return
    cur = dbuf.advance(0, layers[0].ptr, layout.nbytes)
    for l in range(n):
        nxt = dbuf.advance(l + 1, layers[l + 1].ptr, layout.nbytes) if l + 1 < n else None
        ptr, ev = cur
        stream_wait_event(stream, ev)
        with torch.cuda.stream(stream):
            compute(l, layout.views(ptr))
        dbuf.release(ptr, stream)
        cur = nxt
