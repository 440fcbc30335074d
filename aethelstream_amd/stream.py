"""Streamed NF4 layer stack on one GPU (benchmark config 5).

Host-side mirror of flowcast's VRAM double buffer
(flowcast/src/vram_double_buffer.rs:196-301, ready.rs:16-51) over the C ABI:
layers live in pinned host memory (``PinnedBuffer``, the counterpart of
ramflow's PinnedBuffer, ramflow/src/allocator/pinned.rs:306), are copied into
a two-slot device buffer on a copy stream (``VramDoubleBuffer.advance``) and
consumed on the compute stream after waiting on the slot's ready event.

A layer is one contiguous blob: for each matrix, its packed nibbles, uint8
double-quant absmax codes and fp32 scales, each segment 256-byte aligned
(``LayerLayout``), so one hipMemcpyAsync moves a whole layer.

``FlowCastSeam`` is the hand-off of FlowCast's cuda-double-buffer path
(flowcast/src/lib.rs:458-545, ready.rs:20-52): blobs packed by the shard
loader from the on-disk NF4 payloads (``ShardLoader.pack_layer``) are made
resident in pinned memory and published (``prefetch``, the completion side
of FlowCast's prefetch state machine; any thread may call it),
``take_ready`` blocks until the layer is resident or its timeout passes
(``PrefetchMiss``, flowcast/src/error.rs:20-25), copies it into the double
buffer and returns a ``ReadyLayer`` (slab 0 = the slot, the copy event, the
layer's precision and needs_decode), ``retire_layer`` releases it.  The
prefetch policy itself and the file I/O backend are not built: ``prefetch``
packs the blob in the calling thread.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

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


class BlobLayout:
    """Layout of a layer blob packed by the shard loader: one
    ``nf4s_blob_entry`` per parameter (packed, absmax part, scales, each at
    a 256-byte boundary) and the parameters' shapes."""

    def __init__(self, names: Sequence[str], entries: Sequence[_lib.Nf4sBlobEntry],
                 shapes: Sequence[Sequence[int]], nbytes: int):
        self.names = list(names)
        self.entries = list(entries)
        self.shapes = [list(x) for x in shapes]
        self.nbytes = int(nbytes)

    def views(self, base_ptr: int) -> List[Nf4View]:
        """Descriptors of the parameters inside a copy of the blob at base_ptr."""
        out = []
        for e, shape in zip(self.entries, self.shapes):
            d = _lib.Nf4sTensor()
            _lib.check(_lib.load().nf4s_blob_tensor(ctypes.byref(e), base_ptr, ctypes.byref(d)))
            out.append(Nf4View(shape=shape, desc=d))
        return out


# enum nf4s_precision: flowcast/src/config.rs:16-27 Precision, plus NF4.
PRECISIONS = ("FP32", "FP16", "BF16", "INT8", "INT4", "NF4")
PRECISION_NF4 = PRECISIONS.index("NF4")
NF4S_ERR_PREFETCH_MISS = 12


class PrefetchMiss(Exception):
    """``FlowCastError::PrefetchMiss { layer_idx }`` (flowcast/src/error.rs:
    20-25): the layer was not resident before take_ready's timeout."""

    def __init__(self, layer_idx: int, message: str):
        super().__init__(message)
        self.layer_idx = layer_idx


def _timeout_us(timeout: float) -> int:
    """Seconds as the ABI's int64 microseconds; an infinite timeout (wait
    until published) becomes 10^9 s, negative ones are passed on for the
    library to reject."""
    return int(min(float(timeout), 1e9) * 1e6)


class Residency:
    """The ready map of FlowCast's prefetch state machine
    (flowcast/src/state_machine.rs:306-346): layers a prefetcher published as
    resident in pinned memory, each taken once by a waiter (nf4s_residency_*).
    Thread-safe; a waiting call releases the GIL."""

    def __init__(self, num_layers: int):
        h = ctypes.c_void_p()
        _lib.check(_lib.load().nf4s_residency_create(int(num_layers), ctypes.byref(h)))
        self.handle = h

    def publish(self, layer_idx: int, ptr: int, nbytes: int, precision: int = PRECISION_NF4):
        _lib.check(_lib.load().nf4s_residency_publish(self.handle, int(layer_idx), ptr,
                                                      int(nbytes), int(precision)))

    def wait(self, layer_idx: int, timeout: float) -> Tuple[int, int, int]:
        """(pinned pointer, bytes, precision) of the layer once resident;
        ``PrefetchMiss`` after ``timeout`` seconds (0 always misses, as the
        reference checks the deadline first)."""
        p, nb, pr = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int32()
        lib = _lib.load()
        rc = lib.nf4s_residency_wait(self.handle, int(layer_idx), _timeout_us(timeout),
                                     ctypes.byref(p), ctypes.byref(nb), ctypes.byref(pr))
        if rc == NF4S_ERR_PREFETCH_MISS:
            raise PrefetchMiss(layer_idx, lib.nf4s_last_error_message().decode())
        _lib.check(rc)
        return int(p.value or 0), int(nb.value), int(pr.value)

    def close(self) -> None:
        if self.handle:
            _lib.check(_lib.load().nf4s_residency_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class ReadyLayer:
    """flowcast/src/ready.rs:20-52 with the cuda-double-buffer feature:
    ``slab_device_ptrs`` holds (0, slot pointer); the consumer waits on
    ``copy_event`` (``stream_wait_event``) before reading the slot, and hands
    the layer back with ``FlowCastSeam.retire_layer``.  ``precision`` is the
    precision the blob was published in; ``needs_decode`` is True for INT4 /
    INT8 (QuantizedDecoder::needs_decode, flowcast/src/decode.rs:181-183), so
    False for NF4, which the fused GEMMs dequantize in-kernel."""

    layer_idx: int
    slab_device_ptrs: List[Tuple[int, int]]
    copy_event: int
    views: List[Nf4View]
    raw: _lib.Nf4sReadyLayer
    precision: str = "NF4"
    needs_decode: bool = False


class FlowCastSeam:
    """FlowCast::take_ready / retire_layer (flowcast/src/lib.rs:458-498,
    543-545) over the VRAM double buffer, fed from shard-loader blobs.

    ``layer_params`` maps a layer index to the names of its NF4 parameters
    (the blob order).  Blobs are packed into pinned memory when first taken
    (``pin``) and kept, as FlowCast's pinned pool keeps resident layers."""

    def __init__(self, loader, layer_params: Dict[int, Sequence[str]]):
        self.loader = loader
        self.layer_params = {int(k): list(v) for k, v in layer_params.items()}
        self.layouts: Dict[int, BlobLayout] = {}
        for l, names in self.layer_params.items():
            ents, nb = loader.pack_layer(names)
            shapes = []
            for n in names:
                info = loader.param_info(n)
                shapes.append(list(info.shape[:info.ndim]))
            self.layouts[l] = BlobLayout(names, ents, shapes, nb)
        self.pinned: Dict[int, PinnedBuffer] = {}
        cap = max((x.nbytes for x in self.layouts.values()), default=0)
        self.dbuf = VramDoubleBuffer(max(cap, 1))
        self.residency = Residency(max(self.layouts, default=-1) + 1)

    def pin(self, layer_idx: int) -> PinnedBuffer:
        """The layer's blob in pinned memory, packed from the shards on first use."""
        pb = self.pinned.get(layer_idx)
        if pb is None:
            lay = self.layouts[layer_idx]
            pb = PinnedBuffer(max(lay.nbytes, 1))
            _, nb = self.loader.pack_layer(lay.names, pb.ptr, pb.nbytes)
            assert nb == lay.nbytes
            self.pinned[layer_idx] = pb
        return pb

    def prefetch(self, layer_idx: int) -> None:
        """Makes the layer resident (its blob packed into pinned memory on
        first use) and publishes it to the ready map: the completion of a
        prefetch in FlowCast's state machine.  Any thread may call it."""
        pb = self.pin(layer_idx)
        self.residency.publish(layer_idx, pb.ptr, self.layouts[layer_idx].nbytes, PRECISION_NF4)

    def take_ready(self, layer_idx: int, timeout: float = 0.5) -> ReadyLayer:
        """FlowCast::take_ready (flowcast/src/lib.rs:458-498): blocks until
        the layer is resident (``PrefetchMiss`` after ``timeout`` seconds;
        0.5 s is wait_for_layer's default, lib.rs:531-533), takes it, issues
        its H2D copy on the copy stream and returns the ReadyLayer."""
        lay = self.layouts[layer_idx]
        raw = _lib.Nf4sReadyLayer()
        lib = _lib.load()
        rc = lib.nf4s_take_ready_wait(self.dbuf.handle, self.residency.handle, layer_idx,
                                      _timeout_us(timeout), ctypes.byref(raw))
        if rc == NF4S_ERR_PREFETCH_MISS:
            raise PrefetchMiss(layer_idx, lib.nf4s_last_error_message().decode())
        _lib.check(rc)
        return ReadyLayer(layer_idx=layer_idx, slab_device_ptrs=[(0, raw.slab_device_ptr)],
                          copy_event=raw.copy_event, views=lay.views(raw.slab_device_ptr),
                          raw=raw, precision=PRECISIONS[raw.precision],
                          needs_decode=bool(raw.needs_decode))

    def retire_layer(self, layer: ReadyLayer, stream: torch.cuda.Stream) -> None:
        """The work enqueued so far on `stream` is the layer's last use."""
        _lib.check(_lib.load().nf4s_retire_layer(self.dbuf.handle, ctypes.byref(layer.raw),
                                                 stream.cuda_stream))

    def close(self) -> None:
        self.dbuf.close()
        self.residency.close()
        for pb in self.pinned.values():
            pb.close()
        self.pinned.clear()


def stream_layers(seam: FlowCastSeam, order: Sequence[int], compute,
                  stream: torch.cuda.Stream, prefetch: bool = True,
                  timeout: float = 0.5) -> None:
    """The consumer loop of the double pass over the seam: the next layer's
    copy is issued before the current layer's kernels, the compute stream
    waits on each copy event, and each layer retires after its kernels.
    ``compute(layer_idx, views)`` enqueues the kernels on the current stream.
    With ``prefetch`` (the default) each layer is published here just before
    it is taken; without it another thread publishes them (``seam.prefetch``)
    and ``take_ready`` waits up to ``timeout`` seconds for each."""
    order = list(order)
    if not order:
        return

    def take(l):
        if prefetch:
            seam.prefetch(l)
        return seam.take_ready(l, timeout)

    cur = take(order[0])
    for i, l in enumerate(order):
        nxt = take(order[i + 1]) if i + 1 < len(order) else None
        stream_wait_event(stream, cur.copy_event)
        with torch.cuda.stream(stream):
            compute(l, cur.views)
        seam.retire_layer(cur, stream)
        cur = nxt
