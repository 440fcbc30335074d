"""NF4 codec on the GPU: the reference's quantizer and dequant interfaces.

Host-side mirror of
  * shard_engine/src/nf4.rs:6-107 (``NF4_CODES``, ``dequant_nf4_into``,
    ``dequant_nf4_alloc``) with the error behaviour of
    shard_engine/src/error.rs:5-28 (``MalformedIndex``), and
  * shard_engine/python/pipeline/quantizer.py:5-81 (``quantize_nf4``,
    ``Nf4Result``, ``dequantize_nf4``, ``check_fidelity``),
over device (``cuda``) torch tensors.  Every computation runs in
libnf4stream.so; torch only provides device memory and the current stream.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _lib

BLOCK_SIZE = 64          # quantizer.py:12
DQ_GROUP = 256           # blocks per double-quant scale

# shard_engine/src/nf4.rs:6-23
NF4_CODES = torch.tensor([
    -1.0, -0.6961928, -0.52507305, -0.3949175,
    -0.28444138, -0.18477343, -0.09105004, 0.0,
    0.0795803, 0.1609302, 0.2461123, 0.33791524,
    0.44070983, 0.562617, 0.72295684, 1.0,
], dtype=torch.float32)


class ShardEngineError(Exception):
    """shard_engine/src/error.rs:5-28."""


class MalformedIndex(ShardEngineError):
    """``ShardEngineError::MalformedIndex(entry, detail)`` (error.rs:21-23)."""

    def __init__(self, entry: str, detail: str):
        super().__init__(f"malformed index entry '{entry}': {detail}")
        self.entry = entry
        self.detail = detail


def _stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_cuda(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None:
            if not t.is_cuda:
                raise ValueError("NF4 kernels take device tensors (got a CPU tensor)")
            if not t.is_contiguous():
                raise ValueError("NF4 kernels take contiguous tensors")


@dataclass
class Nf4Weight:
    """A device-resident NF4 tensor: packed nibbles plus per-block absmax,
    either fp32 (the reference format, shard_engine/src/index.rs:27-33) or
    double-quantized (uint8 codes + one fp32 scale per ``dq_group`` blocks)."""

    packed: torch.Tensor                  # uint8 [ceil(numel/2)]
    absmax: Optional[torch.Tensor]        # float32 [nblocks] or None
    shape: list = field(default_factory=list)
    block_size: int = BLOCK_SIZE
    absmax_q: Optional[torch.Tensor] = None      # uint8 [nblocks]
    absmax_scale: Optional[torch.Tensor] = None  # float32 [ceil(nblocks/dq_group)]
    dq_group: int = 0

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n

    @property
    def double_quant(self) -> bool:
        return self.absmax_q is not None

    def descriptor(self) -> _lib.Nf4sTensor:
        _require_cuda(self.packed, self.absmax, self.absmax_q, self.absmax_scale)
        am = self.absmax_q if self.double_quant else self.absmax
        return _lib.Nf4sTensor(
            packed=_ptr(self.packed),
            packed_len=self.packed.numel(),
            absmax=None if self.double_quant else _ptr(self.absmax),
            absmax_q=_ptr(self.absmax_q),
            absmax_scale=_ptr(self.absmax_scale),
            absmax_len=0 if am is None else am.numel(),
            scale_len=0 if self.absmax_scale is None else self.absmax_scale.numel(),
            block_size=self.block_size,
            dq_group=self.dq_group if self.double_quant else 0,
        )

    def nbytes(self) -> int:
        b = self.packed.numel()
        if self.double_quant:
            b += self.absmax_q.numel() + 4 * self.absmax_scale.numel()
        else:
            b += 4 * self.absmax.numel()
        return b


def _raise_malformed(exc: _lib.Nf4sError) -> None:
    if exc.status == _lib.NF4S_ERR_ABSMAX_TOO_SMALL:
        raise MalformedIndex("nf4_absmax", exc.message) from None
    if exc.status == _lib.NF4S_ERR_PACKED_TOO_SMALL:
        raise MalformedIndex("nf4_packed", exc.message) from None
    raise exc


def _dequant(w: Nf4Weight, out: torch.Tensor, f16: bool) -> None:
    _require_cuda(out)
    lib = _lib.load()
    desc = w.descriptor()
    fn = lib.nf4s_dequant_f16 if f16 else lib.nf4s_dequant_bf16
    try:
        _lib.check(fn(ctypes.byref(desc), out.numel(), out.data_ptr(), _stream_ptr(out)))
    except _lib.Nf4sError as e:
        _raise_malformed(e)


def dequant_nf4_into(packed: torch.Tensor, absmax: torch.Tensor, output: torch.Tensor,
                     block_size: int) -> None:
    """shard_engine/src/nf4.rs:37-83 on the device: fills ``output`` (float16 or
    bfloat16, length n) with cvt(code[nibble] * absmax[block]).  Raises
    ``MalformedIndex`` where the reference returns it (nf4.rs:46-57)."""
    if output.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("output must be float16 or bfloat16")
    w = Nf4Weight(packed=packed, absmax=absmax, shape=[output.numel()], block_size=block_size)
    _dequant(w, output, f16=output.dtype == torch.float16)


def dequant_nf4_alloc(packed: torch.Tensor, absmax: torch.Tensor, block_size: int,
                      dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """shard_engine/src/nf4.rs:98-107: n = 2 * len(packed) elements."""
    out = torch.empty(2 * packed.numel(), dtype=dtype, device=packed.device)
    dequant_nf4_into(packed, absmax, out, block_size)
    return out


def dequant(w: Nf4Weight, dtype: torch.dtype = torch.bfloat16,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dequantize a (possibly double-quantized) weight to its original shape."""
    if out is None:
        out = torch.empty(w.shape, dtype=dtype, device=w.packed.device)
    _dequant(w, out, f16=out.dtype == torch.float16)
    return out


def dequant_batch(ws: list, outs: Optional[list] = None) -> list:
    """Dequantize several weights (e.g. one decoder layer) to bf16 in one launch."""
    if outs is None:
        outs = [torch.empty(w.shape, dtype=torch.bfloat16, device=w.packed.device) for w in ws]
    for o in outs:
        _require_cuda(o)
    k = len(ws)
    descs = (_lib.Nf4sTensor * k)(*[w.descriptor() for w in ws])
    ns = (ctypes.c_int64 * k)(*[o.numel() for o in outs])
    ptrs = (ctypes.c_void_p * k)(*[o.data_ptr() for o in outs])
    lib = _lib.load()
    stream = _stream_ptr(outs[0]) if k else 0
    try:
        _lib.check(lib.nf4s_dequant_batch_bf16(descs, ns, ptrs, k, stream))
    except _lib.Nf4sError as e:
        _raise_malformed(e)
    return outs


@dataclass
class Nf4Result:
    """quantizer.py:14-19."""

    packed: torch.Tensor
    absmax: torch.Tensor
    original_shape: list
    block_size: int = BLOCK_SIZE


def quantize_nf4(tensor: torch.Tensor, block_size: int = BLOCK_SIZE) -> Nf4Result:
    """quantizer.py:21-53 on the device (bit-exact codes and absmax)."""
    if not tensor.is_cuda:
        raise ValueError("quantize_nf4 runs on the device: pass a cuda tensor")
    original_shape = list(tensor.shape)
    flat = _flat_input(tensor, block_size)
    n = flat.numel()
    packed = torch.empty((n + 1) // 2, dtype=torch.uint8, device=flat.device)
    absmax = torch.empty((n + block_size - 1) // block_size, dtype=torch.float32,
                         device=flat.device)
    _quantize_into(flat, block_size, packed, absmax)
    return Nf4Result(packed=packed, absmax=absmax, original_shape=original_shape,
                     block_size=block_size)


def _flat_input(tensor: torch.Tensor, block_size: int) -> torch.Tensor:
    """The values to quantize as a flat device tensor: bf16 is kept as is
    (the kernels widen it exactly) when block_size is 64, anything else is
    converted to fp32."""
    t = tensor.detach()
    if t.dtype == torch.bfloat16 and block_size == BLOCK_SIZE:
        return t.contiguous().reshape(-1)
    return t.float().contiguous().reshape(-1)


def _quantize_into(flat: torch.Tensor, block_size: int, packed: torch.Tensor,
                   absmax: torch.Tensor) -> None:
    lib = _lib.load()
    fn = lib.nf4s_quantize_bf16 if flat.dtype == torch.bfloat16 else lib.nf4s_quantize
    _lib.check(fn(flat.data_ptr(), flat.numel(), block_size, packed.data_ptr(),
                  absmax.data_ptr(), _stream_ptr(flat)))


def _quantize_dq_into(flat: torch.Tensor, group: int, packed: torch.Tensor,
                      q: torch.Tensor, scale: torch.Tensor) -> None:
    lib = _lib.load()
    fn = lib.nf4s_quantize_dq_bf16 if flat.dtype == torch.bfloat16 else lib.nf4s_quantize_dq
    _lib.check(fn(flat.data_ptr(), flat.numel(), BLOCK_SIZE, group, packed.data_ptr(),
                  q.data_ptr(), scale.data_ptr(), _stream_ptr(flat)))


MAX_FUSED_DQ_GROUP = 8192   # nf4s_quantize_dq keeps a group's absmax in LDS


def dq_encode(absmax: torch.Tensor, group: int = DQ_GROUP):
    """Double-quantize per-block absmax -> (uint8 codes, fp32 scale per group)."""
    _require_cuda(absmax)
    nb = absmax.numel()
    q = torch.empty(nb, dtype=torch.uint8, device=absmax.device)
    scale = torch.empty((nb + group - 1) // group, dtype=torch.float32, device=absmax.device)
    lib = _lib.load()
    _lib.check(lib.nf4s_dq_encode(absmax.data_ptr(), nb, group, q.data_ptr(), scale.data_ptr(),
                                  _stream_ptr(absmax)))
    return q, scale


def quantize_weight(tensor: torch.Tensor, block_size: int = BLOCK_SIZE,
                    double_quant: bool = False, dq_group: int = DQ_GROUP) -> Nf4Weight:
    """Quantize a weight into an :class:`Nf4Weight`, optionally double-quantized
    (one fused launch for block 64 and groups up to MAX_FUSED_DQ_GROUP)."""
    if (double_quant and block_size == BLOCK_SIZE and tensor.is_cuda
            and 0 < dq_group <= MAX_FUSED_DQ_GROUP and dq_group & (dq_group - 1) == 0):
        flat = _flat_input(tensor, block_size)
        n = flat.numel()
        nb = (n + block_size - 1) // block_size
        packed = torch.empty((n + 1) // 2, dtype=torch.uint8, device=flat.device)
        q = torch.empty(nb, dtype=torch.uint8, device=flat.device)
        scale = torch.empty((nb + dq_group - 1) // dq_group, dtype=torch.float32,
                            device=flat.device)
        _quantize_dq_into(flat, dq_group, packed, q, scale)
        return Nf4Weight(packed=packed, absmax=None, shape=list(tensor.shape),
                         block_size=block_size, absmax_q=q, absmax_scale=scale,
                         dq_group=dq_group)
    r = quantize_nf4(tensor, block_size)
    w = Nf4Weight(packed=r.packed, absmax=r.absmax, shape=r.original_shape,
                  block_size=block_size)
    if double_quant:
        q, s = dq_encode(r.absmax, dq_group)
        w = Nf4Weight(packed=r.packed, absmax=None, shape=r.original_shape,
                      block_size=block_size, absmax_q=q, absmax_scale=s, dq_group=dq_group)
    return w


def requantize_(w: Nf4Weight, values: torch.Tensor) -> Nf4Weight:
    """Re-quantize `values` (fp32 or bf16, w.numel elements) into w's own
    buffers on the device, with w's block size and double-quant group: the
    weights an update step modified (doublepass/src/precision.rs:187-202)
    before their write-back (FlowCast::on_weights_updated,
    flowcast/src/lib.rs:501-521).  Allocates nothing on the device."""
    if not values.is_cuda:
        raise ValueError("requantize_ runs on the device: pass a cuda tensor")
    if values.numel() != w.numel:
        raise ValueError(f"requantize_ needs {w.numel} values, got {values.numel()}")
    if not values.is_contiguous():
        raise ValueError("requantize_ takes a contiguous tensor")
    flat = values.detach().reshape(-1)
    if not (flat.dtype == torch.bfloat16 and w.block_size == BLOCK_SIZE):
        if flat.dtype != torch.float32:
            raise ValueError("requantize_ takes float32 values (or bfloat16 for block 64)")
    if w.double_quant:
        if w.block_size != BLOCK_SIZE or w.dq_group > MAX_FUSED_DQ_GROUP:
            raise ValueError("requantize_ of double-quantized weights needs block 64 and "
                             f"dq_group <= {MAX_FUSED_DQ_GROUP}")
        _quantize_dq_into(flat, w.dq_group, w.packed, w.absmax_q, w.absmax_scale)
    else:
        _quantize_into(flat, w.block_size, w.packed, w.absmax)
    return w


def dequantize_nf4(result: Nf4Result) -> torch.Tensor:
    """quantizer.py:55-75: float16 tensor of the original shape."""
    w = Nf4Weight(packed=result.packed, absmax=result.absmax, shape=result.original_shape,
                  block_size=result.block_size)
    return dequant(w, dtype=torch.float16)


def check_fidelity(original: torch.Tensor, result: Nf4Result,
                   threshold: float = 1e-3) -> tuple:
    """quantizer.py:77-81: (mse <= threshold, mse)."""
    deq = dequantize_nf4(result)
    mse = ((original.float() - deq.float()) ** 2).mean().item()
    return mse <= threshold, mse
