"""NF4 shard I/O: the reference's on-disk format, written and read.

Writer: mirror of shard_engine/python/pipeline/writer.py:29-195 without the
network model load (``from_pretrained``): ``write_shards`` takes the tensors
directly.  Each NF4 parameter ``p`` is stored as ``p.__packed__`` (U8),
``p.__absmax__`` (F32) and ``p.__shape__`` (I32) in a safetensors file, and
``shard_index.json`` records absolute byte offsets (8 + header length +
data_offsets, writer.py:29-48).  With ``double_quant=True`` the absmax is
stored as ``p.__absmax_q__`` (U8) + ``p.__absmax_scale__`` (F32) and the entry
carries nf4_absmax_q_offset/_length, nf4_absmax_scale_offset/_length and
nf4_dq_group (an extension the reference's loader does not read).

Reader: ``ShardLoader`` wraps the C loader (aethelstream_amd/csrc/
nf4_loader.hip: mmap'd files, the reference's checks, device dequant) with
the reference's Rust API (shard_engine/src/loader.rs:42-206) and
``PyShardLoader`` with the PyO3 API and exception mapping
(shard_engine/src/ffi.rs:8-63).
"""
from __future__ import annotations

import ctypes
import json
import struct
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Dict, Iterable, List, Optional, Sequence, Tuple

import torch

from . import _lib
from .nf4 import BLOCK_SIZE, DQ_GROUP, Nf4Weight, check_fidelity, quantize_nf4, dq_encode, \
    _stream_ptr


# ---------------------------------------------------------------------------
# Errors (shard_engine/src/error.rs:5-28)
# ---------------------------------------------------------------------------
class ShardEngineError(Exception):
    """Base of the loader errors."""


class ShardIoError(ShardEngineError, IOError):
    """ShardEngineError::Io."""


class ShardJsonError(ShardEngineError, ValueError):
    """ShardEngineError::Json."""


class LayerNotFound(ShardEngineError, KeyError):
    """ShardEngineError::LayerNotFound."""


class ParamNotFound(ShardEngineError, KeyError):
    """ShardEngineError::ParamNotFound."""


class MalformedIndexEntry(ShardEngineError, ValueError):
    """ShardEngineError::MalformedIndex."""


_ERRORS = {
    _lib.NF4S_ERR_IO: ShardIoError,
    _lib.NF4S_ERR_JSON: ShardJsonError,
    _lib.NF4S_ERR_LAYER_NOT_FOUND: LayerNotFound,
    _lib.NF4S_ERR_PARAM_NOT_FOUND: ParamNotFound,
    _lib.NF4S_ERR_MALFORMED_INDEX: MalformedIndexEntry,
    _lib.NF4S_ERR_ABSMAX_TOO_SMALL: MalformedIndexEntry,
    _lib.NF4S_ERR_PACKED_TOO_SMALL: MalformedIndexEntry,
}


def _check(status: int) -> None:
    if status != _lib.NF4S_OK:
        msg = _lib.load().nf4s_last_error_message().decode()
        cls = _ERRORS.get(status)
        if cls is None:
            raise _lib.Nf4sError(status, msg)
        raise cls(msg)


# ---------------------------------------------------------------------------
# Writer (writer.py:29-195)
# ---------------------------------------------------------------------------
def read_safetensors_offsets(filepath) -> Dict[str, Tuple[int, int]]:
    """writer.py:29-48: {tensor: (absolute start, absolute end)}."""
    with open(filepath, "rb") as f:
        header_len = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(header_len).decode("utf-8"))
    base = 8 + header_len
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        if "data_offsets" not in info:
            raise ValueError(f"Tensor {name} missing data_offsets field")
        s, e = info["data_offsets"]
        out[name] = (base + s, base + e)
    return out


def write_shard(filepath, params: Iterable[Tuple[str, torch.Tensor]], precision: str,
                double_quant: bool = False, block_size: int = BLOCK_SIZE,
                dq_group: int = DQ_GROUP) -> Dict[str, dict]:
    """writer.py:50-132 for one shard file; returns its index entries.  NF4
    quantization runs on the device (bit-exact with quantize_nf4); a parameter
    whose round trip fails check_fidelity falls back to fp16 (writer.py:74-77)."""
    from safetensors.torch import save_file
    filepath = Path(filepath)
    to_save: Dict[str, torch.Tensor] = {}
    shapes: Dict[str, List[int]] = {}
    nf4_names = set()
    names = []
    for name, tensor in params:
        names.append(name)
        shapes[name] = list(tensor.shape)
        if precision == "nf4":
            dev = tensor.detach().to("cuda")
            r = quantize_nf4(dev, block_size)
            ok, _ = check_fidelity(dev, r)
            if not ok:
                to_save[name] = tensor.detach().cpu().to(torch.float16)
                continue
            nf4_names.add(name)
            to_save[f"{name}.__packed__"] = r.packed.cpu()
            if double_quant:
                q, s = dq_encode(r.absmax, dq_group)
                to_save[f"{name}.__absmax_q__"] = q.cpu()
                to_save[f"{name}.__absmax_scale__"] = s.cpu()
            else:
                to_save[f"{name}.__absmax__"] = r.absmax.cpu()
            to_save[f"{name}.__shape__"] = torch.tensor(r.original_shape, dtype=torch.int32)
        else:
            to_save[name] = tensor.detach().cpu().to(torch.float16)
    save_file(to_save, str(filepath))
    offs = read_safetensors_offsets(filepath)
    entries = {}
    for name in names:
        if name in nf4_names:
            ps, pe = offs[f"{name}.__packed__"]
            e = {"file_path": filepath.name, "byte_offset": ps, "byte_length": pe - ps,
                 "shape": shapes[name], "dtype": "U8", "precision": "nf4",
                 "nf4_block_size": block_size}
            if double_quant:
                qs, qe = offs[f"{name}.__absmax_q__"]
                ss, se = offs[f"{name}.__absmax_scale__"]
                e.update(nf4_absmax_q_offset=qs, nf4_absmax_q_length=qe - qs,
                         nf4_absmax_scale_offset=ss, nf4_absmax_scale_length=se - ss,
                         nf4_dq_group=dq_group)
            else:
                a_s, a_e = offs[f"{name}.__absmax__"]
                e.update(nf4_absmax_offset=a_s, nf4_absmax_length=a_e - a_s)
            entries[name] = e
        else:
            s, e_ = offs[name]
            entries[name] = {"file_path": filepath.name, "byte_offset": s, "byte_length": e_ - s,
                             "shape": shapes[name], "dtype": "F16", "precision": "fp16"}
    return entries


def write_shards(layers: Dict[object, List[Tuple[str, torch.Tensor]]], output_dir,
                 precision_of: Callable[[object], str] = lambda key: "nf4",
                 double_quant: bool = False) -> Tuple[dict, dict]:
    """writer.py:134-195 over given tensors: ``layers`` maps a layer index (or
    "embed" / "head" / "norm") to its parameters; one shard file per key;
    writes shard_index.json and layer_registry.json."""
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    shard_index, registry = {}, {}
    for key, params in layers.items():
        fname = f"layer_{key}.safetensors" if isinstance(key, int) else f"{key}.safetensors"
        shard_index.update(write_shard(out / fname, params, precision_of(key), double_quant))
        registry[str(key)] = fname
    with open(out / "shard_index.json", "w") as f:
        json.dump(shard_index, f, indent=2)
    with open(out / "layer_registry.json", "w") as f:
        json.dump(registry, f, indent=2)
    return shard_index, registry


# ---------------------------------------------------------------------------
# Reader (shard_engine/src/loader.rs)
# ---------------------------------------------------------------------------
@dataclass
class TensorBuffer:
    """loader.rs:6-20: FP16 bytes of one parameter."""

    data: bytes
    shape: List[int]
    dtype: str = "F16"
    param_name: str = ""


@dataclass
class LayerBuffer:
    """loader.rs:22-33: the raw safetensors bytes of a layer shard."""

    data: bytes
    layer_index: int
    file_path: str


class ShardLoader:
    """shard_engine/src/loader.rs:36-206 over the C loader."""

    def __init__(self, model_dir):
        self.model_dir = str(model_dir)
        h = ctypes.c_void_p()
        _check(_lib.load().nf4s_loader_open(self.model_dir.encode(), ctypes.byref(h)))
        self._h = h.value

    def close(self) -> None:
        if self._h:
            _lib.load().nf4s_loader_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def param_info(self, name: str) -> _lib.Nf4sParamInfo:
        info = _lib.Nf4sParamInfo()
        _check(_lib.load().nf4s_loader_param_info(self._h, name.encode(), ctypes.byref(info)))
        return info

    def load_layer(self, layer_index: int) -> LayerBuffer:
        """loader.rs:53-75."""
        p, n = ctypes.c_void_p(), ctypes.c_int64()
        _check(_lib.load().nf4s_loader_load_layer(self._h, layer_index, ctypes.byref(p),
                                                  ctypes.byref(n)))
        data = ctypes.string_at(p.value, n.value) if n.value else b""
        with open(Path(self.model_dir) / "layer_registry.json") as f:
            fname = json.load(f)[str(layer_index)]
        return LayerBuffer(data=data, layer_index=layer_index,
                           file_path=str(Path(self.model_dir) / fname))

    def load_param_device(self, name: str) -> torch.Tensor:
        """The parameter as a float16 device tensor (NF4 dequantized on the
        device; dequant_nf4_alloc length, nf4.rs:103)."""
        info = self.param_info(name)
        out = torch.empty(info.out_elems, dtype=torch.float16, device="cuda")
        nst = ctypes.c_int64()
        _check(_lib.load().nf4s_loader_staging_size(self._h, name.encode(), ctypes.byref(nst)))
        staging = torch.empty(max(nst.value, 1), dtype=torch.uint8, device="cuda")
        _check(_lib.load().nf4s_loader_load_param_f16(self._h, name.encode(), out.data_ptr(),
                                                      out.numel(), staging.data_ptr(),
                                                      nst.value, _stream_ptr(out)))
        # Dropping `staging` here is safe: the caching allocator reuses its
        # block for work on this same stream, which runs after the dequant.
        return out

    def load_param(self, name: str) -> TensorBuffer:
        """loader.rs:78-206: F16 little-endian bytes on the host."""
        info = self.param_info(name)
        dev = self.load_param_device(name)
        data = dev.view(torch.int16).cpu().numpy().tobytes()
        return TensorBuffer(data=data, shape=list(info.shape[:info.ndim]), dtype="F16",
                            param_name=name)

    def load_param_nf4(self, name: str) -> Nf4Weight:
        """The NF4 payload on the device, undecoded (for the fused GEMM)."""
        info = self.param_info(name)
        if info.precision == 0:
            raise MalformedIndexEntry(f"malformed index entry '{name}': not an nf4 parameter")
        shape = list(info.shape[:info.ndim])
        packed = torch.empty(info.byte_length, dtype=torch.uint8, device="cuda")
        dq = info.precision == 2
        if dq:
            am = torch.empty(info.absmax_len, dtype=torch.uint8, device="cuda")
            sc = torch.empty(info.scale_len, dtype=torch.float32, device="cuda")
        else:
            am = torch.empty(info.absmax_len, dtype=torch.float32, device="cuda")
            sc = None
        _check(_lib.load().nf4s_loader_load_param_nf4(
            self._h, name.encode(), packed.data_ptr(), packed.numel(), am.data_ptr(),
            am.numel() * am.element_size(), None if sc is None else sc.data_ptr(),
            0 if sc is None else 4 * sc.numel(), _stream_ptr(packed)))
        if dq:
            return Nf4Weight(packed=packed, absmax=None, shape=shape, block_size=info.block_size,
                             absmax_q=am, absmax_scale=sc, dq_group=info.dq_group)
        return Nf4Weight(packed=packed, absmax=am, shape=shape, block_size=info.block_size)


    def pack_layer(self, names: Sequence[str], dst_ptr: Optional[int] = None,
                   dst_bytes: int = 0) -> Tuple[List[_lib.Nf4sBlobEntry], int]:
        """The raw NF4 payloads of `names` packed into one host blob at
        `dst_ptr` (pinned memory for an asynchronous H2D copy); with no
        destination only the layout.  Returns (entries, blob bytes)."""
        n = len(names)
        arr = (ctypes.c_char_p * max(n, 1))(*[x.encode() for x in names])
        ents = (_lib.Nf4sBlobEntry * max(n, 1))()
        nb = ctypes.c_int64()
        _check(_lib.load().nf4s_loader_pack_layer(self._h, arr, n, dst_ptr, int(dst_bytes), ents,
                                                  ctypes.byref(nb)))
        return list(ents)[:n], nb.value


class PyShardLoader:
    """The PyO3 class of shard_engine/src/ffi.rs:8-63 with its exception mapping:
    construction and load_layer raise IOError, load_param KeyError when the
    message says "not found" else IOError, param_shape/param_precision KeyError."""

    def __init__(self, model_dir: str):
        try:
            self._inner = ShardLoader(model_dir)
        except ShardEngineError as e:
            raise IOError(str(e)) from None

    def load_layer(self, layer_index: int) -> bytes:
        try:
            return self._inner.load_layer(layer_index).data
        except ShardEngineError as e:
            raise IOError(str(e)) from None

    def load_param(self, param_name: str) -> bytes:
        try:
            return self._inner.load_param(param_name).data
        except ShardEngineError as e:
            msg = str(e)
            if "not found" in msg:
                raise KeyError(msg) from None
            raise IOError(msg) from None

    def param_shape(self, param_name: str) -> List[int]:
        try:
            info = self._inner.param_info(param_name)
        except ShardEngineError as e:
            raise KeyError(str(e)) from None
        return list(info.shape[:info.ndim])

    def param_precision(self, param_name: str) -> str:
        try:
            info = self._inner.param_info(param_name)
        except ShardEngineError as e:
            raise KeyError(str(e)) from None
        return info.precision_str.decode()
