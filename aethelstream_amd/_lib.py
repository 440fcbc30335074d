"""ctypes binding of libnf4stream.so (the C ABI declared in include/nf4stream.h).

The library is the only compute path: if it is missing this module raises,
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libnf4stream.so")

NF4S_OK = 0
NF4S_ERR_INVALID_ARGUMENT = 1
NF4S_ERR_ABSMAX_TOO_SMALL = 2
NF4S_ERR_PACKED_TOO_SMALL = 3
NF4S_ERR_MISALIGNED = 4
NF4S_ERR_UNSUPPORTED_SHAPE = 5
NF4S_ERR_HIP = 6
NF4S_ERR_IO = 7
NF4S_ERR_JSON = 8
NF4S_ERR_LAYER_NOT_FOUND = 9
NF4S_ERR_PARAM_NOT_FOUND = 10
NF4S_ERR_MALFORMED_INDEX = 11


class Nf4sTensor(ctypes.Structure):
    """Mirror of ``struct nf4s_tensor`` (include/nf4stream.h)."""

    _fields_ = [
        ("packed", ctypes.c_void_p),
        ("packed_len", ctypes.c_int64),
        ("absmax", ctypes.c_void_p),
        ("absmax_q", ctypes.c_void_p),
        ("absmax_scale", ctypes.c_void_p),
        ("absmax_len", ctypes.c_int64),
        ("scale_len", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("dq_group", ctypes.c_int32),
    ]


class Nf4sParamInfo(ctypes.Structure):
    """Mirror of ``struct nf4s_param_info`` (include/nf4stream.h)."""

    _fields_ = [
        ("shape", ctypes.c_int64 * 8),
        ("ndim", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("numel", ctypes.c_int64),
        ("byte_length", ctypes.c_int64),
        ("absmax_len", ctypes.c_int64),
        ("scale_len", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("dq_group", ctypes.c_int32),
        ("out_elems", ctypes.c_int64),
        ("precision_str", ctypes.c_char * 16),
        ("dtype_str", ctypes.c_char * 16),
    ]


class Nf4sReadyLayer(ctypes.Structure):
    """Mirror of ``struct nf4s_ready_layer`` (include/nf4stream.h)."""

    _fields_ = [
        ("layer_idx", ctypes.c_uint32),
        ("slab_device_ptr", ctypes.c_void_p),
        ("bytes", ctypes.c_int64),
        ("copy_event", ctypes.c_void_p),
        ("precision", ctypes.c_int32),
        ("needs_decode", ctypes.c_int32),
    ]


class Nf4sBlobEntry(ctypes.Structure):
    """Mirror of ``struct nf4s_blob_entry`` (include/nf4stream.h)."""

    _fields_ = [
        ("packed_off", ctypes.c_int64),
        ("packed_len", ctypes.c_int64),
        ("absmax_off", ctypes.c_int64),
        ("absmax_len", ctypes.c_int64),
        ("scale_off", ctypes.c_int64),
        ("scale_len", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("dq_group", ctypes.c_int32),
    ]


# Every extern "C" symbol of include/nf4stream.h with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_TP = ctypes.POINTER(Nf4sTensor)
SIGNATURES = {
    "nf4s_abi_version": (_I32, []),
    "nf4s_strerror": (ctypes.c_char_p, [_I32]),
    "nf4s_last_error_message": (ctypes.c_char_p, []),
    "nf4s_quantize": (_I32, [_P, _I64, _I32, _P, _P, _P]),
    "nf4s_dq_encode": (_I32, [_P, _I64, _I32, _P, _P, _P]),
    "nf4s_quantize_bf16": (_I32, [_P, _I64, _I32, _P, _P, _P]),
    "nf4s_quantize_dq": (_I32, [_P, _I64, _I32, _I32, _P, _P, _P, _P]),
    "nf4s_quantize_dq_bf16": (_I32, [_P, _I64, _I32, _I32, _P, _P, _P, _P]),
    "nf4s_dequant_f16": (_I32, [_TP, _I64, _P, _P]),
    "nf4s_dequant_bf16": (_I32, [_TP, _I64, _P, _P]),
    "nf4s_dequant_batch_bf16": (_I32, [_TP, ctypes.POINTER(_I64), ctypes.POINTER(_P), _I32, _P]),
    "nf4s_gemm_fwd": (_I32, [_P, _TP, _I64, _I64, _I64, _P, _P]),
    "nf4s_gemm_dgrad": (_I32, [_P, _TP, _I64, _I64, _I64, _P, _P]),
    "nf4s_gemm_fwd_grouped": (_I32, [_P, _TP, ctypes.POINTER(_I64), ctypes.POINTER(_P), _I32,
                                     _I64, _I64, _P]),
    "nf4s_gemm_fwd_swiglu": (_I32, [_P, _TP, _TP, _I64, _I64, _I64, _P, _P]),
    "nf4s_gemm_dgrad_sum": (_I32, [ctypes.POINTER(_P), _TP, ctypes.POINTER(_I64), _I32, _I64,
                                   _I64, _P, _P]),
    "nf4s_gemm_dgrad_sum_ws": (_I32, [ctypes.POINTER(_P), _TP, ctypes.POINTER(_I64), _I32, _I64,
                                      _I64, _P, _P, _I64, _P]),
    "nf4s_gemm_dgrad_workspace_size": (_I32, [ctypes.POINTER(_I64), _I32, _I64, _I64,
                                              ctypes.POINTER(_I64)]),
    "nf4s_gemm_fwd_grouped_ws": (_I32, [_P, _TP, ctypes.POINTER(_I64), ctypes.POINTER(_P), _I32,
                                        _I64, _I64, _P, _I64, _P]),
    "nf4s_gemm_fwd_workspace_size": (_I32, [ctypes.POINTER(_I64), _I32, _I64, _I64,
                                            ctypes.POINTER(_I64)]),
    "nf4s_gemm_fwd_grouped_noalloc": (_I32, [_P, _TP, ctypes.POINTER(_I64), ctypes.POINTER(_P),
                                             _I32, _I64, _I64, _P]),
    "nf4s_gemm_wgrad": (_I32, [_P, _P, _I64, _I64, _I64, _P, _I32, _P]),
    "nf4s_gemm_wgrad_grouped": (_I32, [_P, _P, _P, _I32, _P, _I64, _I64, _I32, _P]),
    "nf4s_rmsnorm_fwd": (_I32, [_P, _P, _I64, _I64, ctypes.c_float, _P, _P, _P]),
    "nf4s_host_alloc": (_I32, [_I64, ctypes.POINTER(_P)]),
    "nf4s_host_free": (_I32, [_P]),
    "nf4s_dbuf_create": (_I32, [_I64, ctypes.POINTER(_P)]),
    "nf4s_dbuf_destroy": (_I32, [_P]),
    "nf4s_dbuf_capacity": (_I64, [_P]),
    "nf4s_dbuf_advance": (_I32, [_P, ctypes.c_uint32, _P, _I64, ctypes.POINTER(_P),
                                 ctypes.POINTER(_P)]),
    "nf4s_dbuf_release": (_I32, [_P, _P, _P]),
    "nf4s_stream_wait_event": (_I32, [_P, _P]),
    "nf4s_take_ready": (_I32, [_P, ctypes.c_uint32, _P, _I64, ctypes.POINTER(Nf4sReadyLayer)]),
    "nf4s_retire_layer": (_I32, [_P, ctypes.POINTER(Nf4sReadyLayer), _P]),
    "nf4s_residency_create": (_I32, [ctypes.c_uint32, ctypes.POINTER(_P)]),
    "nf4s_residency_destroy": (_I32, [_P]),
    "nf4s_residency_publish": (_I32, [_P, ctypes.c_uint32, _P, _I64, _I32]),
    "nf4s_residency_wait": (_I32, [_P, ctypes.c_uint32, _I64, ctypes.POINTER(_P),
                                   ctypes.POINTER(_I64), ctypes.POINTER(_I32)]),
    "nf4s_take_ready_wait": (_I32, [_P, _P, ctypes.c_uint32, _I64,
                                    ctypes.POINTER(Nf4sReadyLayer)]),
    "nf4s_loader_open": (_I32, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "nf4s_loader_close": (_I32, [_P]),
    "nf4s_loader_param_info": (_I32, [_P, ctypes.c_char_p, ctypes.POINTER(Nf4sParamInfo)]),
    "nf4s_loader_load_layer": (_I32, [_P, ctypes.c_uint32, ctypes.POINTER(_P),
                                      ctypes.POINTER(_I64)]),
    "nf4s_loader_staging_size": (_I32, [_P, ctypes.c_char_p, ctypes.POINTER(_I64)]),
    "nf4s_loader_load_param_f16": (_I32, [_P, ctypes.c_char_p, _P, _I64, _P, _I64, _P]),
    "nf4s_loader_load_param_nf4": (_I32, [_P, ctypes.c_char_p, _P, _I64, _P, _I64, _P, _I64,
                                          _P]),
    "nf4s_loader_pack_layer": (_I32, [_P, ctypes.POINTER(ctypes.c_char_p), _I32, _P, _I64,
                                      ctypes.POINTER(Nf4sBlobEntry), ctypes.POINTER(_I64)]),
    "nf4s_blob_tensor": (_I32, [ctypes.POINTER(Nf4sBlobEntry), _P, _TP]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libnf4stream.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m aethelstream_amd.build` "
                "(there is no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue  # tests/test_abi.py requires every declared symbol
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class Nf4sError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status
        self.message = message


def check(status: int) -> None:
    if status != NF4S_OK:
        lib = load()
        msg = lib.nf4s_last_error_message().decode()
        raise Nf4sError(status, msg or lib.nf4s_strerror(status).decode())
