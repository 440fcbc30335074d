"""CPU oracle for the NF4 streamed-weight path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product package ``aethelstream_amd`` never imports it.

Thin ctypes wrapper over ``oracle/_build/libnf4oracle.so`` (built from
``nf4_oracle.c`` by ``oracle/Makefile``); each wrapped function cites the
reference file:line it restates in ``nf4_oracle.h``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libnf4oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, strict IEEE fp32)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i64, i32 = ctypes.c_int64, ctypes.c_int32
        L.or_codebook.argtypes = [P]
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_nf4_code_argmin.argtypes = [ctypes.c_float]
        L.or_nf4_code_argmin.restype = ctypes.c_uint8
        L.or_nf4_code_bracket.argtypes = [ctypes.c_float]
        L.or_nf4_code_bracket.restype = ctypes.c_uint8
        L.or_check_bracket_exhaustive.argtypes = [ctypes.c_int]
        L.or_check_bracket_exhaustive.restype = i64
        L.or_check_steps_exhaustive.argtypes = [P, ctypes.c_int]
        L.or_check_steps_exhaustive.restype = i64
        L.or_quantize_nf4.argtypes = [P, i64, i32, P, P]
        L.or_dq_encode.argtypes = [P, i64, i32, P, P]
        L.or_dq_decode.argtypes = [P, P, i64, i32, P]
        for name in ("or_dequant_f16", "or_dequant_bf16", "or_dequant_f32"):
            f = getattr(L, name)
            f.argtypes = [P, i64, P, i64, P, i64, i32]
            f.restype = ctypes.c_int
        L.or_matmul_tb.argtypes = [P, P, i64, i64, i64, P]
        L.or_dgrad.argtypes = [P, P, i64, i64, i64, P]
        L.or_wgrad.argtypes = [P, P, i64, i64, i64, P]
        L.or_rmsnorm_fwd.argtypes = [P, P, i64, i64, ctypes.c_float, P, P, P]
        L.or_gen_normal.argtypes = [ctypes.c_uint64, i64, ctypes.c_double, P]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def codebook() -> np.ndarray:
    out = np.zeros(16, np.float32)
    lib().or_codebook(_p(out))
    return out


def gen_normal(seed: int, n: int, sigma: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_gen_normal(seed, n, sigma, _p(out))
    return out


def quantize_nf4(x: np.ndarray, block_size: int = 64):
    """quantizer.py:21-53 -> (packed uint8[ceil(n/2)], absmax f32[ceil(n/bs)])."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    n = x.size
    packed = np.zeros((n + 1) // 2, np.uint8)
    absmax = np.zeros((n + block_size - 1) // block_size, np.float32)
    lib().or_quantize_nf4(_p(x), n, block_size, _p(packed), _p(absmax))
    return packed, absmax


def dq_encode(absmax: np.ndarray, group: int = 256):
    absmax = np.ascontiguousarray(absmax, np.float32)
    nb = absmax.size
    q = np.zeros(nb, np.uint8)
    scale = np.zeros((nb + group - 1) // group, np.float32)
    lib().or_dq_encode(_p(absmax), nb, group, _p(q), _p(scale))
    return q, scale


def dq_decode(q: np.ndarray, scale: np.ndarray, group: int = 256) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    scale = np.ascontiguousarray(scale, np.float32)
    out = np.zeros(q.size, np.float32)
    lib().or_dq_decode(_p(q), _p(scale), q.size, group, _p(out))
    return out


def _dequant(fn, dtype, packed, absmax, n, block_size):
    packed = np.ascontiguousarray(packed, np.uint8)
    absmax = np.ascontiguousarray(absmax, np.float32)
    out = np.zeros(n, dtype)
    rc = fn(_p(packed), packed.size, _p(absmax), absmax.size, _p(out), n, block_size)
    if rc == 1:
        raise ValueError("absmax too small")
    if rc == 2:
        raise ValueError("packed too small")
    return out


def dequant_f16(packed, absmax, n, block_size=64) -> np.ndarray:
    """nf4.rs:37-83, f16 bits as uint16."""
    return _dequant(lib().or_dequant_f16, np.uint16, packed, absmax, n, block_size)


def dequant_bf16(packed, absmax, n, block_size=64) -> np.ndarray:
    """nf4.rs:37-83 with bf16 RNE output, bits as uint16."""
    return _dequant(lib().or_dequant_bf16, np.uint16, packed, absmax, n, block_size)


def dequant_f32(packed, absmax, n, block_size=64) -> np.ndarray:
    return _dequant(lib().or_dequant_f32, np.float32, packed, absmax, n, block_size)


def matmul_tb(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """math.rs:9-21: a[m,k] . b[n,k]^T in fp32 (sequential k sum)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    n = b.shape[0]
    c = np.zeros((m, n), np.float32)
    lib().or_matmul_tb(_p(a), _p(b), m, k, n, _p(c))
    return c


def dgrad(dy: np.ndarray, w: np.ndarray) -> np.ndarray:
    """backward.rs:160-168: dy[m,n] . w[n,k] in fp32."""
    dy = np.ascontiguousarray(dy, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, n = dy.shape
    k = w.shape[1]
    dx = np.zeros((m, k), np.float32)
    lib().or_dgrad(_p(dy), _p(w), m, n, k, _p(dx))
    return dx


def wgrad(dy: np.ndarray, x: np.ndarray, dw: np.ndarray = None) -> np.ndarray:
    """backward.rs:87-93: dw[n,k] (+)= sum_m dy[m,n] x[m,k] in fp32."""
    dy = np.ascontiguousarray(dy, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    m, n = dy.shape
    k = x.shape[1]
    out = np.zeros((n, k), np.float32) if dw is None else np.array(dw, np.float32, copy=True)
    lib().or_wgrad(_p(dy), _p(x), m, n, k, _p(out))
    return out


def rmsnorm_fwd(x: np.ndarray, w: np.ndarray, eps: float = 1e-6):
    """math.rs:36-59: returns (y, x_hat, rms) in fp32."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, d = x.shape
    y = np.zeros((m, d), np.float32)
    xh = np.zeros((m, d), np.float32)
    rms = np.zeros(m, np.float32)
    lib().or_rmsnorm_fwd(_p(x), _p(w), m, d, eps, _p(y), _p(xh), _p(rms))
    return y, xh, rms


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Vectorised RNE (same rule as or_f32_to_bf16) for finite inputs."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
