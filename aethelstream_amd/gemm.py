"""NF4-dequant-fused GEMMs on the device (libnf4stream.so).

``linear_fwd``   y = x . W^T   replaces matmul_tb (doublepass/src/math.rs:9-21)
                 at the forward and recompute-forward call sites
                 (doublepass/src/forward.rs:174-176,244,251-252,255;
                 doublepass/src/backward.rs:447-451).
``linear_dgrad`` dx = dy . W   replaces the dY.W loops of single_layer_backward
                 (doublepass/src/backward.rs:79-85,117-129,160-168,284-300).

x / dy are bf16 [M, K] / [M, N] device tensors, W an :class:`Nf4Weight` of
shape [N, K]; accumulation is fp32 in MFMA, the output bf16.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .nf4 import Nf4Weight, _require_cuda, _stream_ptr


def _check_act(t: torch.Tensor, cols: int, name: str) -> None:
    _require_cuda(t)
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16")
    if t.dim() != 2 or t.shape[1] != cols:
        raise ValueError(f"{name} must be [M, {cols}], got {list(t.shape)}")


def linear_fwd(x: torch.Tensor, w: Nf4Weight, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y[M, N] = x[M, K] . W[N, K]^T (bf16 in/out, fp32 accumulate)."""
    n, k = int(w.shape[0]), int(w.shape[1])
    _check_act(x, k, "x")
    m = x.shape[0]
    if out is None:
        out = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    _check_act(out, n, "out")
    desc = w.descriptor()
    _lib.check(_lib.load().nf4s_gemm_fwd(x.data_ptr(), ctypes.byref(desc), m, n, k,
                                         out.data_ptr(), _stream_ptr(x)))
    return out


def linear_dgrad(dy: torch.Tensor, w: Nf4Weight,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dx[M, K] = dy[M, N] . W[N, K] (bf16 in/out, fp32 accumulate)."""
    n, k = int(w.shape[0]), int(w.shape[1])
    _check_act(dy, n, "dy")
    m = dy.shape[0]
    if out is None:
        out = torch.empty(m, k, dtype=torch.bfloat16, device=dy.device)
    _check_act(out, k, "out")
    desc = w.descriptor()
    _lib.check(_lib.load().nf4s_gemm_dgrad(dy.data_ptr(), ctypes.byref(desc), m, n, k,
                                           out.data_ptr(), _stream_ptr(dy)))
    return out


# Name of the reference function this replaces (math.rs:9).
matmul_tb = linear_fwd
