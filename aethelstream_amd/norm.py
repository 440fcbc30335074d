"""RMSNorm forward on the device, producing the fused GEMMs' bf16 operand.

``rms_norm_fwd`` replaces rms_norm_fwd (doublepass/src/math.rs:28-59) at
single_layer_forward's two call sites (doublepass/src/forward.rs:173, 249),
whose output is the input of the q/k/v and gate/up GEMMs.  The reference
returns (y, x_hat, rms) in fp32; here y leaves as bf16 (the GEMM operand) and
rms as fp32 (x_hat = x / rms is recomputed where the backward needs it).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from .nf4 import _require_cuda, _stream_ptr

EPS = 1e-6  # math.rs:45


def rms_norm_fwd(x: torch.Tensor, w: torch.Tensor, eps: float = EPS,
                 out: Optional[torch.Tensor] = None,
                 rms: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [M, d] fp32, w [d] fp32 -> (y [M, d] bf16, rms [M] fp32)."""
    _require_cuda(x, w)
    if x.dtype != torch.float32 or w.dtype != torch.float32:
        raise ValueError("x and w must be float32")
    if x.dim() != 2 or w.dim() != 1 or w.shape[0] != x.shape[1]:
        raise ValueError(f"x must be [M, d] and w [d], got {list(x.shape)} and {list(w.shape)}")
    if not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("x and w must be contiguous")
    m, d = int(x.shape[0]), int(x.shape[1])
    if out is None:
        out = torch.empty(m, d, dtype=torch.bfloat16, device=x.device)
    if rms is None:
        rms = torch.empty(m, dtype=torch.float32, device=x.device)
    # A caller's out / rms is written by the kernel: it must be contiguous
    # device memory on x's device (a host tensor's pointer would reach the
    # kernel, a strided one would be overwritten as if contiguous).
    _require_cuda(out, rms)
    if out.device != x.device or rms.device != x.device:
        raise ValueError("out and rms must be on x's device")
    if out.dtype != torch.bfloat16 or list(out.shape) != [m, d]:
        raise ValueError("out must be a contiguous bfloat16 [M, d] tensor")
    if rms.dtype != torch.float32 or rms.numel() < m:
        raise ValueError("rms must hold M float32 values")
    _lib.check(_lib.load().nf4s_rmsnorm_fwd(x.data_ptr(), w.data_ptr(), m, d, float(eps),
                                            out.data_ptr(), rms.data_ptr(), _stream_ptr(x)))
    return out, rms
