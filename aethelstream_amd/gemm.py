"""NF4-dequant-fused GEMMs on the device (libnf4stream.so).

``linear_fwd``   y = x . W^T   replaces matmul_tb (doublepass/src/math.rs:9-21)
                 at the forward and recompute-forward call sites
                 (doublepass/src/forward.rs:174-176,244,251-252,255;
                 doublepass/src/backward.rs:447-451).
``linear_dgrad`` dx = dy . W   replaces the dY.W loops of single_layer_backward
                 (doublepass/src/backward.rs:79-85,117-129,160-168,284-300).
``linear_fwd_grouped``  y_i = x . W_i^T for weights sharing x, one launch
                 (q/k/v at forward.rs:174-176, gate/up at forward.rs:251-252).
``linear_swiglu``       hidden = silu(x . Wg^T) * (x . Wu^T), the SwiGLU of
                 forward.rs:251-254 fused into the GEMM epilogue.
``linear_dgrad_sum``    dx = sum_i dy_i . W_i, one launch and one rounding
                 (d_h1 at backward.rs:284-300, d_h2 at backward.rs:117-129).
``linear_wgrad``        dW = dy^T . x in fp32, the weight gradients beside them
``linear_wgrad_grouped`` up to 4 of them sharing x in one launch
                 (backward.rs:87-93, 117-129, 160-168, 284-300).

x / dy are bf16 [M, K] / [M, N] device tensors, W an :class:`Nf4Weight` of
shape [N, K]; accumulation is fp32 in MFMA, the output bf16.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

import torch

from . import _lib
from .nf4 import Nf4Weight, _require_cuda, _stream_ptr


def _check_act(t: torch.Tensor, cols: int, name: str) -> None:
    _require_cuda(t)
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16")
    if t.dim() != 2 or t.shape[1] != cols:
        raise ValueError(f"{name} must be [M, {cols}], got {list(t.shape)}")


def linear_fwd(x: torch.Tensor, w: Nf4Weight, out: Optional[torch.Tensor] = None,
               split_k: bool = True) -> torch.Tensor:
    """y[M, N] = x[M, K] . W[N, K]^T (bf16 in/out, fp32 accumulate).  With
    ``split_k`` a last round that would leave most CUs idle runs as split-K
    slices (nf4s_gemm_fwd_grouped_ws)."""
    n, k = int(w.shape[0]), int(w.shape[1])
    if split_k:
        return linear_fwd_grouped(x, [w], None if out is None else [out], split_k=True)[0]
    _check_act(x, k, "x")
    m = x.shape[0]
    if out is None:
        out = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    _check_act(out, n, "out")
    desc = w.descriptor()
    _lib.check(_lib.load().nf4s_gemm_fwd(x.data_ptr(), ctypes.byref(desc), m, n, k,
                                         out.data_ptr(), _stream_ptr(x)))
    return out


def linear_dgrad(dy: torch.Tensor, w: Nf4Weight, out: Optional[torch.Tensor] = None,
                 split_k: bool = True, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dx[M, K] = dy[M, N] . W[N, K] (bf16 in/out, fp32 accumulate).  With
    ``split_k`` a last round that would leave most CUs idle (few tokens) runs
    as split-K slices, as in :func:`linear_dgrad_sum`."""
    n, k = int(w.shape[0]), int(w.shape[1])
    _check_act(dy, n, "dy")
    m = dy.shape[0]
    if out is None:
        out = torch.empty(m, k, dtype=torch.bfloat16, device=dy.device)
    _check_act(out, k, "out")
    if split_k and dgrad_workspace_bytes([n], m, k) > 0:
        return linear_dgrad_sum([dy], [w], out, split_k=True, workspace=workspace)
    desc = w.descriptor()
    _lib.check(_lib.load().nf4s_gemm_dgrad(dy.data_ptr(), ctypes.byref(desc), m, n, k,
                                           out.data_ptr(), _stream_ptr(dy)))
    return out


def dgrad_workspace_bytes(ns: Sequence[int], m: int, k: int) -> int:
    """Workspace nf4s_gemm_dgrad_sum_ws uses for these shapes (0: no split)."""
    arr = (ctypes.c_int64 * len(ns))(*[int(v) for v in ns])
    out = ctypes.c_int64(0)
    _lib.check(_lib.load().nf4s_gemm_dgrad_workspace_size(arr, len(ns), m, k, ctypes.byref(out)))
    return int(out.value)


def _workspace_for(need: int, workspace: Optional[torch.Tensor], ref: torch.Tensor):
    """`workspace` if it holds `need` bytes, else a new buffer from torch's
    caching allocator on ref's device (and stream)."""
    if workspace is not None and workspace.device != ref.device:
        raise ValueError("workspace must be on the operands' device")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=ref.device)
    _require_cuda(workspace)
    if not workspace.is_contiguous():
        raise ValueError("workspace must be contiguous")
    return workspace


def _descs(ws: Sequence[Nf4Weight]):
    arr = (_lib.Nf4sTensor * len(ws))()
    for i, w in enumerate(ws):
        arr[i] = w.descriptor()
    return arr


def fwd_workspace_bytes(ns: Sequence[int], m: int, k: int) -> int:
    """Workspace nf4s_gemm_fwd_grouped_ws uses for these shapes (0: no split)."""
    arr = (ctypes.c_int64 * len(ns))(*[int(v) for v in ns])
    out = ctypes.c_int64(0)
    _lib.check(_lib.load().nf4s_gemm_fwd_workspace_size(arr, len(ns), m, k, ctypes.byref(out)))
    return int(out.value)


def linear_fwd_grouped(x: torch.Tensor, ws: Sequence[Nf4Weight],
                       outs: Optional[Sequence[torch.Tensor]] = None, split_k: bool = True,
                       workspace: Optional[torch.Tensor] = None) -> List[torch.Tensor]:
    """[x . W_i^T for W_i in ws] (1..4 weights of one k) in one launch.  With
    ``split_k`` a last round that would leave most CUs idle runs as split-K
    slices whose fp32 partials go to ``workspace`` (by default a buffer from
    torch's caching allocator on x's stream, so calls on other streams never
    share it)."""
    if not 1 <= len(ws) <= 4:
        raise ValueError("linear_fwd_grouped takes 1 to 4 weights")
    k = int(ws[0].shape[1])
    if any(int(w.shape[1]) != k for w in ws):
        raise ValueError("grouped weights must share k")
    _check_act(x, k, "x")
    m = x.shape[0]
    if outs is None:
        outs = [torch.empty(m, int(w.shape[0]), dtype=torch.bfloat16, device=x.device)
                for w in ws]
    if len(outs) != len(ws):
        raise ValueError("one output per weight")
    for w, o in zip(ws, outs):
        _check_act(o, int(w.shape[0]), "out")
    ns = (ctypes.c_int64 * len(ws))(*[int(w.shape[0]) for w in ws])
    ys = (ctypes.c_void_p * len(ws))(*[o.data_ptr() for o in outs])
    descs = _descs(ws)
    need = fwd_workspace_bytes(list(ns), m, k) if split_k else 0
    if need > 0:
        if workspace is not None and workspace.device != x.device:
            raise ValueError("workspace must be on x's device")
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
        _require_cuda(workspace)
        if not workspace.is_contiguous():
            raise ValueError("workspace must be contiguous")
        _lib.check(_lib.load().nf4s_gemm_fwd_grouped_ws(
            x.data_ptr(), descs, ns, ys, len(ws), m, k, workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), _stream_ptr(x)))
    else:
        _lib.check(_lib.load().nf4s_gemm_fwd_grouped(x.data_ptr(), descs, ns, ys, len(ws), m, k,
                                                     _stream_ptr(x)))
    return list(outs)


def linear_swiglu(x: torch.Tensor, w_gate: Nf4Weight, w_up: Nf4Weight,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """hidden[M, ff] = silu(x . Wg^T) * (x . Wu^T) (forward.rs:251-254; silu_f,
    math.rs:91-93): gate and up stay fp32 in the accumulators, hidden is bf16."""
    ff, k = int(w_gate.shape[0]), int(w_gate.shape[1])
    if [int(d) for d in w_up.shape] != [ff, k]:
        raise ValueError("gate and up weights must have the same shape")
    _check_act(x, k, "x")
    m = x.shape[0]
    if out is None:
        out = torch.empty(m, ff, dtype=torch.bfloat16, device=x.device)
    _check_act(out, ff, "out")
    dg, du = w_gate.descriptor(), w_up.descriptor()
    _lib.check(_lib.load().nf4s_gemm_fwd_swiglu(x.data_ptr(), ctypes.byref(dg), ctypes.byref(du),
                                                m, ff, k, out.data_ptr(), _stream_ptr(x)))
    return out


def linear_dgrad_sum(dys: Sequence[torch.Tensor], ws: Sequence[Nf4Weight],
                     out: Optional[torch.Tensor] = None, split_k: bool = True,
                     workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sum_i dys[i] . W_i (1..4 weights of one k): one launch, fp32 accumulation
    over all weights, one bf16 rounding.  With ``split_k`` a last round that
    would leave most CUs idle (few tokens) runs as split-K slices of the
    weights' concatenated reduction, whose fp32 partials go to ``workspace``
    (by default a buffer from torch's caching allocator on out's stream) and
    are summed in slice order by a second kernel."""
    if not 1 <= len(ws) <= 4 or len(dys) != len(ws):
        raise ValueError("linear_dgrad_sum takes 1 to 4 (dy, W) pairs")
    k = int(ws[0].shape[1])
    if any(int(w.shape[1]) != k for w in ws):
        raise ValueError("summed weights must share k")
    m = dys[0].shape[0]
    for dy, w in zip(dys, ws):
        _check_act(dy, int(w.shape[0]), "dy")
        if dy.shape[0] != m:
            raise ValueError("all dy must have the same number of rows")
    if out is None:
        out = torch.empty(m, k, dtype=torch.bfloat16, device=dys[0].device)
    _check_act(out, k, "out")
    ns = (ctypes.c_int64 * len(ws))(*[int(w.shape[0]) for w in ws])
    dps = (ctypes.c_void_p * len(ws))(*[d.data_ptr() for d in dys])
    descs = _descs(ws)
    need = dgrad_workspace_bytes(list(ns), m, k) if split_k else 0
    if need > 0:
        workspace = _workspace_for(need, workspace, out)
        _lib.check(_lib.load().nf4s_gemm_dgrad_sum_ws(
            dps, descs, ns, len(ws), m, k, out.data_ptr(), workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), _stream_ptr(out)))
    else:
        _lib.check(_lib.load().nf4s_gemm_dgrad_sum(dps, descs, ns, len(ws), m, k,
                                                   out.data_ptr(), _stream_ptr(out)))
    return out


def linear_wgrad(dy: torch.Tensor, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                 accumulate: bool = False) -> torch.Tensor:
    """dW[N, K] = dy[M, N]^T . x[M, K] in fp32 (bf16 inputs), or dW += that sum
    when ``accumulate`` (the micro-batch sum of backward.rs:478-502).  The
    weight gradients of single_layer_backward (backward.rs:87-93, 117-129,
    160-168, 284-300); no NF4 operand."""
    _require_cuda(dy, x)
    if dy.dtype != torch.bfloat16 or x.dtype != torch.bfloat16:
        raise ValueError("dy and x must be bfloat16")
    if dy.dim() != 2 or x.dim() != 2 or dy.shape[0] != x.shape[0]:
        raise ValueError(f"dy [M, N] and x [M, K] must share M, got {list(dy.shape)} and "
                         f"{list(x.shape)}")
    m, n, k = dy.shape[0], dy.shape[1], x.shape[1]
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs an existing out tensor")
        out = torch.empty(n, k, dtype=torch.float32, device=dy.device)
    _require_cuda(out)
    if out.dtype != torch.float32 or list(out.shape) != [n, k]:
        raise ValueError(f"out must be float32 [{n}, {k}]")
    _lib.check(_lib.load().nf4s_gemm_wgrad(dy.data_ptr(), x.data_ptr(), m, n, k, out.data_ptr(),
                                           1 if accumulate else 0, _stream_ptr(dy)))
    return out



def linear_wgrad_grouped(dys: Sequence[torch.Tensor], x: torch.Tensor,
                         outs: Optional[Sequence[torch.Tensor]] = None,
                         accumulate: bool = False) -> List[torch.Tensor]:
    """dW_i = dys[i]^T . x for up to 4 products sharing x, in one launch: the
    d_wq / d_wk / d_wv of backward.rs:284-300 (all from the attention input)
    or d_wg / d_wu of :117-129.  Each result is bit-identical to
    :func:`linear_wgrad` of that product."""
    _require_cuda(x, *dys)
    if not 1 <= len(dys) <= 4:
        raise ValueError(f"linear_wgrad_grouped takes 1 to 4 products, got {len(dys)}")
    if x.dtype != torch.bfloat16 or any(d.dtype != torch.bfloat16 for d in dys):
        raise ValueError("dys and x must be bfloat16")
    if x.dim() != 2 or any(d.dim() != 2 or d.shape[0] != x.shape[0] for d in dys):
        raise ValueError("every dy [M, N_i] must share M with x [M, K]")
    m, k = x.shape
    ns = [d.shape[1] for d in dys]
    if outs is None:
        if accumulate:
            raise ValueError("accumulate needs existing out tensors")
        outs = [torch.empty(n, k, dtype=torch.float32, device=x.device) for n in ns]
    outs = list(outs)
    if len(outs) != len(dys):
        raise ValueError("one out tensor per product")
    _require_cuda(*outs)
    for o, n in zip(outs, ns):
        if o.dtype != torch.float32 or list(o.shape) != [n, k]:
            raise ValueError(f"out must be float32 [{n}, {k}]")
    c = len(dys)
    dps = (ctypes.c_void_p * c)(*[d.data_ptr() for d in dys])
    ops = (ctypes.c_void_p * c)(*[o.data_ptr() for o in outs])
    nsa = (ctypes.c_int64 * c)(*ns)
    _lib.check(_lib.load().nf4s_gemm_wgrad_grouped(dps, nsa, ops, c, x.data_ptr(), m, k,
                                                   1 if accumulate else 0, _stream_ptr(x)))
    return outs

# Name of the reference function this replaces (math.rs:9).
matmul_tb = linear_fwd
