"""nf4s_gemm_fwd_grouped_noalloc (the split-K forward on the library's static
per-GPU scratch) against nf4s_gemm_fwd_grouped_ws with a caller workspace,
both through the C ABI: bit-identical outputs on two calls in a row, the
second smaller, so stale partials of the first call would show in the second.
"""
import ctypes
import os
import subprocess
import sys

import pytest
import torch

from aethelstream_amd import _lib, nf4

pytestmark = pytest.mark.gpu


def _weights(shapes, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [nf4.quantize_weight(torch.randn(n, k, device="cuda", generator=g) * 0.02,
                                double_quant=dq) for n, k, dq in shapes]


def _args(ws, m):
    descs = (_lib.Nf4sTensor * len(ws))(*[w.descriptor() for w in ws])
    ns = (ctypes.c_int64 * len(ws))(*[w.shape[0] for w in ws])
    outs = [torch.full((m, w.shape[0]), float("nan"), dtype=torch.bfloat16, device="cuda")
            for w in ws]
    ys = (ctypes.c_void_p * len(ws))(*[o.data_ptr() for o in outs])
    return descs, ns, outs, ys


def _workspace_bytes(ns, count, m, k):
    b = ctypes.c_int64()
    _lib.check(_lib.load().nf4s_gemm_fwd_workspace_size(ns, count, m, k, ctypes.byref(b)))
    return b.value


def _run_pair(ws, m, k, seed):
    """Returns (noalloc outputs, workspace outputs, workspace bytes)."""
    lib = _lib.load()
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    d1, ns, out_na, ys1 = _args(ws, m)
    print(f"noalloc m={m} k={k} ns={list(ns)}", flush=True)
    _lib.check(lib.nf4s_gemm_fwd_grouped_noalloc(x.data_ptr(), d1, ns, ys1, len(ws), m, k,
                                                 stream))
    d2, ns2, out_ws, ys2 = _args(ws, m)
    nbytes = _workspace_bytes(ns2, len(ws), m, k)
    work = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
    _lib.check(lib.nf4s_gemm_fwd_grouped_ws(x.data_ptr(), d2, ns2, ys2, len(ws), m, k,
                                            work.data_ptr(), nbytes, stream))
    torch.cuda.synchronize()
    return out_na, out_ws, nbytes


def test_noalloc_equals_workspace_entry_point_twice():
    # Call 1: 8 output tiles on 256 CUs -> the largest split (64 MiB of
    # partials at 32 slices).  Call 2: fewer tiles, rows and steps, a ragged
    # m, and a double-quant + fp32-absmax pair (two launches on the scratch).
    cases = [
        (_weights([(640, 8192, True), (384, 8192, True)], 1), 512, 8192),
        (_weights([(256, 4096, True), (128, 4096, False)], 2), 300, 4096),
    ]
    for i, (ws, m, k) in enumerate(cases):
        a, b, nbytes = _run_pair(ws, m, k, seed=10 + i)
        assert nbytes > 0, "the case must take the split-K path"
        for ya, yb in zip(a, b):
            assert not torch.isnan(ya).any()
            assert torch.equal(ya, yb), f"call {i}: noalloc output differs"


def test_noalloc_without_split_matches_plain_forward():
    # Whole rounds (no split): the plain grouped forward, bit for bit.
    lib = _lib.load()
    ws = _weights([(128 * 256, 512, True)], 3)
    m, k = 512, 512
    x = torch.randn(m, k, device="cuda").to(torch.bfloat16)
    d, ns, out, ys = _args(ws, m)
    assert _workspace_bytes(ns, 1, m, k) == 0
    _lib.check(lib.nf4s_gemm_fwd_grouped_noalloc(x.data_ptr(), d, ns, ys, 1, m, k,
                                                 torch.cuda.current_stream().cuda_stream))
    d2, ns2, ref, ys2 = _args(ws, m)
    _lib.check(lib.nf4s_gemm_fwd_grouped(x.data_ptr(), d2, ns2, ys2, 1, m, k,
                                         torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(out[0], ref[0])


def test_noalloc_captured_in_a_graph_replays_bit_exact():
    """The entry point under HIP graph capture (its callers' case): one eager
    call first (loads the code object on this device), then the captured
    call (split-K launch + fixup on the static scratch, no memset) is
    replayed three times with new x contents written eagerly between the
    replays; every replay equals the workspace entry point run eagerly on the
    same x, bit for bit."""
    lib = _lib.load()
    ws = _weights([(640, 8192, True), (384, 8192, True)], 4)
    m, k = 512, 8192
    g = torch.Generator(device="cuda").manual_seed(20)
    x = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    d, ns, outs, ys = _args(ws, m)
    assert _workspace_bytes(ns, len(ws), m, k) > 0, "the case must take the split-K path"
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.nf4s_gemm_fwd_grouped_noalloc(x.data_ptr(), d, ns, ys, len(ws), m, k, stream))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(lib.nf4s_gemm_fwd_grouped_noalloc(
            x.data_ptr(), d, ns, ys, len(ws), m, k, torch.cuda.current_stream().cuda_stream))
    for rep in range(3):
        x.copy_(torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16))
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        d2, ns2, ref, ys2 = _args(ws, m)
        nbytes = _workspace_bytes(ns2, len(ws), m, k)
        work = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        _lib.check(lib.nf4s_gemm_fwd_grouped_ws(x.data_ptr(), d2, ns2, ys2, len(ws), m, k,
                                                work.data_ptr(), nbytes, stream))
        torch.cuda.synchronize()
        for a, b in zip(outs, ref):
            assert not torch.isnan(a).any(), f"replay {rep} left outputs unwritten"
            assert torch.equal(a, b), f"replay {rep} differs from the eager call"


_RESERVE_PROBE = r"""
import ctypes, sys, torch
sys.path.insert(0, sys.argv[1])
from aethelstream_amd import _lib, gemm, nf4
def free():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0]
lib = _lib.load()
w = nf4.quantize_weight(torch.randn(640, 8192, device="cuda") * 0.02, double_quant=True)
x = torch.randn(512, 8192, device="cuda").to(torch.bfloat16)
y = torch.empty(512, 640, dtype=torch.bfloat16, device="cuda")
gemm.linear_fwd(x, w)
gemm.linear_dgrad(torch.randn(512, 640, device="cuda").to(torch.bfloat16), w)
f0 = free()
d = (_lib.Nf4sTensor * 1)(w.descriptor())
ns = (ctypes.c_int64 * 1)(640)
ys = (ctypes.c_void_p * 1)(y.data_ptr())
_lib.check(lib.nf4s_gemm_fwd_grouped_noalloc(x.data_ptr(), d, ns, ys, 1, 512, 8192,
                                             torch.cuda.current_stream().cuda_stream))
f1 = free()
print(f0 - f1)
"""


def test_scratch_reserved_only_by_the_noalloc_entry_point():
    """The 64 MiB array lives in a code object of its own, which HIP loads on
    a GPU at its first use there.  In a fresh process the other GEMM entry
    points (forward with split-K, input gradient) leave it unreserved, and
    the first no-allocation call reserves it: device free memory drops by at
    least 64 MiB across that call alone (its outputs and inputs exist
    before)."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("fresh process: GEMM calls, then the first noalloc call", flush=True)
    r = subprocess.run([sys.executable, "-c", _RESERVE_PROBE, root], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    dropped = int(r.stdout.strip().splitlines()[-1])
    assert dropped >= 64 << 20, f"first noalloc call reserved only {dropped} bytes"
