"""Streamed layer stack (flowcast VramDoubleBuffer semantics) on the GPU."""
import pytest
import torch

from aethelstream_amd import _lib, gemm, nf4
from aethelstream_amd import stream as st

pytestmark = pytest.mark.gpu
SHAPES = [("q", 256, 128), ("k", 64, 128), ("down", 128, 256)]


def _layers(n, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [[nf4.quantize_weight(torch.randn(r, c, device="cuda", generator=g) * 0.02,
                                 double_quant=True) for _, r, c in SHAPES] for _ in range(n)]


def test_streamed_outputs_equal_resident_outputs():
    n, m = 7, 192
    layout = st.LayerLayout(SHAPES)
    dev_layers = _layers(n)
    host = []
    for ws in dev_layers:
        pb = st.PinnedBuffer(layout.nbytes)
        layout.pack_into(pb.tensor, ws)
        host.append(pb)
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(m, 128, device="cuda", generator=g).to(torch.bfloat16)
    xd = torch.randn(m, 256, device="cuda", generator=g).to(torch.bfloat16)
    ins = [x, x, xd]
    ref = [[gemm.linear_fwd(a, w) for a, w in zip(ins, ws)] for ws in dev_layers]
    out = [[torch.empty(m, r, dtype=torch.bfloat16, device="cuda") for _, r, _ in SHAPES]
           for _ in range(n)]
    dbuf = st.VramDoubleBuffer(layout.nbytes)
    stream = torch.cuda.Stream()

    def compute(l, views):
        for a, w, y in zip(ins, views, out[l]):
            gemm.linear_fwd(a, w, y)

    # The host enqueues every layer without waiting: the events alone order
    # copies and kernels.
    torch.cuda.synchronize()
    st.run_stack(host, layout, dbuf, compute, stream)
    torch.cuda.synchronize()
    for l in range(n):
        for a, b in zip(out[l], ref[l]):
            assert torch.equal(a, b), f"layer {l} differs"
    dbuf.close()
    for pb in host:
        pb.close()


def test_slot_reuse_invariant_and_capacity_error():
    layout = st.LayerLayout(SHAPES)
    pb = st.PinnedBuffer(layout.nbytes)
    dbuf = st.VramDoubleBuffer(layout.nbytes)
    assert dbuf.slot_capacity() == layout.nbytes
    stream = torch.cuda.current_stream()
    ptrs = []
    for i in range(4):
        p, ev = dbuf.advance(i, pb.ptr, layout.nbytes)
        st.stream_wait_event(stream, ev)
        dbuf.release(p, stream)
        ptrs.append(p)
    # vram_double_buffer.rs:258-262: call N's buffer is reused at call N+2.
    assert ptrs[0] == ptrs[2] and ptrs[1] == ptrs[3] and ptrs[0] != ptrs[1]
    # vram_double_buffer.rs:269-275.
    with pytest.raises(_lib.Nf4sError, match="src len .* exceeds slot capacity"):
        dbuf.advance(9, pb.ptr, layout.nbytes + 1)
    with pytest.raises(_lib.Nf4sError, match="not a slot"):
        dbuf.release(pb.ptr, stream)
    torch.cuda.synchronize()
    dbuf.close()
    pb.close()


def test_layer_blob_roundtrip():
    layout = st.LayerLayout(SHAPES)
    ws = _layers(1, seed=3)[0]
    pb = st.PinnedBuffer(layout.nbytes)
    layout.pack_into(pb.tensor, ws)
    dev = pb.tensor.to("cuda")
    views = layout.views(dev.data_ptr())
    for v, w in zip(views, ws):
        a = nf4.dequant(w)
        b = torch.empty_like(a)
        import ctypes
        _lib.check(_lib.load().nf4s_dequant_bf16(ctypes.byref(v.descriptor()), b.numel(),
                                                 b.data_ptr(), 0))
        torch.cuda.synchronize()
        assert torch.equal(a, b)
    pb.close()
