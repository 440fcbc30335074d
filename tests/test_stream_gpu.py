"""Streamed layer stack (flowcast VramDoubleBuffer semantics) on the GPU."""
import ctypes
import threading
import time

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


def test_take_ready_wait_failed_copy_leaves_layer_taken():
    """nf4s_take_ready_wait takes the layer from the residency table before
    it issues the copy; a copy that fails (here a blob larger than the slot,
    vram_double_buffer.rs:269-275) returns the copy's error, and the layer
    stays taken, as the reference's take_ready drops the taken slot when its
    advance fails (flowcast/src/lib.rs:460-476): a second wait misses until
    the layer is published again, and the table itself stays usable."""
    layout = st.LayerLayout(SHAPES)
    pb = st.PinnedBuffer(layout.nbytes + 64)
    dbuf = st.VramDoubleBuffer(layout.nbytes)
    res = st.Residency(2)
    lib = _lib.load()
    out = _lib.Nf4sReadyLayer()
    res.publish(1, pb.ptr, layout.nbytes + 64, st.PRECISION_NF4)
    rc = lib.nf4s_take_ready_wait(dbuf.handle, res.handle, 1, 100000, ctypes.byref(out))
    assert rc == 1 and b"exceeds slot capacity" in lib.nf4s_last_error_message()
    with pytest.raises(st.PrefetchMiss, match="prefetch miss on layer 1"):
        res.wait(1, 0.02)
    res.publish(1, pb.ptr, layout.nbytes, st.PRECISION_NF4)
    _lib.check(lib.nf4s_take_ready_wait(dbuf.handle, res.handle, 1, 100000, ctypes.byref(out)))
    assert out.layer_idx == 1 and out.bytes == layout.nbytes
    assert out.precision == st.PRECISION_NF4 and out.needs_decode == 0
    stream = torch.cuda.current_stream()
    _lib.check(lib.nf4s_retire_layer(dbuf.handle, ctypes.byref(out),
                                     ctypes.c_void_p(stream.cuda_stream)))
    torch.cuda.synchronize()
    res.close()
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


LAYER_SHAPES = [("q", 256, 256), ("k", 64, 256), ("v", 64, 256), ("o", 256, 256),
                ("gate", 512, 256), ("up", 512, 256), ("down", 256, 512)]


def _write_model(root, n_layers, seed):
    from aethelstream_amd import shard
    g = torch.Generator(device="cuda").manual_seed(seed)
    layers = {l: [(f"model.layers.{l}.{nm}", torch.randn(r, c, device="cuda", generator=g) * 0.02)
                  for nm, r, c in LAYER_SHAPES] for l in range(n_layers)}
    shard.write_shards(layers, root, double_quant=True)
    return {l: [nm for nm, _ in ps] for l, ps in layers.items()}


def _layer_fwd(x, hid, views, outs):
    gemm.linear_fwd_grouped(x, views[0:3], outs[0:3])
    gemm.linear_fwd(x, views[3], outs[3])
    gemm.linear_fwd_grouped(x, views[4:6], outs[4:6])
    gemm.linear_fwd(hid, views[6], outs[6])


def test_flowcast_seam_streams_shard_layers(tmp_path):
    """Layers written by write_shards, packed from the shard files into pinned
    blobs by the loader, streamed through take_ready / retire_layer: each
    layer's 7 outputs equal the outputs over the same weights loaded resident
    (load_param_nf4), bit for bit."""
    from aethelstream_amd import shard
    n, m = 6, 320
    names = _write_model(tmp_path, n, seed=21)
    L = shard.ShardLoader(tmp_path)
    g = torch.Generator(device="cuda").manual_seed(22)
    x = torch.randn(m, 256, device="cuda", generator=g).to(torch.bfloat16)
    hid = torch.randn(m, 512, device="cuda", generator=g).to(torch.bfloat16)
    ref = []
    for l in range(n):
        ws = [L.load_param_nf4(nm) for nm in names[l]]
        outs = [torch.empty(m, r, dtype=torch.bfloat16, device="cuda") for _, r, _ in LAYER_SHAPES]
        _layer_fwd(x, hid, ws, outs)
        ref.append(outs)
    seam = st.FlowCastSeam(L, names)
    got = [[torch.full((m, r), float("nan"), dtype=torch.bfloat16, device="cuda")
            for _, r, _ in LAYER_SHAPES] for _ in range(n)]
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    # Forward order, then the recompute's reverse order (double pass).
    order = list(range(n)) + list(reversed(range(n)))
    seen = []

    def compute(l, views):
        seen.append(l)
        _layer_fwd(x, hid, views, got[l])

    st.stream_layers(seam, order, compute, stream)
    torch.cuda.synchronize()
    assert seen == order
    for l in range(n):
        for a, b in zip(got[l], ref[l]):
            assert torch.equal(a, b), f"layer {l} differs"
    # The same double pass with the layers published by another thread (the
    # prefetcher side of take_ready), each at most one layer ahead and after
    # a delay: take_ready blocks until the layer is resident.
    for outs in got:
        for o in outs:
            o.fill_(float("nan"))
    seen.clear()
    taken = [0]
    lock = threading.Condition()

    def prefetcher():
        for i, l in enumerate(order):
            with lock:
                lock.wait_for(lambda: taken[0] >= i - 1, timeout=10)
            time.sleep(0.002)
            seam.prefetch(l)

    def compute2(l, views):
        compute(l, views)
        with lock:
            taken[0] += 1
            lock.notify_all()

    th = threading.Thread(target=prefetcher)
    th.start()
    st.stream_layers(seam, order, compute2, stream, prefetch=False, timeout=10.0)
    th.join()
    torch.cuda.synchronize()
    assert seen == order
    for l in range(n):
        for a, b in zip(got[l], ref[l]):
            assert torch.equal(a, b), f"layer {l} differs (prefetcher thread)"
    # A layer nobody published: PrefetchMiss after the timeout.
    with pytest.raises(st.PrefetchMiss, match="prefetch miss on layer 4"):
        seam.take_ready(4, timeout=0.02)
    # Protocol errors: a second retire, and a take_ready into a slot whose
    # layer was never retired.
    for l in (0, 1, 2, 3):
        seam.prefetch(l)
    r0 = seam.take_ready(0)
    assert r0.precision == "NF4" and r0.needs_decode is False
    stream_c = torch.cuda.current_stream()
    st.stream_wait_event(stream_c, r0.copy_event)
    seam.retire_layer(r0, stream_c)
    with pytest.raises(_lib.Nf4sError, match="not handed out or is released"):
        seam.retire_layer(r0, stream_c)
    r1 = seam.take_ready(1)
    seam.take_ready(2)                       # the slot r0 held, released
    with pytest.raises(_lib.Nf4sError, match="which was not released"):
        seam.take_ready(3)                   # r1's slot: still held
    st.stream_wait_event(stream_c, r1.copy_event)
    seam.retire_layer(r1, stream_c)
    torch.cuda.synchronize()
    seam.close()
    L.close()


LAYER_70B = [("q", 8192, 8192), ("k", 1024, 8192), ("v", 1024, 8192), ("o", 8192, 8192),
             ("gate", 28672, 8192), ("up", 28672, 8192), ("down", 8192, 28672)]


def test_config5_80_streamed_70b_layers():
    """Benchmark config 5 at its workload: 80 double-quantized 70B-shaped
    layers (441 MB blobs) in pinned memory, 4096 tokens, streamed through the
    double buffer while the previous layer's fused forwards run.  The blobs
    alternate between two distinct layers, so a slot read before its copy
    completed (or refilled before its last reader finished) shows as the
    other layer's outputs.  Each layer's 7 outputs are compared on the compute
    stream, in stream order, with the resident outputs of its blob before the
    next layer overwrites them; one layer is also checked against fp32."""
    M, nlayers = 4096, 80
    layout = st.LayerLayout(LAYER_70B)
    assert layout.nbytes == 441397248
    g = torch.Generator(device="cuda").manual_seed(50)
    distinct = []
    for s in range(2):
        gw = torch.Generator(device="cuda").manual_seed(100 + s)
        distinct.append([nf4.quantize_weight(torch.randn(r, c, device="cuda", generator=gw) * 0.02,
                                             double_quant=True) for _, r, c in LAYER_70B])
    print(f"config5: packing {nlayers} pinned blobs of {layout.nbytes} B", flush=True)
    host = []
    for l in range(nlayers):
        pb = st.PinnedBuffer(layout.nbytes)
        layout.pack_into(pb.tensor, distinct[l % 2])
        host.append(pb)
    x = torch.randn(M, 8192, device="cuda", generator=g).to(torch.bfloat16)
    hid = torch.randn(M, 28672, device="cuda", generator=g).to(torch.bfloat16)
    ins = [x, x, x, x, x, x, hid]
    ref = []
    for ws in distinct:
        outs = [torch.empty(M, r, dtype=torch.bfloat16, device="cuda") for _, r, _ in LAYER_70B]
        _layer_fwd(x, hid, ws, outs)
        ref.append(outs)
    outs = [torch.full((M, r), float("nan"), dtype=torch.bfloat16, device="cuda")
            for _, r, _ in LAYER_70B]
    bad = torch.zeros(nlayers, dtype=torch.int32, device="cuda")
    dbuf = st.VramDoubleBuffer(layout.nbytes)
    stream = torch.cuda.Stream()

    def compute(l, views):
        _layer_fwd(x, hid, views, outs)
        # On the compute stream, before layer l+1's kernels are enqueued.
        diff = torch.stack([(a != b).any() for a, b in zip(outs, ref[l % 2])])
        bad[l] = diff.to(torch.int32).sum()

    torch.cuda.synchronize()
    print("config5: streaming", flush=True)
    st.run_stack(host, layout, dbuf, compute, stream)
    torch.cuda.synchronize()
    assert bad.sum().item() == 0, f"layers with differing outputs: {bad.nonzero().flatten().tolist()}"
    # The resident outputs of blob 0 (equal to streamed layers 0, 2, ...)
    # against fp32 over the dequantized weights.
    for (nm, r, c), w, a, y in zip(LAYER_70B, distinct[0], ins, ref[0]):
        wf = nf4.dequant(w).float()
        yf = a.float() @ wf.t()
        rel = ((y.float() - yf).norm() / yf.norm()).item()
        assert rel <= 4e-3, f"{nm}: rel-L2 {rel:.3e} vs fp32"
        del wf, yf
    dbuf.close()
    for pb in host:
        pb.close()
