"""GPU parity of the NF4-fused GEMMs.

Small shapes: against the oracle's matmul_tb / dY.W loops (doublepass/src/
math.rs:9-21, backward.rs:160-168) fed with the reference's own weight path
(f16 dequant widened to fp32, shard_provider.rs:50-64), rel-L2 <= 1e-2 (the
north_star tolerance); and against fp32 on the same bf16 operands, rel-L2 <=
4e-3 (bf16 output rounding only).  Layer shapes (7B, 70B): against a torch
fp32 GPU matmul over the bit-checked bf16 dequantized weights, plus sampled
rows in fp64 on the CPU."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from aethelstream_amd import _lib, gemm, nf4

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_REF = 1e-2     # north_star: rel-L2 vs the reference fp32 path
TOL_SAME = 4e-3    # same bf16 operands: only the bf16 output rounding differs


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _weight(n, k, seed, dq=False):
    w32 = oracle.gen_normal(seed, n * k, 0.02)
    w = nf4.quantize_weight(torch.from_numpy(w32).to(DEV).view(n, k), double_quant=dq)
    return w


def _deq_host(w, f16: bool) -> np.ndarray:
    """Oracle dequant (fp32 values of the f16 or bf16 result) of a device weight."""
    pk = w.packed.cpu().numpy()
    if w.double_quant:
        am = oracle.dq_decode(w.absmax_q.cpu().numpy(), w.absmax_scale.cpu().numpy(), w.dq_group)
    else:
        am = w.absmax.cpu().numpy()
    n = w.numel
    if f16:
        return oracle.dequant_f16(pk, am, n).view(np.float16).astype(np.float32).reshape(w.shape)
    return oracle.bf16_bits_to_f32(oracle.dequant_bf16(pk, am, n)).reshape(w.shape)


def _act(m, k, seed):
    a = oracle.gen_normal(seed, m * k, 1.0)
    t = torch.from_numpy(a).to(DEV).view(m, k).to(torch.bfloat16)
    return t, t.float().cpu().numpy()


SMALL = [(1, 128, 64), (64, 128, 64), (512, 128, 128), (700, 300, 192), (513, 257, 320),
         (1024, 256, 1024)]


@pytest.mark.parametrize("m,n,k", SMALL)
@pytest.mark.parametrize("dq", [False, True])
def test_fwd_small_vs_oracle(m, n, k, dq):
    w = _weight(n, k, 11 + n + k, dq)
    x, xh = _act(m, k, 5 + m)
    y = gemm.linear_fwd(x, w)
    torch.cuda.synchronize()
    yh = y.float().cpu().numpy()
    ref = oracle.matmul_tb(xh, _deq_host(w, f16=True))          # reference numerics
    assert rel_l2(yh, ref) <= TOL_REF
    same = oracle.matmul_tb(xh, _deq_host(w, f16=False))        # same bf16 operands
    assert rel_l2(yh, same) <= TOL_SAME


# k % 256 == 0 takes the forward kernel with batched weight loads (two steps
# of packed nibbles and four steps of absmax per load); the shapes above
# with k % 256 != 0 take the per-step loads.
BATCHED = [(1, 64, 256), (700, 300, 256), (513, 257, 512), (64, 130, 768), (640, 192, 1024)]


@pytest.mark.parametrize("m,n,k", BATCHED)
@pytest.mark.parametrize("dq_group", [0, 4, 8, 256])
def test_fwd_batched_small_vs_oracle(m, n, k, dq_group):
    w32 = oracle.gen_normal(31 + n + k, n * k, 0.02)
    w = nf4.quantize_weight(torch.from_numpy(w32).to(DEV).view(n, k),
                            double_quant=dq_group > 0, dq_group=dq_group or nf4.DQ_GROUP)
    x, xh = _act(m, k, 9 + m)
    y = gemm.linear_fwd(x, w)
    torch.cuda.synchronize()
    yh = y.float().cpu().numpy()
    assert rel_l2(yh, oracle.matmul_tb(xh, _deq_host(w, f16=True))) <= TOL_REF
    assert rel_l2(yh, oracle.matmul_tb(xh, _deq_host(w, f16=False))) <= TOL_SAME


def _misaligned(t: torch.Tensor, by: int) -> torch.Tensor:
    """A copy of t whose data pointer is `by` elements past an allocation."""
    buf = torch.empty(t.numel() + by, dtype=t.dtype, device=t.device)
    v = buf[by:by + t.numel()]
    v.copy_(t)
    return v


@pytest.mark.parametrize("m,n,k", [(700, 300, 256), (513, 257, 1024), (1024, 256, 2048)])
@pytest.mark.parametrize("dq", [False, True])
def test_fwd_batched_equals_per_step(m, n, k, dq):
    # The same weights through both forward kernels: absmax (or its codes)
    # moved off the alignment the batched loads need selects the per-step
    # kernel.  Same products, same reduction order: bit-identical outputs.
    w = _weight(n, k, 41 + n + k, dq)
    x, _ = _act(m, k, 13 + m)
    y_batched = gemm.linear_fwd(x, w, split_k=False)
    if dq:
        w2 = nf4.Nf4Weight(packed=w.packed, absmax=None, shape=w.shape, absmax_q=_misaligned(w.absmax_q, 1),
                           absmax_scale=w.absmax_scale, dq_group=w.dq_group)
    else:
        w2 = nf4.Nf4Weight(packed=w.packed, absmax=_misaligned(w.absmax, 1), shape=w.shape)
    y_step = gemm.linear_fwd(x, w2, split_k=False)
    torch.cuda.synchronize()
    assert torch.equal(y_batched.view(torch.int16), y_step.view(torch.int16))


@pytest.mark.parametrize("m,n,k", [(700, 256, 128), (513, 512, 1024), (1024, 1024, 384)])
@pytest.mark.parametrize("dq_group", [0, 2, 256])
def test_dgrad_batched_equals_per_step(m, n, k, dq_group):
    # The input gradient's batched absmax loads (n % 256, k % 128) against the
    # per-step loads, selected by moving the absmax (or its codes) off the
    # alignment the pair loads need: same products, same reduction order,
    # bit-identical outputs.  dq_group 2: each scale covers exactly a pair.
    # Unsplit: the two producers' split-K slices are sized to their own step
    # granularity (4 and 2), which changes the fp32 order of a split sum.
    dq = dq_group > 0
    w32 = oracle.gen_normal(43 + n + k, n * k, 0.02)
    w = nf4.quantize_weight(torch.from_numpy(w32).to(DEV).view(n, k), double_quant=dq,
                            dq_group=dq_group or nf4.DQ_GROUP)
    dy, _ = _act(m, n, 11 + m)
    dx_batched = gemm.linear_dgrad(dy, w, split_k=False)
    if dq:
        w2 = nf4.Nf4Weight(packed=w.packed, absmax=None, shape=w.shape,
                           absmax_q=_misaligned(w.absmax_q, 1), absmax_scale=w.absmax_scale,
                           dq_group=w.dq_group)
    else:
        w2 = nf4.Nf4Weight(packed=w.packed, absmax=_misaligned(w.absmax, 1), shape=w.shape)
    dx_step = gemm.linear_dgrad(dy, w2, split_k=False)
    torch.cuda.synchronize()
    assert torch.equal(dx_batched.view(torch.int16), dx_step.view(torch.int16))


@pytest.mark.parametrize("m,n,k", [(1, 64, 128), (64, 128, 64), (512, 128, 128),
                                   (700, 320, 300 - 300 % 64 + 64), (513, 256, 320)])
@pytest.mark.parametrize("dq", [False, True])
def test_dgrad_small_vs_oracle(m, n, k, dq):
    w = _weight(n, k, 21 + n + k, dq)
    dy, dyh = _act(m, n, 7 + m)
    dx = gemm.linear_dgrad(dy, w)
    torch.cuda.synchronize()
    dxh = dx.float().cpu().numpy()
    ref = oracle.dgrad(dyh, _deq_host(w, f16=True))
    assert rel_l2(dxh, ref) <= TOL_REF
    same = oracle.dgrad(dyh, _deq_host(w, f16=False))
    assert rel_l2(dxh, same) <= TOL_SAME


def test_output_layout_exact_on_integer_data():
    # Small integers times exactly representable weights: every product and
    # partial sum is exact in fp32, so any misplaced row/column or reduction
    # index shows up as an exact mismatch.
    m, n, k = 512, 128, 128
    codes = np.arange(n * k) % 16
    packed = ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)
    absmax = np.ones(n * k // 64, np.float32)
    w = nf4.Nf4Weight(packed=torch.from_numpy(packed).to(DEV), absmax=torch.from_numpy(absmax).to(DEV),
                      shape=[n, k])
    rng = np.random.default_rng(0)
    x = rng.integers(-2, 3, (m, k)).astype(np.float32)
    y = gemm.linear_fwd(torch.from_numpy(x).to(DEV).to(torch.bfloat16), w).float().cpu().numpy()
    wd = _deq_host(w, f16=False).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T
    ref_bf = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(ref.astype(np.float32)))
    assert np.max(np.abs(y - ref_bf)) <= np.max(np.abs(ref)) * 2 ** -7
    dyh = rng.integers(-2, 3, (m, n)).astype(np.float32)
    dx = gemm.linear_dgrad(torch.from_numpy(dyh).to(DEV).to(torch.bfloat16), w).float().cpu().numpy()
    ref = dyh.astype(np.float64) @ wd
    assert np.max(np.abs(dx - ref)) <= np.max(np.abs(ref)) * 2 ** -7


def _layer_check(m, n, k, dq, seed, dgrad=False):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = nf4.quantize_weight(torch.randn(n, k, device=DEV, generator=g) * 0.02, double_quant=dq)
    wd = nf4.dequant(w)                                   # bf16, bit-checked kernel
    if not dgrad:
        x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
        y = gemm.linear_fwd(x, w)
        ref = x.float() @ wd.float().t()
    else:
        x = torch.randn(m, n, device=DEV, generator=g).to(torch.bfloat16)
        y = gemm.linear_dgrad(x, w)
        ref = x.float() @ wd.float()
    torch.cuda.synchronize()
    err = ((y.float() - ref).norm() / ref.norm()).item()
    assert err <= TOL_SAME, err
    # fp64 on the CPU for a few rows (independent of the GPU fp32 GEMM).
    rows = [0, m // 3, m - 1]
    xs = x[rows].double().cpu().numpy()
    wdh = wd.double().cpu().numpy()
    ref64 = xs @ (wdh if dgrad else wdh.T)
    assert rel_l2(y[rows].double().cpu().numpy(), ref64) <= TOL_SAME
    del w, wd, x, y, ref


@pytest.mark.parametrize("name,n,k", [("gate/up", 11008, 4096), ("down", 4096, 11008)])
def test_fwd_7b_shapes(name, n, k):
    # Benchmark config 3: 4096 tokens x NF4 W^T.
    _layer_check(4096, n, k, dq=True, seed=3)


@pytest.mark.parametrize("name,n,k", [("q/o", 8192, 8192), ("k/v", 1024, 8192),
                                      ("gate/up", 28672, 8192), ("down", 8192, 28672)])
@pytest.mark.parametrize("dgrad", [False, True])
def test_70b_shapes(name, n, k, dgrad):
    # Benchmark config 4: 8192 tokens, forward and input-gradient.
    _layer_check(8192, n, k, dq=True, seed=4, dgrad=dgrad)


def test_gemm_argument_errors():
    w = _weight(128, 96, 1)
    x = torch.zeros(4, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(Exception, match="k % 64"):
        gemm.linear_fwd(x, w)
    w = _weight(96, 128, 1)
    dy = torch.zeros(4, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(Exception, match="n % 64"):
        gemm.linear_dgrad(dy, w)


# Grouped launches: forward over weights that share x (q/k/v, gate/up) and
# the summed input gradient (d_h1 = dq.Wq + dk.Wk + dv.Wv, d_h2 = d_gate.Wg +
# d_up.Wu).

@pytest.mark.parametrize("m,k,ns,dqs", [
    (700, 256, [300, 64, 130], [True, True, True]),        # batched loads, ragged
    (513, 320, [257, 128], [False, False]),                # per-step loads
    (640, 512, [384, 128, 128, 200], [True, False, True, False]),  # mixed kinds
])
def test_fwd_grouped_equals_separate(m, k, ns, dqs):
    ws = [_weight(n, k, 51 + i * 7 + n, dq) for i, (n, dq) in enumerate(zip(ns, dqs))]
    x, _ = _act(m, k, 17 + m)
    ys = gemm.linear_fwd_grouped(x, ws, split_k=False)
    sep = [gemm.linear_fwd(x, w, split_k=False) for w in ws]
    torch.cuda.synchronize()
    for y, s in zip(ys, sep):
        assert torch.equal(y.view(torch.int16), s.view(torch.int16))


@pytest.mark.parametrize("m,k,ns", [(700, 192, [128, 64, 64]), (513, 256, [320, 128]),
                                    (64, 128, [64]), (1024, 512, [256, 64, 64, 128]),
                                    (640, 256, [256, 512])])
@pytest.mark.parametrize("dq", [False, True])
def test_dgrad_sum_small_vs_oracle(m, k, ns, dq):
    ws = [_weight(n, k, 61 + i * 5 + n, dq) for i, n in enumerate(ns)]
    acts = [_act(m, n, 23 + i + m) for i, n in enumerate(ns)]
    dx = gemm.linear_dgrad_sum([a for a, _ in acts], ws)
    torch.cuda.synchronize()
    dxh = dx.float().cpu().numpy()
    ref = sum(oracle.dgrad(ah, _deq_host(w, f16=True)) for (_, ah), w in zip(acts, ws))
    assert rel_l2(dxh, ref) <= TOL_REF
    same = sum(oracle.dgrad(ah, _deq_host(w, f16=False)).astype(np.float64)
               for (_, ah), w in zip(acts, ws))
    assert rel_l2(dxh, same) <= TOL_SAME


@pytest.mark.parametrize("name,ns,k", [("d_h1 = dq.Wq + dk.Wk + dv.Wv", [8192, 1024, 1024], 8192),
                                       ("d_h2 = d_gate.Wg + d_up.Wu", [28672, 28672], 8192)])
def test_dgrad_sum_70b_shapes(name, ns, k):
    # Benchmark config 4 input gradients as the reference accumulates them.
    m = 8192
    g = torch.Generator(device=DEV).manual_seed(8)
    ws = [nf4.quantize_weight(torch.randn(n, k, device=DEV, generator=g) * 0.02, double_quant=True)
          for n in ns]
    dys = [torch.randn(m, n, device=DEV, generator=g).to(torch.bfloat16) for n in ns]
    dx = gemm.linear_dgrad_sum(dys, ws)
    ref = torch.zeros(m, k, device=DEV)
    for dy, w in zip(dys, ws):
        ref += dy.float() @ nf4.dequant(w).float()
    torch.cuda.synchronize()
    err = ((dx.float() - ref).norm() / ref.norm()).item()
    assert err <= TOL_SAME, err
    del ws, dys, dx, ref


def test_grouped_argument_errors():
    w = _weight(128, 128, 2)
    wq = _weight(128, 128, 3, dq=True)
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        gemm.linear_fwd_grouped(x, [])
    with pytest.raises(ValueError):
        gemm.linear_fwd_grouped(x, [w] * 5)
    with pytest.raises(Exception, match="double-quantized"):
        gemm.linear_dgrad_sum([x, x], [w, wq])


# SwiGLU fused into the forward epilogue: hidden = silu(x.Wg^T) * (x.Wu^T)
# (forward.rs:251-254, silu_f at math.rs:91-93).

def _silu(v):
    v = np.asarray(v, np.float64)
    return v / (1.0 + np.exp(-v))


@pytest.mark.parametrize("m,ff,k", [(700, 300, 256), (513, 130, 320), (64, 64, 1024),
                                    (1, 192, 512), (1024, 256, 768)])
@pytest.mark.parametrize("dq", [False, True])
def test_swiglu_small_vs_oracle(m, ff, k, dq):
    wg = _weight(ff, k, 71 + ff + k, dq)
    wu = _weight(ff, k, 72 + ff + k, dq)
    x, xh = _act(m, k, 29 + m)
    h = gemm.linear_swiglu(x, wg, wu)
    torch.cuda.synchronize()
    hh = h.float().cpu().numpy()
    for f16, tol in ((True, TOL_REF), (False, TOL_SAME)):
        gate = oracle.matmul_tb(xh, _deq_host(wg, f16=f16)).astype(np.float64)
        up = oracle.matmul_tb(xh, _deq_host(wu, f16=f16)).astype(np.float64)
        assert rel_l2(hh, _silu(gate) * up) <= tol


def test_swiglu_70b_shape():
    # Benchmark config 4 gate/up at 8192 tokens, double-quant.
    m, ff, k = 8192, 28672, 8192
    g = torch.Generator(device=DEV).manual_seed(12)
    wg = nf4.quantize_weight(torch.randn(ff, k, device=DEV, generator=g) * 0.02, double_quant=True)
    wu = nf4.quantize_weight(torch.randn(ff, k, device=DEV, generator=g) * 0.02, double_quant=True)
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    h = gemm.linear_swiglu(x, wg, wu)
    gate = x.float() @ nf4.dequant(wg).float().t()
    up = x.float() @ nf4.dequant(wu).float().t()
    ref = torch.nn.functional.silu(gate) * up
    torch.cuda.synchronize()
    err = ((h.float() - ref).norm() / ref.norm()).item()
    assert err <= TOL_SAME, err
    del wg, wu, x, h, gate, up, ref


def test_swiglu_argument_errors():
    w = _weight(128, 128, 2)
    wq = _weight(128, 128, 3, dq=True)
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(Exception, match="double-quantized"):
        gemm.linear_swiglu(x, w, wq)
    with pytest.raises(ValueError):
        gemm.linear_swiglu(x, w, _weight(64, 128, 4))


# Split-K last round (nf4s_gemm_fwd_grouped_ws): tiles of a last round that
# would leave most CUs idle run as K slices; the fixup kernel sums their fp32
# partials in slice order.  Only the fp32 summation order changes, so both the
# split and the unsplit result stay within TOL_SAME of fp32 on the same
# operands.  Shapes (on a 256-CU MI355X): T = 100 tiles -> 2 slices; 16 tiles
# of ragged M and N -> 8 slices of 4 steps; the per-step producer with an odd
# step count; a 7B gate/up pair (1376 tiles, the last 96 split in 2); 70B k
# alone (128 tiles); a group mixing double-quant and fp32-absmax weights, which
# runs one launch per kind over one workspace.
SPLIT = [(512, [12800], 1024, True), (513, [1000], 2048, True), (512, [3840], 1344, False),
         (512, [3840], 1344, True), (4096, [11008, 11008], 4096, True),
         (8192, [1024], 8192, True), (700, [3000, 1200], 512, False),
         (512, [6400, 1000, 6400], 1024, (True, False, False))]


@pytest.mark.parametrize("m,ns,k,dq", SPLIT)
def test_fwd_split_k_tail(m, ns, k, dq):
    print(f"split-K m={m} ns={ns} k={k} dq={dq}", flush=True)
    need = gemm.fwd_workspace_bytes(ns, m, k)
    dqs = dq if isinstance(dq, tuple) else (dq,) * len(ns)
    ws = [_weight(n, k, 61 + n + i, d) for i, (n, d) in enumerate(zip(ns, dqs))]
    x, xf = _act(m, k, 19 + m)
    ys = gemm.linear_fwd_grouped(x, ws, split_k=True)
    ref = gemm.linear_fwd_grouped(x, ws, split_k=False)
    torch.cuda.synchronize()
    for w, y, r in zip(ws, ys, ref):
        wdq = nf4.dequant(w).float()
        exact = x.float() @ wdq.t()
        torch.cuda.synchronize()
        e_split = float((y.float() - exact).norm() / exact.norm())
        e_ref = float((r.float() - exact).norm() / exact.norm())
        assert e_split <= TOL_SAME and e_ref <= TOL_SAME, (e_split, e_ref)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert need > 0  # these shapes do split on a 256-CU part


def test_fwd_split_k_small_workspace_falls_back():
    """A workspace smaller than one tile's partial sums, handed straight to the
    C entry point (the Python wrapper would replace it): no split, the unsplit
    result bit for bit."""
    m, n, k = 512, 12800, 1024
    w = _weight(n, k, 71, True)
    x, _ = _act(m, k, 23)
    small = torch.empty(4096, dtype=torch.uint8, device=DEV)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    ns = (ctypes.c_int64 * 1)(n)
    ys = (ctypes.c_void_p * 1)(y.data_ptr())
    descs = (_lib.Nf4sTensor * 1)(w.descriptor())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.load().nf4s_gemm_fwd_grouped_ws(x.data_ptr(), descs, ns, ys, 1, m, k,
                                                    small.data_ptr(), 4096, stream))
    r = gemm.linear_fwd(x, w, split_k=False)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), r.view(torch.int16))


def test_fwd_split_k_twice_in_a_row():
    """Two split launches on one stream reuse one workspace: the second (a
    smaller shape) must not see the first's partials."""
    ws_buf = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    for m, n, k, seed in ((512, 12800, 1024, 81), (256, 6400, 512, 82)):
        w = _weight(n, k, seed, True)
        x, _ = _act(m, k, seed)
        y = gemm.linear_fwd_grouped(x, [w], split_k=True, workspace=ws_buf)[0]
        exact = x.float() @ nf4.dequant(w).float().t()
        torch.cuda.synchronize()
        assert float((y.float() - exact).norm() / exact.norm()) <= TOL_SAME



# Split-K input gradient: few tokens leave a last round of at most half the
# CUs, whose tiles then run as slices of the weights' concatenated reduction.
# Cases: the batched producer (4 slices of 4 steps); the per-step producer
# with a slice that straddles two summed weights (steps 10 + 5, slices of 4);
# the 70B d_h1 sum at 512 tokens (slices of 40 steps, the last one over the
# end of Wq and all of Wk and Wv); two row blocks at ragged m.
DGRAD_SPLIT = [(256, [1024], 1024, True), (300, [640, 320], 512, False),
               (512, [8192, 1024, 1024], 8192, True), (1000, [2048], 4096, True)]


@pytest.mark.parametrize("m,ns,k,dq", DGRAD_SPLIT)
def test_dgrad_split_k_tail(m, ns, k, dq):
    print(f"dgrad split-K m={m} ns={ns} k={k} dq={dq}", flush=True)
    ws = [_weight(n, k, 91 + n + i, dq) for i, n in enumerate(ns)]
    dys = [_act(m, n, 29 + n + i)[0] for i, n in enumerate(ns)]
    need = gemm.dgrad_workspace_bytes(ns, m, k)
    got = gemm.linear_dgrad_sum(dys, ws, split_k=True)
    ref = gemm.linear_dgrad_sum(dys, ws, split_k=False)
    exact = sum(d.float() @ nf4.dequant(w).float() for d, w in zip(dys, ws))
    torch.cuda.synchronize()
    e_split = float((got.float() - exact).norm() / exact.norm())
    e_ref = float((ref.float() - exact).norm() / exact.norm())
    assert e_split <= TOL_SAME and e_ref <= TOL_SAME, (e_split, e_ref)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert need > 0  # these shapes do split on a 256-CU part
    if len(ns) == 1:
        one = gemm.linear_dgrad(dys[0], ws[0])
        torch.cuda.synchronize()
        assert torch.equal(one.view(torch.int16), got.view(torch.int16))


def test_dgrad_split_k_small_workspace_falls_back():
    """A workspace too small for the split, handed straight to the C entry
    point: no split, the unsplit result bit for bit."""
    m, n, k = 256, 1024, 1024
    w = _weight(n, k, 73, True)
    dy, _ = _act(m, n, 31)
    small = torch.empty(4096, dtype=torch.uint8, device=DEV)
    dx = torch.empty(m, k, dtype=torch.bfloat16, device=DEV)
    ns = (ctypes.c_int64 * 1)(n)
    dps = (ctypes.c_void_p * 1)(dy.data_ptr())
    descs = (_lib.Nf4sTensor * 1)(w.descriptor())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.load().nf4s_gemm_dgrad_sum_ws(dps, descs, ns, 1, m, k, dx.data_ptr(),
                                                  small.data_ptr(), 4096, stream))
    r = gemm.linear_dgrad(dy, w, split_k=False)
    torch.cuda.synchronize()
    assert torch.equal(dx.view(torch.int16), r.view(torch.int16))


def test_dgrad_split_k_twice_in_a_row():
    """Two split launches on one stream reuse one workspace: the second (a
    smaller shape) must not see the first's partials."""
    ws_buf = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    for m, n, k, seed in ((512, 2048, 2048, 83), (256, 1024, 512, 84)):
        w = _weight(n, k, seed, True)
        dy, _ = _act(m, n, seed)
        dx = gemm.linear_dgrad(dy, w, split_k=True, workspace=ws_buf)
        exact = dy.float() @ nf4.dequant(w).float()
        torch.cuda.synchronize()
        assert float((dx.float() - exact).norm() / exact.norm()) <= TOL_SAME

# Seeded random shapes: ragged m, any n for the forward (n % 64 == 0 for the
# input gradient), k a multiple of 64 (per-step and batched producers), both
# absmax formats, the forward with its default split-K.  Each against torch
# fp32 over the same bf16 operands and the dequantized weight.
RANDOM_CASES = 16


@pytest.mark.parametrize("case", range(RANDOM_CASES))
def test_random_shapes_fwd_and_dgrad(case):
    rng = np.random.default_rng(9100 + case)
    m = int(rng.integers(1, 2049))
    k = 64 * int(rng.integers(1, 65))
    n_fwd = int(rng.integers(1, 3073))
    n_dg = 64 * int(rng.integers(1, 49))
    dq = bool(rng.integers(0, 2))
    print(f"random case {case}: m={m} k={k} n_fwd={n_fwd} n_dgrad={n_dg} dq={dq}", flush=True)
    x, _ = _act(m, k, 300 + case)
    w = _weight(n_fwd, k, 400 + case, dq)
    y = gemm.linear_fwd(x, w)
    ref = x.float() @ nf4.dequant(w).float().t()
    torch.cuda.synchronize()
    assert rel_l2(y.float().cpu().numpy(), ref.cpu().numpy()) <= TOL_SAME
    wd = _weight(n_dg, k, 500 + case, dq)
    dy, _ = _act(m, n_dg, 600 + case)
    dx = gemm.linear_dgrad(dy, wd)
    ref = dy.float() @ nf4.dequant(wd).float()
    torch.cuda.synchronize()
    assert rel_l2(dx.float().cpu().numpy(), ref.cpu().numpy()) <= TOL_SAME


# Both epilogues: outputs that take 16-byte stores go through the LDS
# read-back (store_tile_lds), the others through direct 8-byte or element
# stores (store_tile).  The same accumulators must give the same bits either
# way: outputs whose base is 2 bytes off 16-byte alignment take the direct
# path.  Ragged rows and a ragged last output tile on both kernels.
@pytest.mark.parametrize("m,n,k,dq", [(300, 256, 256, True), (777, 640, 384, False),
                                      (1024, 136, 512, True)])
def test_unaligned_output_equals_aligned(m, n, k, dq):
    print(f"epilogue paths m={m} n={n} k={k} dq={dq}", flush=True)
    x, _ = _act(m, k, 700 + m)
    w = _weight(n, k, 710 + n, dq)
    y = gemm.linear_fwd(x, w, split_k=False)
    flat = torch.empty(m * n + 8, dtype=torch.bfloat16, device=DEV)
    y_off = flat[1:1 + m * n].view(m, n)
    gemm.linear_fwd(x, w, out=y_off, split_k=False)
    dy, _ = _act(m, n - n % 64 if n % 64 else n, 720 + m)
    wd = _weight(dy.shape[1], k, 730 + n, dq)
    dx = gemm.linear_dgrad(dy, wd)
    flat2 = torch.empty(m * k + 8, dtype=torch.bfloat16, device=DEV)
    dx_off = flat2[1:1 + m * k].view(m, k)
    gemm.linear_dgrad(dy, wd, out=dx_off)
    torch.cuda.synchronize()
    assert y_off.data_ptr() % 16 == 2 and dx_off.data_ptr() % 16 == 2
    assert torch.equal(y.view(torch.int16), y_off.view(torch.int16))
    assert torch.equal(dx.view(torch.int16), dx_off.view(torch.int16))
    ref = x.float() @ nf4.dequant(w).float().t()
    assert rel_l2(y.float().cpu().numpy(), ref.cpu().numpy()) <= TOL_SAME


# 64 output tiles per 512-row block switch the tile order to XCD pairs
# sharing a row block (tiles_m % 4 == 0): ragged rows and a ragged last
# output tile under that order, forward (n) and input gradient (k).
@pytest.mark.parametrize("m,wide", [(1800, 8128), (4096, 8192), (2048, 8136)])
def test_xcd_pair_tile_order(m, wide):
    print(f"xcd-pair order m={m} wide={wide}", flush=True)
    k = 256
    x, _ = _act(m, k, 700 + m)
    w = _weight(wide, k, 701, True)
    y = gemm.linear_fwd(x, w)
    ref = x.float() @ nf4.dequant(w).float().t()
    torch.cuda.synchronize()
    assert rel_l2(y.float().cpu().numpy(), ref.cpu().numpy()) <= TOL_SAME
    n = 128
    wd = _weight(n, wide - wide % 64, 702, True)
    dy, _ = _act(m, n, 703)
    dx = gemm.linear_dgrad(dy, wd)
    ref = dy.float() @ nf4.dequant(wd).float()
    torch.cuda.synchronize()
    assert rel_l2(dx.float().cpu().numpy(), ref.cpu().numpy()) <= TOL_SAME



@pytest.mark.parametrize("name,ns,k", [("[q,k,v]", [8192, 1024, 1024], 8192),
                                       ("[gate,up]", [28672, 28672], 8192)])
def test_fwd_grouped_70b_launches(name, ns, k):
    """The grouped launches config 4 times, at their size (M = 8192): the
    [q,k,v] launch (1280 tiles, 5 whole rounds) and the [gate,up] launch
    (XCD-pair tile order across two groups).  Bit-equal to separate unsplit
    launches of each weight, and within the bf16 output rounding of fp32."""
    m = 8192
    g = torch.Generator(device=DEV).manual_seed(81)
    ws = [nf4.quantize_weight(torch.randn(n, k, device=DEV, generator=g) * 0.02, double_quant=True)
          for n in ns]
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    ys = gemm.linear_fwd_grouped(x, ws)
    for y, w in zip(ys, ws):
        sep = gemm.linear_fwd(x, w, split_k=False)
        assert torch.equal(y.view(torch.int16), sep.view(torch.int16)), name
        ref = x.float() @ nf4.dequant(w).float().t()
        err = ((y.float() - ref).norm() / ref.norm()).item()
        assert err <= TOL_SAME, (name, err)
        del sep, ref
    torch.cuda.synchronize()


def test_zero_tokens_and_empty_tensors():
    """Zero tokens through every GEMM entry point, and empty tensors through
    quantize and dequant: empty outputs, no launch errors, and the stream
    stays usable (a normal call after them is still exact)."""
    w = _weight(256, 128, 3, dq=True)
    w2 = _weight(128, 128, 4, dq=True)
    x0 = torch.zeros(0, 128, dtype=torch.bfloat16, device=DEV)
    assert gemm.linear_fwd(x0, w).shape == (0, 256)
    assert gemm.linear_fwd(x0, w, split_k=False).shape == (0, 256)
    ys = gemm.linear_fwd_grouped(x0, [w, w2])
    assert [tuple(y.shape) for y in ys] == [(0, 256), (0, 128)]
    dy0 = torch.zeros(0, 256, dtype=torch.bfloat16, device=DEV)
    assert gemm.linear_dgrad(dy0, w).shape == (0, 128)
    dx = gemm.linear_dgrad_sum([dy0, torch.zeros(0, 128, dtype=torch.bfloat16, device=DEV)],
                               [w, w2])
    assert dx.shape == (0, 128)
    assert gemm.linear_swiglu(x0, w, _weight(256, 128, 5, dq=True)).shape == (0, 256)
    r = nf4.quantize_nf4(torch.zeros(0, dtype=torch.float32, device=DEV))
    assert r.packed.numel() == 0 and r.absmax.numel() == 0
    assert nf4.dequant(nf4.Nf4Weight(packed=r.packed, absmax=r.absmax, shape=[0])).numel() == 0
    x, xh = _act(64, 128, 6)
    y = gemm.linear_fwd(x, w)
    torch.cuda.synchronize()
    ref = xh.astype(np.float64) @ _deq_host(w, f16=False).astype(np.float64).T
    assert rel_l2(y.float().cpu().numpy(), ref) <= TOL_SAME
