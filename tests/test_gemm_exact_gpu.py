"""The fused GEMMs consume exactly the reference's dequantized weights.

With one-hot activations every output of y = x.W^T is a single product
1.0 * W[n, j] added onto exact zeros in fp32, so y = W^T bit for bit (a bf16
value survives fp32 accumulation and the bf16 output rounding unchanged).
Likewise dx = dy.W with one-hot dy gives rows of W.  Comparing those outputs
with the dequantized weights (shard_engine/src/nf4.rs:37-83: one fp32 product
code * absmax, then round to nearest even) checks the kernels' in-register
product-table lookups, double-quant absmax decode and tile layouts element by
element, at the 7B and 70B layer shapes the bench times, through every
producer and launch form: batched (k % 256 == 0) and per-step weight loads,
grouped and summed launches, and the split-K forms with fp32 partials.

The device dequant that serves as the expected value is itself compared with
the oracle's dequant here (whole weight for small shapes, sampled rows for
the layer shapes).  Values compare as numbers, so +0 and -0 are equal: a
zero weight (code 7, or an absmax of 0) gives +0 out of an fp32 sum."""
import numpy as np
import pytest
import torch

import oracle
from aethelstream_amd import gemm, nf4

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _weight(n, k, seed, dq):
    w32 = oracle.gen_normal(seed, n * k, 0.02)
    return nf4.quantize_weight(torch.from_numpy(w32).to(DEV).view(n, k), double_quant=dq)


def _oracle_rows(w, rows) -> np.ndarray:
    """Oracle bf16 dequant (as fp32) of the given rows of a device weight."""
    n, k = w.shape
    assert k % 2 == 0 and k % w.block_size == 0
    pk = w.packed.cpu().numpy()
    if w.double_quant:
        am = oracle.dq_decode(w.absmax_q.cpu().numpy(), w.absmax_scale.cpu().numpy(), w.dq_group)
    else:
        am = w.absmax.cpu().numpy()
    bpr = k // w.block_size
    out = np.empty((len(rows), k), np.float32)
    for i, r in enumerate(rows):
        bits = oracle.dequant_bf16(np.ascontiguousarray(pk[r * k // 2:(r + 1) * k // 2]),
                                   np.ascontiguousarray(am[r * bpr:(r + 1) * bpr]), k)
        out[i] = oracle.bf16_bits_to_f32(bits)
    return out


def _dequant_checked(w, all_rows=False):
    """Device bf16 dequant of w, checked against the oracle."""
    wd = nf4.dequant(w)
    n = w.shape[0]
    rows = list(range(n)) if all_rows else sorted({0, 1, 63, 64, n // 2, n - 65, n - 1})
    got = wd[rows].float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), _oracle_rows(w, rows).view(np.uint32))
    return wd


def _eye(m, cols, offset=0):
    """[m, cols] bf16 with a 1 at (i, offset + i) for i < min(m, cols - offset)."""
    e = torch.zeros(m, cols, dtype=torch.bfloat16, device=DEV)
    r = torch.arange(min(m, cols - offset), device=DEV)
    e[r, r + offset] = 1
    return e


def _same(a, b):
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = int((a != b).sum())
    assert bad == 0, f"{bad} of {a.numel()} outputs differ from the dequantized weight"


SMALL = [(128, 64, False), (384, 320, True), (192, 1024, False), (4096, 256, True)]


@pytest.mark.parametrize("n,k,dq", SMALL)
def test_small_fwd_and_dgrad_equal_weight(n, k, dq):
    w = _weight(n, k, 11, dq)
    wd = _dequant_checked(w, all_rows=True)
    _same(gemm.linear_fwd(_eye(k, k), w), wd.t())
    _same(gemm.linear_dgrad(_eye(n, n), w), wd)
    # a few one-hot rows instead of the full identity (ragged M, partial tiles)
    y = gemm.linear_fwd(_eye(37, k, offset=5), w)
    _same(y, wd.t()[5:42])


LAYER = {
    "7b_gate": (11008, 4096), "7b_down": (4096, 11008),
    "70b_q": (8192, 8192), "70b_k": (1024, 8192), "70b_gate": (28672, 8192),
    "70b_down": (8192, 28672),
}


@pytest.mark.parametrize("name", list(LAYER))
def test_layer_fwd_equals_weight(name):
    n, k = LAYER[name]
    w = _weight(n, k, 21, dq=True)
    wd = _dequant_checked(w)
    print(f"one-hot forward {name}", flush=True)
    x = _eye(k, k)
    _same(gemm.linear_fwd(x, w), wd.t())                   # split-K tail where it applies
    _same(gemm.linear_fwd(x, w, split_k=False), wd.t())


@pytest.mark.parametrize("name", ["7b_gate", "70b_q", "70b_gate", "70b_down"])
def test_layer_dgrad_equals_weight(name):
    n, k = LAYER[name]
    w = _weight(n, k, 22, dq=True)
    wd = _dequant_checked(w)
    print(f"one-hot input gradient {name}", flush=True)
    _same(gemm.linear_dgrad(_eye(n, n), w), wd)
    # 256 tokens: few output tiles, so the split reduction runs
    _same(gemm.linear_dgrad(_eye(256, n, offset=n - 256), w), wd[n - 256:])


def test_grouped_qkv_and_gate_up_fwd_equal_weights():
    ws = [_weight(n, 8192, 30 + i, dq=True) for i, n in enumerate((8192, 1024, 1024))]
    wds = [_dequant_checked(w) for w in ws]
    ys = gemm.linear_fwd_grouped(_eye(8192, 8192), ws)
    for y, wd in zip(ys, wds):
        _same(y, wd.t())
    gu = [_weight(11008, 4096, 40 + i, dq=True) for i in range(2)]
    gds = [_dequant_checked(w) for w in gu]
    ys = gemm.linear_fwd_grouped(_eye(4096, 4096), gu)         # 1376 tiles: split-K tail
    for y, wd in zip(ys, gds):
        _same(y, wd.t())


def test_summed_dgrad_equals_each_weight():
    ws = [_weight(n, 8192, 50 + i, dq=True) for i, n in enumerate((8192, 1024, 1024))]
    wds = [_dequant_checked(w) for w in ws]
    m = 1024
    for i, w in enumerate(ws):
        # dY_i one-hot on rows 0..m-1, the others zero: dx = rows 0..m-1 of W_i
        dys = [_eye(m, v.shape[0]) if j == i else
               torch.zeros(m, v.shape[0], dtype=torch.bfloat16, device=DEV)
               for j, v in enumerate(ws)]
        _same(gemm.linear_dgrad_sum(dys, ws), wds[i][:m])
        _same(gemm.linear_dgrad_sum(dys, ws, split_k=False), wds[i][:m])
