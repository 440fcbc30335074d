"""Fused GEMMs on weights whose absmax blocks are wider than 64 elements.

The shard index names a block size per tensor (shard_engine/src/index.rs:33;
dequant_nf4_into takes it as an argument, nf4.rs:37-42), while the writer
uses 64 (quantizer.py:12).  The fused kernels take every block size 64 << s
(one 64-deep reduction step never straddles two blocks) with whole blocks
per row.  Checked here for 128 and 256, fp32 and double-quantized absmax:
one-hot activations return the dequantized weights exactly (forward and
input gradient, split-K and summed forms included), and random activations
agree with the fp32 product over the oracle's dequant of the same block
size (matmul_tb, doublepass/src/math.rs:9-21) to the bf16 output rounding.
Other block sizes are rejected."""
import numpy as np
import pytest
import torch

import oracle
from aethelstream_amd import _lib, gemm, nf4

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_SAME = 4e-3


def _weight(n, k, seed, bs, dq):
    w32 = oracle.gen_normal(seed, n * k, 0.02)
    return nf4.quantize_weight(torch.from_numpy(w32).to(DEV).view(n, k), block_size=bs,
                               double_quant=dq)


def _oracle_dequant(w) -> np.ndarray:
    pk = w.packed.cpu().numpy()
    if w.double_quant:
        am = oracle.dq_decode(w.absmax_q.cpu().numpy(), w.absmax_scale.cpu().numpy(), w.dq_group)
    else:
        am = w.absmax.cpu().numpy()
    return oracle.bf16_bits_to_f32(
        oracle.dequant_bf16(pk, am, w.numel, w.block_size)).reshape(w.shape)


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("bs", [128, 256])
@pytest.mark.parametrize("dq", [False, True])
def test_fwd_and_dgrad_one_hot_exact(bs, dq):
    n, k, m = 384, 1024, 1024
    w = _weight(n, k, 11 + bs, bs, dq)
    wd = nf4.dequant(w)
    assert np.array_equal(wd.float().cpu().numpy(), _oracle_dequant(w))
    idx = torch.arange(m, device=DEV) % k
    x = torch.zeros(m, k, device=DEV, dtype=torch.bfloat16)
    x[torch.arange(m, device=DEV), idx] = 1.0
    for split in (False, True):
        y = gemm.linear_fwd(x, w, split_k=split)
        assert torch.equal(y.float(), wd.t()[idx].float()), f"fwd split={split}"
    jdx = torch.arange(m, device=DEV) % n
    dy = torch.zeros(m, n, device=DEV, dtype=torch.bfloat16)
    dy[torch.arange(m, device=DEV), jdx] = 1.0
    for split in (False, True):
        dx = gemm.linear_dgrad(dy, w, split_k=split)
        assert torch.equal(dx.float(), wd[jdx].float()), f"dgrad split={split}"


@pytest.mark.parametrize("bs", [128, 256])
def test_random_operands_vs_oracle_dequant(bs):
    m, k = 700, 768
    ws = [_weight(300, k, 31, bs, True), _weight(128, k, 32, bs, False)]
    a = oracle.gen_normal(33, m * k, 1.0)
    x = torch.from_numpy(a).to(DEV).view(m, k).to(torch.bfloat16)
    xs = x.float().cpu().numpy()
    ys = gemm.linear_fwd_grouped(x, ws)
    for w, y in zip(ws, ys):
        ref = oracle.matmul_tb(xs, _oracle_dequant(w))
        assert _rel(y.float().cpu().numpy(), ref) <= TOL_SAME
    # Summed input gradient over a block-128/256 weight and a block-64 one.
    n0, n1 = 256, 320
    w0 = _weight(n0, k, 34, bs, True)
    w1 = _weight(n1, k, 35, 64, True)
    d0 = torch.from_numpy(oracle.gen_normal(36, m * n0, 1.0)).to(DEV).view(m, n0).to(torch.bfloat16)
    d1 = torch.from_numpy(oracle.gen_normal(37, m * n1, 1.0)).to(DEV).view(m, n1).to(torch.bfloat16)
    dx = gemm.linear_dgrad_sum([d0, d1], [w0, w1])
    ref = (d0.float().cpu().numpy() @ _oracle_dequant(w0)
           + d1.float().cpu().numpy() @ _oracle_dequant(w1))
    assert _rel(dx.float().cpu().numpy(), ref) <= TOL_SAME


def test_swiglu_block_128_matches_unfused_epilogue():
    m, ff, k = 512, 256, 512
    wg, wu = _weight(ff, k, 41, 128, True), _weight(ff, k, 42, 128, True)
    x = torch.from_numpy(oracle.gen_normal(43, m * k, 1.0)).to(DEV).view(m, k).to(torch.bfloat16)
    h = gemm.linear_swiglu(x, wg, wu)
    g, u = gemm.linear_fwd_grouped(x, [wg, wu], split_k=False)
    ref = torch.nn.functional.silu(g.float()) * u.float()
    # The fused epilogue works on the fp32 accumulators, the reference here
    # on bf16-rounded gate and up: bf16-level agreement.
    assert _rel(h.float().cpu().numpy(), ref.cpu().numpy()) <= 1e-2


def test_other_block_sizes_rejected():
    x = torch.zeros(64, 192, device=DEV, dtype=torch.bfloat16)
    w32 = _weight(128, 192, 51, 32, False)       # blocks narrower than a step
    with pytest.raises(_lib.Nf4sError, match="block_size 64 << s"):
        gemm.linear_fwd(x, w32)
    w128 = _weight(128, 192, 52, 128, False)     # 192 = 1.5 blocks per row
    with pytest.raises(_lib.Nf4sError, match="whole blocks per row"):
        gemm.linear_fwd(x, w128)
    dy = torch.zeros(64, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(_lib.Nf4sError, match="whole blocks per row"):
        gemm.linear_dgrad(dy, w128)
