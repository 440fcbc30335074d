"""GPU parity of the weight gradient dW = dy^T . x (bf16 in, fp32 out).

Against the oracle's restatement of the d_wd loop (doublepass/src/
backward.rs:87-93) on the same bf16 values widened to fp32: only the fp32
summation order differs, so rel-L2 <= 1e-5 (TOL_SAME); bit-exact on
small-integer data, whose every partial sum is an exactly representable
fp32 integer.  Layer shapes: against a torch fp32 GPU matmul of the same
operands, plus rows in fp64 on the CPU.  The accumulate flag is the
micro-batch sum of backward.rs:478-502."""
import numpy as np
import pytest
import torch

import oracle
from aethelstream_amd import _lib, gemm

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_SAME = 1e-5


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _bf16(m, k, seed, sigma=1.0):
    t = torch.from_numpy(oracle.gen_normal(seed, m * k, sigma)).to(DEV).view(m, k).to(torch.bfloat16)
    return t, t.float().cpu().numpy()


# (m, n, k): tile multiples, ragged tokens (m % 64 != 0), ragged n / k (not
# multiples of 256), a single token, and more tiles than CUs.
SMALL = [(64, 256, 256), (128, 512, 256), (1, 256, 256), (100, 264, 136), (777, 520, 1000),
         (4096, 512, 768), (64, 4096, 4352)]


@pytest.mark.parametrize("m,n,k", SMALL)
def test_wgrad_small_vs_oracle(m, n, k):
    print(f"wgrad m={m} n={n} k={k}", flush=True)
    dy, dyf = _bf16(m, n, 11 + m)
    x, xf = _bf16(m, k, 23 + k)
    dw = gemm.linear_wgrad(dy, x)
    torch.cuda.synchronize()
    ref = oracle.wgrad(dyf, xf)
    assert dw.shape == (n, k) and dw.dtype == torch.float32
    assert rel_l2(dw.cpu().numpy(), ref) <= TOL_SAME


def test_wgrad_exact_on_integers():
    """Small integers: every product and partial sum is an exact fp32 integer,
    so the result is bit-identical to the oracle whatever the summation order;
    this pins the output layout and the token/column mapping of both
    operands."""
    m, n, k = 300, 264, 520
    g = torch.Generator().manual_seed(3)
    dyi = torch.randint(-4, 5, (m, n), generator=g).float()
    xi = torch.randint(-4, 5, (m, k), generator=g).float()
    dw = gemm.linear_wgrad(dyi.to(DEV).to(torch.bfloat16), xi.to(DEV).to(torch.bfloat16))
    torch.cuda.synchronize()
    ref = oracle.wgrad(dyi.numpy(), xi.numpy())
    assert np.array_equal(dw.cpu().numpy(), ref)


# Launches whose rounds are all full take the XCD-block tile order (each
# XCD's workgroups cover 4 x 8 tiles per round): 256 and 512 tiles, with
# ragged tokens, a ragged last tile row and accumulate.  Small integers make
# every element exact, so this pins the order's tile coordinates bit for bit.
@pytest.mark.parametrize("m,n,k,acc", [(64, 4096, 4096, False), (100, 8128, 2048, True),
                                       (192, 2048, 16384, False)])
def test_wgrad_xcd_block_order_exact(m, n, k, acc):
    print(f"wgrad xcd blocks m={m} n={n} k={k} acc={acc}", flush=True)
    g = torch.Generator().manual_seed(m + n)
    dyi = torch.randint(-3, 4, (m, n), generator=g).float()
    xi = torch.randint(-3, 4, (m, k), generator=g).float()
    ref = dyi.double().t() @ xi.double()
    dw = torch.full((n, k), 2.0 if acc else float("nan"), device=DEV)
    gemm.linear_wgrad(dyi.to(DEV).to(torch.bfloat16), xi.to(DEV).to(torch.bfloat16), out=dw,
                      accumulate=acc)
    torch.cuda.synchronize()
    want = (ref + 2.0 if acc else ref).float()
    assert torch.equal(dw.cpu(), want)


def test_wgrad_accumulate_two_micro_batches():
    """dW = sum over micro-batches (backward.rs:478-502): the second call
    accumulates into the first call's fp32 result; a smaller second batch."""
    n, k = 264, 392
    dy1, dyf1 = _bf16(200, n, 5)
    x1, xf1 = _bf16(200, k, 6)
    dy2, dyf2 = _bf16(70, n, 7)
    x2, xf2 = _bf16(70, k, 8)
    dw = gemm.linear_wgrad(dy1, x1)
    gemm.linear_wgrad(dy2, x2, out=dw, accumulate=True)
    torch.cuda.synchronize()
    ref = oracle.wgrad(dyf2, xf2, oracle.wgrad(dyf1, xf1))
    assert rel_l2(dw.cpu().numpy(), ref) <= TOL_SAME


def test_wgrad_zero_tokens():
    dy = torch.empty(0, 256, dtype=torch.bfloat16, device=DEV)
    x = torch.empty(0, 128, dtype=torch.bfloat16, device=DEV)
    dw = torch.full((256, 128), 7.0, device=DEV)
    gemm.linear_wgrad(dy, x, out=dw, accumulate=True)
    torch.cuda.synchronize()
    assert bool((dw == 7.0).all())
    gemm.linear_wgrad(dy, x, out=dw)
    torch.cuda.synchronize()
    assert bool((dw == 0.0).all())


def test_wgrad_output_bounds_untouched():
    """Ragged n and k: the kernel writes exactly [n, k] of a larger buffer's
    leading part and nothing past it."""
    m, n, k = 130, 264, 136
    dy, dyf = _bf16(m, n, 31)
    x, xf = _bf16(m, k, 32)
    buf = torch.full((n * k + 4096,), -3.0, device=DEV)
    out = buf[: n * k].view(n, k)
    gemm.linear_wgrad(dy, x, out=out)
    torch.cuda.synchronize()
    assert rel_l2(out.cpu().numpy(), oracle.wgrad(dyf, xf)) <= TOL_SAME
    assert bool((buf[n * k:] == -3.0).all())


@pytest.mark.parametrize("name,m,n,k", [
    ("7b_wd", 4096, 4096, 11008),       # d_wd: dy [M, d], hidden [M, ff]
    ("70b_wg", 8192, 28672, 8192),      # d_wg: d_gate [M, ff], h2 [M, d]
    ("70b_wk", 8192, 1024, 8192),       # d_wk with GQA k/v width
])
def test_wgrad_layer_shapes(name, m, n, k):
    print(f"wgrad {name} m={m} n={n} k={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(9)
    dy = torch.randn(m, n, device=DEV, generator=g).to(torch.bfloat16)
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    dw = gemm.linear_wgrad(dy, x)
    ref = dy.float().t().contiguous() @ x.float()
    torch.cuda.synchronize()
    err = float((dw - ref).norm() / ref.norm())
    assert err <= TOL_SAME, err
    # Two rows in fp64 on the CPU.
    dyc = dy.float().cpu().numpy().astype(np.float64)
    xc = x.float().cpu().numpy().astype(np.float64)
    for r in (0, n - 1):
        row = dyc[:, r] @ xc
        assert rel_l2(dw[r].cpu().numpy(), row) <= TOL_SAME


def test_wgrad_rejects_bad_width():
    dy = torch.zeros(64, 12, dtype=torch.bfloat16, device=DEV)
    x = torch.zeros(64, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.Nf4sError) as e:
        gemm.linear_wgrad(dy, x)
    assert e.value.status == _lib.NF4S_ERR_UNSUPPORTED_SHAPE


# Grouped launches (products sharing x, backward.rs:284-300 and :117-129):
# every product's tiles run the same code as a launch of their own, so each
# dW must equal the single-product result bit for bit, whatever tile order
# the stacked grid takes (ragged widths, 2-4 products, 64-tile rounds that
# take the XCD-block order, accumulate).
@pytest.mark.parametrize("m,ns,k,acc", [
    (100, [264, 8, 1000], 136, False),             # ragged widths and tokens
    (64, [8192, 4096, 4096], 2048, False),         # 64 x 8 tiles = 2 full rounds
    (130, [512, 256, 256, 1024], 512, True),       # four products, accumulate
    (1, [256, 256], 256, False),                   # one token
])
def test_wgrad_grouped_equals_single(m, ns, k, acc):
    print(f"wgrad grouped m={m} ns={ns} k={k} acc={acc}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(m + k)
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    dys = [torch.randn(m, n, device=DEV, generator=g).to(torch.bfloat16) for n in ns]
    init = [torch.randn(n, k, device=DEV, generator=g) for n in ns]
    singles = []
    for dy, i0 in zip(dys, init):
        out = i0.clone()
        gemm.linear_wgrad(dy, x, out=out, accumulate=acc)
        singles.append(out)
    outs = [i0.clone() for i0 in init]
    gemm.linear_wgrad_grouped(dys, x, outs=outs, accumulate=acc)
    torch.cuda.synchronize()
    for a, b in zip(outs, singles):
        assert torch.equal(a, b)


def test_wgrad_grouped_exact_on_integers():
    # Small integers: every dW element is exact, so this pins each product's
    # rows and columns (a product offset or a swapped dy shows up).
    m, ns, k = 96, [2048, 256, 256], 1024
    g = torch.Generator().manual_seed(5)
    xi = torch.randint(-3, 4, (m, k), generator=g).float()
    dyi = [torch.randint(-3, 4, (m, n), generator=g).float() for n in ns]
    outs = gemm.linear_wgrad_grouped([d.to(DEV).to(torch.bfloat16) for d in dyi],
                                     xi.to(DEV).to(torch.bfloat16))
    torch.cuda.synchronize()
    for d, o in zip(dyi, outs):
        assert torch.equal(o.cpu(), (d.double().t() @ xi.double()).float())


def test_wgrad_grouped_70b_qkv():
    # Config 4's d_wq, d_wk, d_wv from one attention input: 40 x 32 tiles.
    m, k = 8192, 8192
    print(f"wgrad grouped 70b qkv m={m} k={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(21)
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    dys = [torch.randn(m, n, device=DEV, generator=g).to(torch.bfloat16)
           for n in (8192, 1024, 1024)]
    outs = gemm.linear_wgrad_grouped(dys, x)
    for dy, o in zip(dys, outs):
        assert torch.equal(o, gemm.linear_wgrad(dy, x))
    ref = dys[1].float().t().contiguous() @ x.float()
    torch.cuda.synchronize()
    assert float((outs[1] - ref).norm() / ref.norm()) <= TOL_SAME
