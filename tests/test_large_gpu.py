"""Tensors past 2^31 elements: int64 indexing through quantize, dequant and
the fused GEMMs, where an int32 offset would wrap.

- Quantize (quantizer.py:21-53) of 2^31 + 4197 fp32 values (an odd count:
  a partial last block and a code-0 pad nibble) against the step form of the
  quantizer's argmin on the same GPU (the reference of
  test_quantize_exhaustive_gpu.py), and the block absmax against torch's max.
- Dequant (nf4.rs:37-83) of that tensor against torch's fp32 product and RNE
  conversion of the kernel's own codes.
- The fused forward and input gradient over a double-quantized weight of
  262720 x 8192 (2^31 + 4.7 M elements) with one-hot activations, whose
  outputs are the weight's own bf16 values (test_gemm_exact_gpu.py),
  compared with the dequantized weight: every column of y = x.W^T, and dx
  rows taken from the start, the middle and past element 2^31 of W.

Every comparison runs over the whole tensor in chunks, so a wrapped write
anywhere shows up."""
import numpy as np
import pytest
import torch

import oracle
from aethelstream_amd import code_steps, gemm, nf4

pytestmark = pytest.mark.gpu
DEV = "cuda"
N_BIG = (1 << 31) + 4096 + 101
CH = 1 << 26  # elements per checked chunk (a multiple of 64)


def _steps():
    return torch.tensor(np.array(code_steps.steps(), np.uint32).view(np.float32), device=DEV)


def _codebook():
    return torch.from_numpy(oracle.codebook().astype(np.float32)).to(DEV)


def test_quantize_and_dequant_past_2g_elements():
    print(f"quantize + dequant of {N_BIG} elements", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.empty(N_BIG, dtype=torch.float32, device=DEV)
    x.normal_(0.0, 0.02, generator=g)
    r = nf4.quantize_nf4(x)
    nb = (N_BIG + 63) // 64
    assert r.absmax.numel() == nb and r.packed.numel() == (N_BIG + 1) // 2
    assert int(r.packed[-1]) & 15 == 0                    # pad nibble of the odd count
    w = nf4.Nf4Weight(packed=r.packed, absmax=r.absmax, shape=[N_BIG], block_size=64)
    wd = nf4.dequant(w)
    steps, cb = _steps(), _codebook()
    bad_am = bad_code = bad_deq = 0
    for lo in range(0, N_BIG, CH):
        hi = min(lo + CH, N_BIG)
        n = hi - lo
        xs = x[lo:hi]
        xb = torch.cat([xs, xs.new_zeros((-n) % 64)]).view(-1, 64)
        am = xb.abs().amax(1)
        b0 = lo // 64
        bad_am += int((r.absmax[b0:b0 + am.numel()] != am).sum())
        q = (xb / am.clamp(min=1e-8)[:, None]).reshape(-1)[:n]
        want = torch.searchsorted(steps, q, right=True)
        pk = r.packed[lo // 2:(hi + 1) // 2]
        codes = torch.stack([pk >> 4, pk & 15], dim=1).reshape(-1)[:n].to(torch.int64)
        bad_code += int((codes != want).sum())
        amx = r.absmax[b0:b0 + am.numel()].repeat_interleave(64)[:n]
        ref = (cb[codes] * amx).to(torch.bfloat16)
        bad_deq += int((wd[lo:hi].view(torch.int16) != ref.view(torch.int16)).sum())
        del xs, xb, am, q, want, pk, codes, amx, ref
    torch.cuda.synchronize()
    assert (bad_am, bad_code, bad_deq) == (0, 0, 0)
    del x, r, w, wd
    torch.cuda.empty_cache()


def _eye(m, cols, offset=0):
    e = torch.zeros(m, cols, dtype=torch.bfloat16, device=DEV)
    r = torch.arange(min(m, cols - offset), device=DEV)
    e[r, r + offset] = 1
    return e


def test_fused_gemms_on_a_weight_past_2g_elements():
    n, k = (1 << 18) + 576, 8192
    print(f"one-hot GEMMs over a {n} x {k} NF4 weight", flush=True)
    g = torch.Generator(device=DEV).manual_seed(6)
    w32 = torch.empty(n, k, dtype=torch.float32, device=DEV)
    w32.normal_(0.0, 0.02, generator=g)
    w = nf4.quantize_weight(w32, double_quant=True)
    del w32
    torch.cuda.empty_cache()
    wd = nf4.dequant(w)                                    # [n, k] bf16
    y = gemm.linear_fwd(_eye(k, k), w)                     # [k, n] = W^T
    bad = 0
    for c0 in range(0, n, 1 << 15):
        c1 = min(c0 + (1 << 15), n)
        bad += int((y[:, c0:c1] != wd[c0:c1].t()).sum())
    assert bad == 0
    del y
    for r0 in (0, n // 2, n - 256):                        # n - 256 rows start past 2^31 elements
        dx = gemm.linear_dgrad(_eye(256, n, offset=r0), w)
        assert int((dx != wd[r0:r0 + 256]).sum()) == 0, r0
    assert (n - 256) * k > 1 << 31
    del wd, w
    torch.cuda.empty_cache()
