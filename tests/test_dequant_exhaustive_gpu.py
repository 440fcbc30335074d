"""NF4 dequant (shard_engine/src/nf4.rs:37-83: one fp32 product code * absmax,
then the f16 / bf16 conversion, round to nearest even) on the device for
EVERY finite fp32 absmax >= 0 (0 .. FLT_MAX, 2^31 values) and all 16 codes,
in both output formats, plus +inf and NaN absmax.

Reference: torch on the same GPU, `(codes[c] * absmax).to(dtype)` (one IEEE
fp32 multiply, then RNE), whose conversions the first test checks against a
numpy restatement of RNE on the CPU.  Each 32-element block holds codes 0..15
twice with one absmax (block_size 32: the fast kernel's path)."""
import numpy as np
import pytest
import torch

import oracle
from aethelstream_amd import nf4

pytestmark = pytest.mark.gpu
DEV = "cuda"
CHUNK = 1 << 25  # absmax values per launch (2^30 outputs)


def _bf16_rne(x: np.ndarray) -> np.ndarray:
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)  # quiet NaN, sign kept
    return r


def test_torch_gpu_conversions_are_rne():
    rng = np.random.default_rng(9)
    x = rng.integers(0, 1 << 32, 1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[np.isfinite(x)]
    t = torch.from_numpy(x).to(DEV)
    got_bf = t.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got_bf, _bf16_rne(x))
    got_h = t.to(torch.float16).view(torch.int16).cpu().numpy().view(np.uint16)
    with np.errstate(over="ignore"):                    # overflow to inf is the point
        want_h = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got_h, want_h)


def test_torch_gpu_multiply_is_ieee():
    """The reference's fp32 product on the GPU, denormal inputs and results
    included (no flush to zero), against numpy's IEEE multiply."""
    rng = np.random.default_rng(10)
    am = rng.integers(0, 0x7F800000, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    am[:4096] = rng.integers(0, 1 << 24, 4096, dtype=np.uint64).astype(np.uint32).view(np.float32)
    codes = oracle.codebook().astype(np.float32)
    want = (am[:, None] * codes[None, :]).view(np.uint32)
    got = (torch.from_numpy(am).to(DEV)[:, None] * torch.from_numpy(codes).to(DEV)[None, :])
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)
    denormal = ((want & 0x7F800000) == 0) & ((want & 0x7FFFFFFF) != 0)
    assert np.count_nonzero(denormal) > 4096                   # denormal results exercised


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dequant_every_absmax_every_code(dtype):
    print(f"exhaustive dequant {dtype}", flush=True)
    codes = torch.from_numpy(oracle.codebook().astype(np.float32)).to(DEV)
    one_block = torch.tensor([(2 * i << 4) | (2 * i + 1) for i in range(8)] * 2,
                             dtype=torch.uint8, device=DEV)            # codes 0..15 twice
    top = 0x7F7FFFFF                                                   # FLT_MAX
    specials = torch.tensor([0x7F800000, 0x7FC00000], dtype=torch.int64, device=DEV)
    bad = 0
    for lo in range(0, top + 1, CHUNK):
        nb = min(CHUNK, top + 1 - lo)
        bits = torch.arange(lo, lo + nb, dtype=torch.int64, device=DEV)
        if lo + nb > top:
            bits = torch.cat([bits, specials])                         # +inf, NaN
        am = bits.to(torch.int32).view(torch.float32)
        nblk = am.numel()
        w = nf4.Nf4Weight(packed=one_block.repeat(nblk), absmax=am, shape=[nblk * 32],
                          block_size=32)
        got = nf4.dequant(w, dtype=dtype).view(nblk, 32)
        want = (am[:, None] * codes[None, :]).to(dtype)
        gi = got.view(torch.int16)
        wi = want.view(torch.int16)
        # NaN outputs compare as NaN (payloads are not part of the format).
        gn = torch.isnan(got)
        same = (gi[:, :16] == wi) | (gn[:, :16] & torch.isnan(want))
        same2 = (gi[:, 16:] == wi) | (gn[:, 16:] & torch.isnan(want))
        bad += int((~same).sum()) + int((~same2).sum())
        del bits, am, w, got, want, gi, wi, gn, same, same2
    torch.cuda.synchronize()
    assert bad == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dequant_double_quant_every_code_many_scales(dtype):
    """Double-quant absmax: block absmax = (float)q * scale, one fp32 multiply
    (the decode the device kernels apply before the product table), for every
    8-bit code q times 65536 random finite fp32 scales (a 256-block group per
    scale, huge scales overflowing to inf included), then all 16 NF4 codes."""
    print(f"double-quant dequant {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(12)
    nscale = 1 << 16
    sbits = torch.randint(0, 0x7F800000, (nscale,), generator=g, device=DEV, dtype=torch.int64)
    scale = sbits.to(torch.int32).view(torch.float32)
    q = torch.arange(256, dtype=torch.uint8, device=DEV).repeat(nscale)
    nblk = q.numel()
    one_block = torch.tensor([(2 * i << 4) | (2 * i + 1) for i in range(8)] * 4,
                             dtype=torch.uint8, device=DEV)            # codes 0..15, 4 times
    w = nf4.Nf4Weight(packed=one_block.repeat(nblk), absmax=None, shape=[nblk * 64],
                      block_size=64, absmax_q=q, absmax_scale=scale, dq_group=256)
    got = nf4.dequant(w, dtype=dtype).view(nblk, 4, 16)
    codes = torch.from_numpy(oracle.codebook().astype(np.float32)).to(DEV)
    am = q.float() * scale.repeat_interleave(256)
    want = (am[:, None] * codes[None, :]).to(dtype)[:, None, :].expand(nblk, 4, 16)
    same = (got.view(torch.int16) == want.view(torch.int16)) | (torch.isnan(got) & torch.isnan(want))
    torch.cuda.synchronize()
    assert int((~same).sum()) == 0
    assert bool(torch.isinf(am).any()) and bool((am == 0).any())  # overflow and q = 0 exercised
