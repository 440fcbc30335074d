"""Block-64 quantize (quantizer.py:21-53) on the device over EVERY fp32 input
up to the block absmax, for absmax values chosen to cover each branch of the
kernel's code path: the fast quotient v * rcp(s) with its exact-quotient
fallback near the steps, the 1e-8 clamp (quantizer.py:36), and absmax >=
2^126 (the exact quotient for the whole lane).

Reference: code = #{k : RN(v / s) >= S_k} with s = clamp(absmax, 1e-8), the
step form of the first-index argmin of quantizer.py:40-41 that
tests/test_code_steps.py checks against the oracle exhaustively over every
fp32 in [-1, 1]; the quotient comes from torch's fp32 division on the GPU,
which the first test checks is correctly rounded (against numpy on the CPU).
Each block holds the absmax at element 0 (so the kernel's absmax is s) and
63 values under test."""
import numpy as np
import pytest
import torch

from aethelstream_amd import code_steps, nf4

pytestmark = pytest.mark.gpu
DEV = "cuda"

SCALES = [1.0, 0.7071067690849304, 0.021700000390410423, 1.5e-3, 3.0, 77700.0,
          1.0000000036274937e-15, 9.0e-9, 3.0e38]
CHUNK = 63 << 22  # test values per launch (about 264 M)


def _steps():
    return torch.tensor(np.array(code_steps.steps(), np.uint32).view(np.float32), device=DEV)


def test_torch_gpu_division_is_correctly_rounded():
    rng = np.random.default_rng(3)
    a = rng.standard_normal(1 << 22).astype(np.float32)
    b = (np.abs(rng.standard_normal(1 << 22)) + 1e-3).astype(np.float32)
    a[:1000] = np.float32(1e-40)       # subnormal numerators
    ref = (a / b).view(np.uint32)
    got = (torch.from_numpy(a).to(DEV) / torch.from_numpy(b).to(DEV)).cpu().numpy().view(np.uint32)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("s", SCALES)
def test_quantize_every_fp32_up_to_absmax(s):
    s32 = np.float32(s)
    top = int(np.array([s32], np.float32).view(np.uint32)[0])
    print(f"exhaustive quantize absmax={s32!r} ({2 * (top + 1)} values)", flush=True)
    steps = _steps()
    safe = torch.clamp(torch.tensor(float(s32), dtype=torch.float32, device=DEV), min=1e-8)
    bad = 0
    for sign in (0, 0x80000000):
        for lo in range(0, top + 1, CHUNK):
            n = min(CHUNK, top + 1 - lo)
            nb = -(-n // 63)
            bits = torch.arange(lo, lo + nb * 63, dtype=torch.int64, device=DEV)
            bits = torch.where(bits <= top, bits, torch.zeros_like(bits)) | sign
            bits = torch.where(bits >= 1 << 31, bits - (1 << 32), bits)  # as int32 bits
            v = bits.to(torch.int32).view(torch.float32).view(nb, 63)
            x = torch.cat([torch.full((nb, 1), float(s32), dtype=torch.float32, device=DEV), v],
                          dim=1).reshape(-1)
            r = nf4.quantize_nf4(x)
            assert torch.equal(r.absmax, torch.full((nb,), float(s32), dtype=torch.float32,
                                                    device=DEV))
            pk = r.packed
            codes = torch.stack([pk >> 4, pk & 15], dim=1).reshape(nb, 64)[:, 1:]
            want = torch.searchsorted(steps, v / safe, right=True)
            bad += int((codes.to(torch.int64) != want).sum())
            del bits, v, x, r, pk, codes, want
    torch.cuda.synchronize()
    assert bad == 0
