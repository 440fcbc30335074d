"""Writes tests/golden/nf4_golden.npz: seeded inputs with the outputs of an
op-by-op torch (CPU) restatement of the reference quantizer and dequantizer.

The reference module is not imported: the steps below restate
shard_engine/python/pipeline/quantizer.py:21-53 (quantize_nf4) and :55-75
(dequantize_nf4) with the same torch CPU kernels the reference calls (fp32
division, abs, argmin with first-index ties, uint8 packing, .to(float16)),
so the fixtures carry torch's own numerics for the edge cases below.  The C
oracle (oracle/nf4_oracle.c) is checked against these vectors in
tests/test_oracle.py.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "nf4_golden.npz")

CODES = torch.tensor([
    -1.0, -0.6961928, -0.52507305, -0.3949175,
    -0.28444138, -0.18477343, -0.09105004, 0.0,
    0.0795803, 0.1609302, 0.2461123, 0.33791524,
    0.44070983, 0.562617, 0.72295684, 1.0,
], dtype=torch.float32)  # quantizer.py:5-10


def torch_quantize(flat: torch.Tensor, bs: int = 64):
    n = flat.numel()
    pad = (bs - n % bs) % bs
    if pad:
        flat = torch.cat([flat, torch.zeros(pad, dtype=torch.float32)])
    blocks = flat.view(-1, bs)
    absmax = blocks.abs().max(dim=1).values
    safe = absmax.clamp(min=1e-8)
    norm = blocks / safe.unsqueeze(1)
    idx = (norm.unsqueeze(2) - CODES.view(1, 1, 16)).abs().argmin(dim=2).to(torch.uint8)
    idx = idx.flatten()[:n]
    if idx.numel() % 2:
        idx = torch.cat([idx, torch.zeros(1, dtype=torch.uint8)])
    packed = (idx[0::2] << 4) | idx[1::2]
    return packed, absmax


def torch_dequant(packed: torch.Tensor, absmax: torch.Tensor, n: int, bs: int, dtype):
    hi = (packed >> 4).to(torch.int64)
    lo = (packed & 0x0F).to(torch.int64)
    idx = torch.stack([hi, lo], dim=1).flatten()[:n]
    am = absmax.repeat_interleave(bs)[:n]
    return (CODES[idx] * am).to(dtype)


def cases():
    g = torch.Generator().manual_seed(1234)
    out = {}
    out["normal_w"] = (torch.randn(64 * 64, generator=g) * 0.02).float()
    out["fp16_randn"] = torch.randn(64, 64, generator=g, dtype=torch.float32).half().float().flatten()
    out["fp16_x1000"] = (torch.randn(32, 64, generator=g) * 1000).half().float().flatten()
    out["odd_201"] = torch.randn(201, generator=g).float()
    out["zeros"] = torch.zeros(64 * 4)
    tiny = torch.randn(64 * 4, generator=g) * 1e-10           # absmax < 1e-8 clamp
    sub = torch.randn(64 * 2, generator=g) * 1e-40             # fp32 subnormals
    out["tiny_and_subnormal"] = torch.cat([tiny, sub]).float()
    # Values on and next to every code midpoint, in blocks with absmax 1 and 0.37.
    mids = []
    for scale in (1.0, 0.37):
        for i in range(15):
            m = np.float32((CODES[i].item() + CODES[i + 1].item()) / 2 * scale)
            for d in range(-2, 3):
                mids.append(np.nextafter(m, np.float32(np.inf) if d > 0 else -np.float32(np.inf))
                            if d else m)
        mids.append(np.float32(scale))
        while len(mids) % 64:
            mids.append(np.float32(0.0))
    out["midpoints"] = torch.tensor(np.array(mids, np.float32))
    return out


def main():
    data = {}
    for name, x in cases().items():
        x = x.contiguous()
        n = x.numel()
        packed, absmax = torch_quantize(x.clone())
        data[f"{name}__x"] = x.numpy()
        data[f"{name}__packed"] = packed.numpy()
        data[f"{name}__absmax"] = absmax.numpy()
        data[f"{name}__f16"] = torch_dequant(packed, absmax, n, 64, torch.float16).view(torch.int16).numpy().view(np.uint16)
        data[f"{name}__bf16"] = torch_dequant(packed, absmax, n, 64, torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}: {len(data)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
