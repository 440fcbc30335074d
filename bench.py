"""Benchmark of the NF4 streamed-weight path on one MI355X.

Headline (``value``): NF4 dequant to bf16 of a full Llama-7B-shaped decoder
layer (benchmark config 2: q/k/v/o 4096x4096, gate/up 11008x4096, down
4096x11008; block 64; absmax double-quantized to uint8 in groups of 256 with
an fp32 scale), one grouped launch per step, inputs resident in HBM.
``value`` = algorithmic bytes (packed + uint8 absmax + fp32 scales + bf16 out
= 509,149,440 B) / average kernel time (HIP events on the launch stream), GB/s.

"dequant_cold": the same launch with inputs that cannot be cache hits: 4
distinct 7B layers (416 MB of NF4 inputs, beyond the 256 MB Infinity Cache)
dequantized in rotation, with its own roofline fraction.
"dequant_host_roundtrip": the same layer through the reference's host-slice
API (fp32 absmax in, f16 out, both in pinned host memory): H2D + dequant + D2H
per matrix on one stream, the PCIe-inclusive rate (never ``value``).

Also reported under "gemm": the NF4-dequant-fused GEMM in TFLOP/s against the
bf16 dense MFMA peak,
  config 3: 4096 tokens x (gate, up 11008x4096; down 4096x11008), forward;
  config 4: one 70B layer (q/o 8192x8192, k/v 1024x8192, gate/up 28672x8192,
            down 8192x28672; double-quant), 8192 tokens: forward +
            recompute-forward + input-gradient over all 7 matrices.

Under "stream", config 5: 80 70B layers in pinned host memory streamed
through a two-slot device buffer (H2D on a copy stream) while the previous
layer's forward GEMMs run, 4096 tokens: layers/s, H2D GB/s, overlap.

Config 4 also reports the forward pass with SwiGLU fused into the gate/up
epilogue (hidden = silu(x.Wg^T) * (x.Wu^T), forward.rs:251-254) next to the
grouped gate/up launch that writes gate and up.

Also under "gemm": "bf16_gemm_reference", a plain bf16 GEMM (torch.matmul,
hipBLASLt) of the 70B gate shape on the same box, and what an unfused path
(dequantize the layer to bf16, then that GEMM rate) would reach on config 4.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--workload all|dequant|dequant-cold|gemm|stream|quantize]
                       [--stream-layers L]
                       [--copy-calibration]
                       [--gemm-shape NAME [--gemm-mode fwd|dgrad|wgrad|swiglu] [--gemm-rotate R]]
  --workload dequant-cold runs only the cold-input dequant leg and prints its
  line (profiling).
  --workload quantize runs config 1 alone (oracle quantize on one core, then the
  device quantize of the same matrix) and prints only its line (profiling).
  --crossover times the 70B layer's forward and input-gradient passes fused and
  unfused at 256-8192 tokens and prints only that line.
  --gemm-shape times one fused GEMM (70b_q, 70b_k, 70b_gate, 70b_down, 7b_gate,
  7b_down) `steps` times after `warmup` and prints only its line (profiling);
  --gemm-mode bf16-reference times torch.matmul in bf16 on that shape instead;
  --gemm-rotate R (forward) cycles R distinct weights of the shape, so that the
  weight reads of a launch cannot be Infinity-Cache hits left by the last one.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, 2.5 PFLOP/s
ROOT = os.path.dirname(os.path.abspath(__file__))
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "dequant_7b_layer_pmc.txt")

LAYER_7B = [("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
            ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]
GEMM_7B = [("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]
LAYER_70B = [("q", 8192, 8192), ("k", 1024, 8192), ("v", 1024, 8192), ("o", 8192, 8192),
             ("gate", 28672, 8192), ("up", 28672, 8192), ("down", 8192, 28672)]
# name -> (tokens M, W rows N, W columns K)
GEMM_SHAPES = {"70b_q": (8192, 8192, 8192), "70b_k": (8192, 1024, 8192),
               "70b_gate": (8192, 28672, 8192), "70b_down": (8192, 8192, 28672),
               "7b_gate": (4096, 11008, 4096), "7b_down": (4096, 4096, 11008)}


# Seconds of untimed warm-up before each timed workload (--warm-seconds).
WARM_S = 0.5


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
    ap.add_argument("--warm-seconds", type=float, default=WARM_S,
                    help="untimed warm-up before each timed workload, after --warmup calls")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time budget of the dequant cpu_baseline sample")
    ap.add_argument("--workload", choices=["all", "dequant", "dequant-cold", "gemm", "stream",
                                           "quantize"],
                    default="all")
    ap.add_argument("--crossover", action="store_true",
                    help="time the 70B layer's fused and unfused passes over token counts "
                         "(256-8192) and print only that line")
    ap.add_argument("--stream-layers", type=int, default=80,
                    help="config 5: number of 70B layers held in pinned host memory")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (PMC byte calibration)")
    ap.add_argument("--gemm-shape", choices=sorted(GEMM_SHAPES), default=None,
                    help="only time one fused GEMM shape (for profiling)")
    ap.add_argument("--gemm-rotate", type=int, default=1,
                    help="with --gemm-shape and --gemm-mode fwd: cycle through this many "
                         "distinct weights of the shape (weights beyond the Infinity Cache)")
    ap.add_argument("--gemm-mode", choices=["fwd", "dgrad", "wgrad", "swiglu", "bf16-reference"],
                    default="fwd",
                    help="wgrad: the weight gradient dW[n,k] = dy^T.x over m tokens (fp32 out); "
                         "bf16-reference: torch.matmul (hipBLASLt) of the same shape in bf16")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_weights(torch, nf4, shapes, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    ws = []
    for _, r, c in shapes:
        wf = torch.randn(r, c, device="cuda", generator=g) * 0.02
        ws.append(nf4.quantize_weight(wf, double_quant=True))
        del wf
    torch.cuda.synchronize()
    return ws


def timed(torch, fn, steps, warmup, warm_s=None, name=None):
    """Average ms of fn() over `steps` runs, HIP events on the current stream
    (the stream every call here launches on).  Untimed warm-up: `warmup`
    calls, then more calls until `warm_s` seconds have passed (WARM_S by
    default): the GPU clock ramps up under load over a few tens of ms, and a
    workload timed right after an idle phase (weight generation, another
    config's setup) measured up to 15 % slow.  `name` labels the timed
    launches with a marker range (roctx), which rocprofv3 --marker-trace
    records, so a kernel trace can attribute them to their workload."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    deadline = time.perf_counter() + (WARM_S if warm_s is None else warm_s)
    while time.perf_counter() < deadline:
        fn()
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    if name:
        torch.cuda.nvtx.range_push(name)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    if name:
        torch.cuda.nvtx.range_pop()
    return start.elapsed_time(end) / steps


def read_traffic(path=TRAFFIC_FILE):
    """HBM bytes per dequant launch from a committed rocprofv3 PMC summary."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1].strip()))
    except OSError:
        pass
    return None


class pinned_core:
    """Pins the calling thread (the bench's main thread, which runs the oracle)
    to one core for the CPU legs and restores its mask afterwards, in-process:
    the GPU process never re-executes itself.  The reference path is
    single-threaded (shard_engine and doublepass start no threads)."""

    def __enter__(self):
        self.prev = os.sched_getaffinity(0)
        self.core = min(self.prev)
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.prev)


def host_facts() -> dict:
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(),
            "allowed_cores": len(os.sched_getaffinity(0))}


def algorithmic_bytes_fp32_absmax(shapes, bs=64) -> int:
    """The reference's own format (fp32 absmax, nf4.rs:37-83): 0.5 + 4/64 + 2
    bytes per element with f16 out."""
    total = 0
    for _, r, c in shapes:
        n = r * c
        total += n // 2 + 4 * ((n + bs - 1) // bs) + 2 * n
    return total


def cpu_baseline_dequant(ws, budget_s, core):
    """The oracle's dequant (scalar C restatement of shard_engine/src/nf4.rs:37-83,
    fp32 absmax in and f16 out, as the reference) on one pinned core, over
    whole matrices of the same layer until ~budget_s of CPU time.  The layer's
    double-quantized absmax is decoded to fp32 outside the timed region: the
    reference's format has fp32 absmax and no decode."""
    import oracle
    done_bytes, elapsed, mats, i = 0, 0.0, 0, 0
    while elapsed < budget_s and mats < 64:
        w = ws[i % len(ws)]
        pk = w.packed.cpu().numpy()
        am = oracle.dq_decode(w.absmax_q.cpu().numpy(), w.absmax_scale.cpu().numpy(),
                              w.dq_group)
        t0 = time.perf_counter()
        oracle.dequant_f16(pk, am, w.numel, w.block_size)
        elapsed += time.perf_counter() - t0
        done_bytes += algorithmic_bytes_fp32_absmax([("", w.shape[0], w.shape[1])])
        mats += 1
        i += 1
    return {
        "value": round(done_bytes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{mats} whole matrices of the same 7B layer in the reference's fp32-absmax "
                  f"format ({done_bytes} algorithmic bytes at 2.5625 B/element, "
                  f"{elapsed:.1f} s): oracle f16 dequant, 1 thread pinned to core {core}",
    }


def cpu_baseline_quantize(core):
    """Config 1 on the CPU: the oracle's quantize_nf4 (restatement of
    shard_engine/python/pipeline/quantizer.py:21-53) of one fp32 4096 x 4096
    ~ N(0, 0.02) matrix, one pinned core.  Returns the leg and its outputs
    (the device run is checked against them)."""
    import oracle
    x = oracle.gen_normal(1, 4096 * 4096, 0.02)
    t0 = time.perf_counter()
    pk, am = oracle.quantize_nf4(x)
    dt = time.perf_counter() - t0
    leg = {"value": round(x.nbytes / dt / 1e6, 2), "unit": "MB/s of fp32 input", "cores": 1,
           "kind": "port", "sample": f"config 1: one 4096x4096 fp32 matrix ({dt:.2f} s), "
                                     f"core {core}"}
    return leg, x, pk, am


def cpu_baseline_gemm(core, rows=8):
    """The oracle's matmul_tb (doublepass/src/math.rs:9-21) and its dY.W loop
    (doublepass/src/backward.rs:79-85), fp32, one pinned core, on `rows`-row
    slices of the 7B down projection; cost is linear in the row count."""
    import oracle
    d, ff = 4096, 11008
    w = oracle.gen_normal(12, d * ff, 0.02).reshape(d, ff)        # Wd [d, ff]
    h = oracle.gen_normal(11, rows * ff, 1.0).reshape(rows, ff)    # hidden [rows, ff]
    dy = oracle.gen_normal(13, rows * d, 1.0).reshape(rows, d)     # dY [rows, d]
    t0 = time.perf_counter()
    oracle.matmul_tb(h, w)                    # [rows, d] = hidden . Wd^T
    t1 = time.perf_counter()
    oracle.dgrad(dy, w)                       # [rows, ff] = dY . Wd
    t2 = time.perf_counter()
    fl = 2.0 * rows * d * ff
    return {
        "fwd": {"value": round(fl / (t1 - t0) / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
                "kind": "port", "sample": f"{rows} rows of the 7B down forward, hidden . Wd^T "
                f"({t1 - t0:.2f} s, core {core}); time scales linearly in M"},
        "dgrad": {"value": round(fl / (t2 - t1) / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
                  "kind": "port", "sample": f"{rows} rows of d_hidden = dY . Wd "
                  f"(backward.rs:79-85, {t2 - t1:.2f} s, core {core}); linear in M"},
    }


def bench_quantize_config1(torch, nf4, x, pk_ref, am_ref, args):
    """Config 1 on the device: nf4s_quantize of the same fp32 4096 x 4096
    matrix the CPU leg quantized (inputs resident), codes and absmax compared
    with the oracle's bit for bit."""
    import numpy as np
    from aethelstream_amd import _lib
    import ctypes
    xd = torch.from_numpy(x).cuda()
    n = xd.numel()
    packed = torch.empty((n + 1) // 2, dtype=torch.uint8, device="cuda")
    absmax = torch.empty((n + 63) // 64, dtype=torch.float32, device="cuda")
    lib = _lib.load()

    def run():
        _lib.check(lib.nf4s_quantize(xd.data_ptr(), n, 64, packed.data_ptr(),
                                     absmax.data_ptr(), torch.cuda.current_stream().cuda_stream))

    ms = timed(torch, run, args.steps, args.warmup, name="config1_quantize")
    torch.cuda.synchronize()
    exact = bool(np.array_equal(packed.cpu().numpy(), pk_ref) and
                 np.array_equal(absmax.cpu().numpy().view(np.uint32), am_ref.view(np.uint32)))
    moved = 4 * n + packed.numel() + 4 * absmax.numel()
    return {"ms": round(ms, 5), "input_gbs": round(4 * n / (ms * 1e-3) / 1e9, 2),
            "bytes_moved_gbs": round(moved / (ms * 1e-3) / 1e9, 2),
            "codes_absmax_bit_exact_vs_oracle": exact}


def bench_dequant(torch, nf4, args):
    log("building the 7B layer (quantize + double-quant on device)")
    ws = make_weights(torch, nf4, LAYER_7B, seed=2)
    outs = [torch.empty(w.shape, dtype=torch.bfloat16, device="cuda") for w in ws]
    log("timing the grouped dequant")
    ms = timed(torch, lambda: nf4.dequant_batch(ws, outs), args.steps, args.warmup,
               name="config2_dequant")
    return ws, ms


COLD_LAYERS = 4
COLD_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "dequant_7b_cold_pmc.txt")


def bench_dequant_cold(torch, nf4, args, ws0=None):
    """The headline launch on inputs that cannot be cache hits: COLD_LAYERS
    distinct 7B layers (each its own packed codes, absmax codes and scales,
    104 MB; 416 MB together, beyond the 256 MB Infinity Cache) and as many
    output sets, one layer per step in rotation, so every launch reads
    inputs last touched COLD_LAYERS - 1 launches (1.5 GB of traffic) ago."""
    log(f"cold-input dequant: {COLD_LAYERS} distinct 7B layers in rotation")
    layers = [ws0] if ws0 is not None else []
    while len(layers) < COLD_LAYERS:
        layers.append(make_weights(torch, nf4, LAYER_7B, seed=20 + len(layers)))
    outs = [[torch.empty(w.shape, dtype=torch.bfloat16, device="cuda") for w in ws]
            for ws in layers]
    it = [0]

    def step():
        i = it[0] % COLD_LAYERS
        it[0] += 1
        nf4.dequant_batch(layers[i], outs[i])

    steps = max(COLD_LAYERS, (args.steps + COLD_LAYERS - 1) // COLD_LAYERS * COLD_LAYERS)
    ms = timed(torch, step, steps, COLD_LAYERS, name="config2_dequant_cold")
    nbytes = algorithmic_bytes_dq(LAYER_7B)
    gbs = nbytes / (ms * 1e-3) / 1e9
    in_bytes = sum(w.packed.numel() + w.absmax_q.numel() + 4 * w.absmax_scale.numel()
                   for ws in layers for w in ws)
    return {"gbs": round(gbs, 2), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "us_per_launch": round(ms * 1e3, 2), "layers_rotated": COLD_LAYERS,
            "input_bytes_rotated": in_bytes,
            "output_bytes_rotated": sum(o.numel() * 2 for os_ in outs for o in os_),
            "steps": steps, "traffic": read_traffic(COLD_TRAFFIC_FILE),
            "note": "same grouped launch as value; each launch's inputs were last read "
                    f"{COLD_LAYERS - 1} launches earlier, with 416 MB of other inputs and "
                    "1.2 GB of other outputs in between"}


def bench_dequant_host(torch, nf4, args):
    """PCIe-inclusive rate of the reference's host-slice API (nf4.rs:37-83:
    packed and absmax in host memory, f16 out to host memory) as the Rust
    `hip` body runs it: per matrix of the 7B layer, H2D copy of packed bytes
    and fp32 absmax (the reference's on-disk format), the f16 dequant, D2H
    copy of the output; pinned host buffers, device staging kept, one stream.
    Not the headline: the headline's inputs are already resident in HBM."""
    g = torch.Generator(device="cuda").manual_seed(3)
    mats = []
    for _, r, c in LAYER_7B:
        w = nf4.quantize_weight(torch.randn(r, c, device="cuda", generator=g) * 0.02,
                                double_quant=False)
        n = r * c
        ph = torch.empty(w.packed.numel(), dtype=torch.uint8, pin_memory=True)
        ah = torch.empty(w.absmax.numel(), dtype=torch.float32, pin_memory=True)
        ph.copy_(w.packed)
        ah.copy_(w.absmax)
        oh = torch.empty(n, dtype=torch.float16, pin_memory=True)
        od = torch.empty(n, dtype=torch.float16, device="cuda")
        mats.append((ph, ah, oh, w.packed, w.absmax, od))
    torch.cuda.synchronize()

    def step():
        for ph, ah, oh, pd, ad, od in mats:
            pd.copy_(ph, non_blocking=True)
            ad.copy_(ah, non_blocking=True)
            nf4.dequant_nf4_into(pd, ad, od, 64)
            oh.copy_(od, non_blocking=True)

    ms = timed(torch, step, max(2, args.steps // 10), 1, name="dequant_host_roundtrip")
    n_el = sum(r * c for _, r, c in LAYER_7B)
    alg = n_el // 2 + 4 * (n_el // 64) + 2 * n_el
    return {"gbs": round(alg / (ms * 1e-3) / 1e9, 2), "ms": round(ms, 3),
            "algorithmic_bytes": alg, "h2d_bytes": n_el // 2 + 4 * (n_el // 64),
            "d2h_bytes": 2 * n_el,
            "note": "7B layer, fp32 absmax, f16 out; per matrix H2D + dequant + D2H on one "
                    "stream, pinned host buffers"}


def bench_gemm(torch, nf4, gemm, args):
    res = {}
    # Config 3: 7B MLP GEMMs, forward, 4096 tokens.
    log("config 3: 7B gate/up/down forward")
    ws = make_weights(torch, nf4, GEMM_7B, seed=3)
    g = torch.Generator(device="cuda").manual_seed(30)
    x = torch.randn(4096, 4096, device="cuda", generator=g).to(torch.bfloat16)
    xd = torch.randn(4096, 11008, device="cuda", generator=g).to(torch.bfloat16)
    ys = [torch.empty(4096, w.shape[0], dtype=torch.bfloat16, device="cuda") for w in ws]
    acts = [x, x, xd]

    def cfg3():
        # gate and up share x: one grouped launch (forward.rs:251-252).
        gemm.linear_fwd_grouped(x, ws[:2], ys[:2])
        gemm.linear_fwd(xd, ws[2], ys[2])
    steps = max(3, args.steps // 5)
    ms3 = timed(torch, cfg3, steps, 2, name="config3")
    fl3 = sum(2.0 * 4096 * w.shape[0] * w.shape[1] for w in ws)
    tf3 = fl3 / (ms3 * 1e-3) / 1e12
    res["config3_7b_mlp_fwd"] = {"tflops": round(tf3, 1), "ms": round(ms3, 4), "flop": fl3,
                                 "launches": "[gate,up] grouped, down",
                                 "frac_of_bf16_peak": round(tf3 / BF16_PEAK_TFLOPS, 4)}
    del ws, x, xd, ys, acts
    torch.cuda.empty_cache()

    # Config 4: a 70B layer, forward + recompute-forward + dgrad, 8192 tokens.
    log("config 4: 70B layer forward + recompute + dgrad")
    M = 8192
    ws = make_weights(torch, nf4, LAYER_70B, seed=4)
    g = torch.Generator(device="cuda").manual_seed(40)
    h = torch.randn(M, 8192, device="cuda", generator=g).to(torch.bfloat16)
    hid = torch.randn(M, 28672, device="cuda", generator=g).to(torch.bfloat16)
    ins = [h, h, h, h, h, h, hid]                    # q k v o gate up : down
    ys = [torch.empty(M, w.shape[0], dtype=torch.bfloat16, device="cuda") for w in ws]
    dys = [torch.randn(M, w.shape[0], device="cuda", generator=g).to(torch.bfloat16) for w in ws]
    dxs = [torch.empty(M, w.shape[1], dtype=torch.bfloat16, device="cuda") for w in ws]

    # The layer's GEMMs as single_layer_forward / single_layer_backward
    # issue them: q/k/v and gate/up share their input (forward.rs:174-176,
    # 251-252); the input gradients of q/k/v and of gate/up are sums
    # (backward.rs:284-300, 117-129).
    def fwd_pass():
        gemm.linear_fwd_grouped(h, ws[0:3], ys[0:3])        # q, k, v
        gemm.linear_fwd(h, ws[3], ys[3])                    # o
        gemm.linear_fwd_grouped(h, ws[4:6], ys[4:6])        # gate, up
        gemm.linear_fwd(hid, ws[6], ys[6])                  # down

    def dgrad_pass():
        gemm.linear_dgrad_sum(dys[0:3], ws[0:3], dxs[0])    # d_h1
        gemm.linear_dgrad(dys[3], ws[3], dxs[3])            # d_attn_out
        gemm.linear_dgrad_sum(dys[4:6], ws[4:6], dxs[4])    # d_h2
        gemm.linear_dgrad(dys[6], ws[6], dxs[6])            # d_hidden

    def layer_step():
        fwd_pass()      # forward
        fwd_pass()      # double-pass recompute forward
        dgrad_pass()    # input gradient

    # The weight gradients beside the input gradients (backward.rs:87-93,
    # 117-129, 160-168, 284-300): dW_i = dy_i^T . input_i in fp32, plain bf16
    # GEMMs (no NF4 operand), reported apart from the NF4 path's rate; those
    # that share an input (q/k/v, gate/up) in one grouped launch, and all
    # seven as single launches for comparison.
    dws = [torch.empty(w.shape[0], w.shape[1], dtype=torch.float32, device="cuda") for w in ws]

    def wgrad_pass():
        gemm.linear_wgrad_grouped(dys[0:3], h, dws[0:3])     # d_wq, d_wk, d_wv
        gemm.linear_wgrad(dys[3], h, dws[3])                 # d_wo
        gemm.linear_wgrad_grouped(dys[4:6], h, dws[4:6])     # d_wg, d_wu
        gemm.linear_wgrad(dys[6], hid, dws[6])               # d_wd

    def wgrad_pass_single():
        for dy, a, dw in zip(dys, ins, dws):
            gemm.linear_wgrad(dy, a, dw)

    steps4 = max(2, args.steps // 10)
    ms_f = timed(torch, fwd_pass, steps4, 1, name="config4_fwd_pass")
    ms_d = timed(torch, dgrad_pass, steps4, 1, name="config4_dgrad_pass")
    ms_l = timed(torch, layer_step, steps4, 1, name="config4_layer_step")
    fl_pass = sum(2.0 * M * w.shape[0] * w.shape[1] for w in ws)
    per = {}
    for (name, _, _), a, w, y, dy, dx in zip(LAYER_70B, ins, ws, ys, dys, dxs):
        f = 2.0 * M * w.shape[0] * w.shape[1]
        mf = timed(torch, lambda: gemm.linear_fwd(a, w, y), steps4, 1, name=f"fwd_{name}")
        md = timed(torch, lambda: gemm.linear_dgrad(dy, w, dx), steps4, 1, name=f"dgrad_{name}")
        per[name] = {"fwd_tflops": round(f / (mf * 1e-3) / 1e12, 1),
                     "dgrad_tflops": round(f / (md * 1e-3) / 1e12, 1)}
    # The first forward of a double-pass step only hands `hidden` to down:
    # SwiGLU fused into the gate/up epilogue (forward.rs:251-254).
    hsw = torch.empty(M, 28672, dtype=torch.bfloat16, device="cuda")

    def fwd_pass_swiglu():
        gemm.linear_fwd_grouped(h, ws[0:3], ys[0:3])
        gemm.linear_fwd(h, ws[3], ys[3])
        gemm.linear_swiglu(h, ws[4], ws[5], hsw)
        gemm.linear_fwd(hsw, ws[6], ys[6])

    ms_fs = timed(torch, fwd_pass_swiglu, steps4, 1, name="config4_fwd_pass_swiglu")
    ms_w = timed(torch, wgrad_pass, steps4, 1, name="config4_wgrad_pass")
    ms_w1 = timed(torch, wgrad_pass_single, steps4, 1, name="config4_wgrad_pass_single")
    fl_gu = 2 * 2.0 * M * 28672 * 8192
    ms_gu = timed(torch, lambda: gemm.linear_fwd_grouped(h, ws[4:6], ys[4:6]), steps4, 1,
                  name="gate_up_grouped")
    ms_sw = timed(torch, lambda: gemm.linear_swiglu(h, ws[4], ws[5], hsw), steps4, 1,
                  name="gate_up_swiglu")
    # The unfused alternative, measured end to end: each pass dequantizes the
    # layer's 7 weights to bf16 (one grouped launch), then runs the same
    # products as plain bf16 GEMMs in torch (hipBLASLt): x . W^T forward,
    # dY . W input gradient with the sums accumulated by addmm.
    wbf = [torch.empty(w.shape, dtype=torch.bfloat16, device="cuda") for w in ws]

    def unfused_fwd_pass():
        nf4.dequant_batch(ws, wbf)
        for a, wb, y in zip(ins, wbf, ys):
            torch.matmul(a, wb.t(), out=y)

    def unfused_dgrad_pass():
        nf4.dequant_batch(ws, wbf)
        torch.matmul(dys[0], wbf[0], out=dxs[0])
        dxs[0].addmm_(dys[1], wbf[1])
        dxs[0].addmm_(dys[2], wbf[2])
        torch.matmul(dys[3], wbf[3], out=dxs[3])
        torch.matmul(dys[4], wbf[4], out=dxs[4])
        dxs[4].addmm_(dys[5], wbf[5])
        torch.matmul(dys[6], wbf[6], out=dxs[6])

    def unfused_layer_step():
        unfused_fwd_pass()
        unfused_fwd_pass()
        unfused_dgrad_pass()

    ms_u = timed(torch, unfused_layer_step, steps4, 1, name="config4_unfused_layer_step")
    ms_uf = timed(torch, unfused_fwd_pass, steps4, 1, name="config4_unfused_fwd_pass")
    del wbf
    # RMSNorm before q/k/v and before gate/up (forward.rs:173, 249), run
    # unfused: its time bounds what fusing it into the GEMM could save.
    from aethelstream_amd import norm
    xr = torch.randn(M, 8192, device="cuda", generator=g)
    wr = 1.0 + 0.1 * torch.randn(8192, device="cuda", generator=g)
    hr = torch.empty(M, 8192, dtype=torch.bfloat16, device="cuda")
    rr = torch.empty(M, dtype=torch.float32, device="cuda")
    ms_rn = timed(torch, lambda: norm.rms_norm_fwd(xr, wr, out=hr, rms=rr), args.steps, 1,
                  name="rmsnorm_70b")

    def fwd_pass_with_norms():
        norm.rms_norm_fwd(xr, wr, out=hr, rms=rr)
        gemm.linear_fwd_grouped(hr, ws[0:3], ys[0:3])
        gemm.linear_fwd(h, ws[3], ys[3])
        norm.rms_norm_fwd(xr, wr, out=hr, rms=rr)
        gemm.linear_fwd_grouped(hr, ws[4:6], ys[4:6])
        gemm.linear_fwd(hid, ws[6], ys[6])

    ms_fn = timed(torch, fwd_pass_with_norms, steps4, 1, name="config4_fwd_pass_with_rmsnorm")
    del xr, hr
    tf_l = 3 * fl_pass / (ms_l * 1e-3) / 1e12
    res["config4_70b_layer"] = {
        "tflops": round(tf_l, 1), "ms_per_layer_step": round(ms_l, 3),
        "flop_per_pass": fl_pass, "passes": 3,
        "launches": "fwd: [q,k,v] grouped, o, [gate,up] grouped, down; dgrad: dq.Wq+dk.Wk+dv.Wv "
                    "summed, o, d_gate.Wg+d_up.Wu summed, down",
        "frac_of_bf16_peak": round(tf_l / BF16_PEAK_TFLOPS, 4),
        "fwd_pass_tflops": round(fl_pass / (ms_f * 1e-3) / 1e12, 1),
        "fwd_pass_swiglu_tflops": round(fl_pass / (ms_fs * 1e-3) / 1e12, 1),
        "gate_up_grouped_tflops": round(fl_gu / (ms_gu * 1e-3) / 1e12, 1),
        "gate_up_swiglu_fused_tflops": round(fl_gu / (ms_sw * 1e-3) / 1e12, 1),
        "dgrad_pass_tflops": round(fl_pass / (ms_d * 1e-3) / 1e12, 1),
        "wgrad_pass_tflops": round(fl_pass / (ms_w * 1e-3) / 1e12, 1),
        "wgrad_pass_single_launch_tflops": round(fl_pass / (ms_w1 * 1e-3) / 1e12, 1),
        "per_matrix": per,
        "unfused_measured": {
            "op": "per pass: nf4s_dequant_batch_bf16 of the 7 weights, then torch.matmul / "
                  "addmm in bf16 (hipBLASLt)",
            "tflops": round(3 * fl_pass / (ms_u * 1e-3) / 1e12, 1),
            "ms_per_layer_step": round(ms_u, 3),
            "fwd_pass_tflops": round(fl_pass / (ms_uf * 1e-3) / 1e12, 1),
            "fused_speedup": round(ms_u / ms_l, 3),
        },
        "rmsnorm": {
            "op": "nf4s_rmsnorm_fwd, x fp32 [8192, 8192] -> bf16, unfused",
            "us": round(ms_rn * 1e3, 2),
            "gbs": round(6 * M * 8192 / (ms_rn * 1e-3) / 1e9, 1),
            "fwd_pass_ms": round(ms_f, 3),
            "fwd_pass_with_two_rmsnorms_ms": round(ms_fn, 3),
            "share_of_fwd_pass": round((ms_fn - ms_f) / ms_fn, 4),
        },
    }
    return res


def bench_stream(torch, nf4, gemm, nlayers, M=4096):
    """Config 5: `nlayers` 70B-shaped NF4 layers (double-quant) in pinned host
    memory, each copied H2D on a side stream while the previous layer's
    fused forward GEMMs run on the compute stream (flowcast's VRAM double
    buffer), M tokens."""
    from aethelstream_amd import stream as st
    layout = st.LayerLayout(LAYER_70B)
    t0 = time.perf_counter()
    distinct = [make_weights(torch, nf4, LAYER_70B, seed=100 + i) for i in range(4)]
    host = []
    for l in range(nlayers):
        pb = st.PinnedBuffer(layout.nbytes)
        layout.pack_into(pb.tensor, distinct[l % len(distinct)])
        host.append(pb)
    # The resident copy holds the last layer's blob: after the streamed run,
    # its outputs must equal the last streamed layer's.
    resident = torch.empty(layout.nbytes, dtype=torch.uint8, device="cuda")
    resident.copy_(host[nlayers - 1].tensor)
    del distinct
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    dbuf = st.VramDoubleBuffer(layout.nbytes)
    g = torch.Generator(device="cuda").manual_seed(50)
    x = torch.randn(M, 8192, device="cuda", generator=g).to(torch.bfloat16)
    hid = torch.randn(M, 28672, device="cuda", generator=g).to(torch.bfloat16)
    ins = [x, x, x, x, x, x, hid]
    outs = [torch.empty(M, r, dtype=torch.bfloat16, device="cuda") for _, r, _ in LAYER_70B]
    comp = torch.cuda.current_stream()

    def compute(l, views):
        gemm.linear_fwd_grouped(x, views[0:3], outs[0:3])
        gemm.linear_fwd(x, views[3], outs[3])
        gemm.linear_fwd_grouped(x, views[4:6], outs[4:6])
        gemm.linear_fwd(hid, views[6], outs[6])

    def wall(fn, name):
        # A marker range per phase, so a kernel + memory-copy trace can
        # attribute the copies and the GEMMs to it.
        torch.cuda.synchronize()
        torch.cuda.nvtx.range_push(name)
        t = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        t = time.perf_counter() - t
        torch.cuda.nvtx.range_pop()
        return t

    def copies_only():
        for l in range(nlayers):
            p, ev = dbuf.advance(l, host[l].ptr, layout.nbytes)
            st.stream_wait_event(comp, ev)
            dbuf.release(p, comp)

    rviews = layout.views(resident.data_ptr())

    def compute_only():
        for l in range(nlayers):
            compute(l, rviews)

    def streamed():
        st.run_stack(host, layout, dbuf, compute, comp)

    wall(streamed, "config5_warmup")
    t_h2d = wall(copies_only, "config5_copies_only")
    t_comp = wall(compute_only, "config5_compute_only")
    t_tot = wall(streamed, "config5_streamed")
    last = [o.clone() for o in outs]
    compute(nlayers - 1, rviews)
    torch.cuda.synchronize()
    if not all(torch.equal(a, b) for a, b in zip(last, outs)):
        raise RuntimeError("config 5: the last streamed layer's outputs differ from the "
                           "resident run over the same blob")
    del last
    fl = nlayers * sum(2.0 * M * r * c for _, r, c in LAYER_70B)
    dbuf.close()
    for pb in host:
        pb.close()
    return {
        "layers": nlayers, "tokens": M, "layer_bytes": layout.nbytes,
        "layers_per_s": round(nlayers / t_tot, 2),
        "ms_per_layer": round(1e3 * t_tot / nlayers, 3),
        "h2d_gbs": round(nlayers * layout.nbytes / t_h2d / 1e9, 2),
        "t_h2d_s": round(t_h2d, 4), "t_compute_s": round(t_comp, 4), "t_total_s": round(t_tot, 4),
        "overlap": round((t_h2d + t_comp - t_tot) / min(t_h2d, t_comp), 3),
        "tflops_streamed": round(fl / t_tot / 1e12, 1),
        "tflops_resident": round(fl / t_comp / 1e12, 1),
        "setup_s": round(setup_s, 1),
        "last_layer_equals_resident": True,
    }


def bench_one_gemm(torch, nf4, gemm, args):
    """One fused GEMM shape, args.steps timed launches (HIP events)."""
    m, n, k = GEMM_SHAPES[args.gemm_shape]
    g = torch.Generator(device="cuda").manual_seed(7)
    w = nf4.quantize_weight(torch.randn(n, k, device="cuda", generator=g) * 0.02, double_quant=True)
    if args.gemm_mode == "fwd" and args.gemm_rotate > 1:
        # Distinct weights of the shape in rotation (--gemm-rotate): each
        # launch reads NF4 bytes last read gemm_rotate - 1 launches earlier.
        rot = [w] + [nf4.quantize_weight(torch.randn(n, k, device="cuda", generator=g) * 0.02,
                                         double_quant=True)
                     for _ in range(args.gemm_rotate - 1)]
        a = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
        o = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        it = [0]

        def fn():
            gemm.linear_fwd(a, rot[it[0] % len(rot)], o)
            it[0] += 1
    elif args.gemm_mode == "fwd":
        a = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
        o = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        fn = lambda: gemm.linear_fwd(a, w, o)
    elif args.gemm_mode == "bf16-reference":
        a = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
        b = torch.randn(n, k, device="cuda", generator=g).to(torch.bfloat16)
        o = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        fn = lambda: torch.matmul(a, b.t(), out=o)
    elif args.gemm_mode == "swiglu":
        # hidden = silu(x.Wg^T) * (x.Wu^T), gate and up both of this shape.
        wu = nf4.quantize_weight(torch.randn(n, k, device="cuda", generator=g) * 0.02,
                                 double_quant=True)
        a = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
        o = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        fn = lambda: gemm.linear_swiglu(a, w, wu, o)
    elif args.gemm_mode == "wgrad":
        a = torch.randn(m, n, device="cuda", generator=g).to(torch.bfloat16)
        b = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
        o = torch.empty(n, k, dtype=torch.float32, device="cuda")
        fn = lambda: gemm.linear_wgrad(a, b, o)
    else:
        a = torch.randn(m, n, device="cuda", generator=g).to(torch.bfloat16)
        o = torch.empty(m, k, dtype=torch.bfloat16, device="cuda")
        fn = lambda: gemm.linear_dgrad(a, w, o)
    ms = timed(torch, fn, args.steps, args.warmup, name=f"{args.gemm_shape}_{args.gemm_mode}")
    tf = (4.0 if args.gemm_mode == "swiglu" else 2.0) * m * n * k / (ms * 1e-3) / 1e12
    print(json.dumps({"gemm_shape": args.gemm_shape, "mode": args.gemm_mode, "m": m, "n": n,
                      "k": k, "ms": round(ms, 4), "tflops": round(tf, 1),
                      "weights_rotated": max(1, args.gemm_rotate)}), flush=True)


def bench_crossover(torch, nf4, gemm, args):
    """The 70B layer's forward and input-gradient passes, fused against
    unfused (dequantize the 7 weights to bf16 in one launch, then torch bf16
    GEMMs, as unfused_measured), over token counts: where the fused kernels'
    saving (no bf16 copy of the weights written and read) outweighs their
    lower MFMA rate.  Prints one JSON line."""
    ws = make_weights(torch, nf4, LAYER_70B, seed=4)
    wbf = [torch.empty(w.shape, dtype=torch.bfloat16, device="cuda") for w in ws]
    g = torch.Generator(device="cuda").manual_seed(41)
    fl_w = sum(2.0 * w.shape[0] * w.shape[1] for w in ws)
    rows = []
    for M in (256, 512, 1024, 2048, 4096, 8192):
        h = torch.randn(M, 8192, device="cuda", generator=g).to(torch.bfloat16)
        hid = torch.randn(M, 28672, device="cuda", generator=g).to(torch.bfloat16)
        ins = [h, h, h, h, h, h, hid]
        ys = [torch.empty(M, w.shape[0], dtype=torch.bfloat16, device="cuda") for w in ws]
        dys = [torch.randn(M, w.shape[0], device="cuda", generator=g).to(torch.bfloat16)
               for w in ws]
        dxs = [torch.empty(M, w.shape[1], dtype=torch.bfloat16, device="cuda") for w in ws]

        def fused_fwd():
            gemm.linear_fwd_grouped(h, ws[0:3], ys[0:3])
            gemm.linear_fwd(h, ws[3], ys[3])
            gemm.linear_fwd_grouped(h, ws[4:6], ys[4:6])
            gemm.linear_fwd(hid, ws[6], ys[6])

        def fused_dgrad():
            gemm.linear_dgrad_sum(dys[0:3], ws[0:3], dxs[0])
            gemm.linear_dgrad(dys[3], ws[3], dxs[3])
            gemm.linear_dgrad_sum(dys[4:6], ws[4:6], dxs[4])
            gemm.linear_dgrad(dys[6], ws[6], dxs[6])

        def unfused_fwd():
            nf4.dequant_batch(ws, wbf)
            for a, wb, y in zip(ins, wbf, ys):
                torch.matmul(a, wb.t(), out=y)

        def unfused_dgrad():
            nf4.dequant_batch(ws, wbf)
            torch.matmul(dys[0], wbf[0], out=dxs[0])
            dxs[0].addmm_(dys[1], wbf[1])
            dxs[0].addmm_(dys[2], wbf[2])
            torch.matmul(dys[3], wbf[3], out=dxs[3])
            torch.matmul(dys[4], wbf[4], out=dxs[4])
            dxs[4].addmm_(dys[5], wbf[5])
            torch.matmul(dys[6], wbf[6], out=dxs[6])

        k = max(3, args.steps // 5)
        t = {name: timed(torch, fn, k, 1, warm_s=0.2, name=f"crossover_{name}_m{M}")
             for name, fn in (("fused_fwd", fused_fwd), ("unfused_fwd", unfused_fwd),
                              ("fused_dgrad", fused_dgrad), ("unfused_dgrad", unfused_dgrad))}
        fl = M * fl_w
        rows.append({"tokens": M,
                     **{f"{n}_ms": round(v, 4) for n, v in t.items()},
                     **{f"{n}_tflops": round(fl / (v * 1e-3) / 1e12, 1) for n, v in t.items()},
                     "fwd_unfused_over_fused_time": round(t["unfused_fwd"] / t["fused_fwd"], 3),
                     "dgrad_unfused_over_fused_time": round(t["unfused_dgrad"] / t["fused_dgrad"],
                                                            3)})
        log(f"crossover M={M}: {rows[-1]}")
        del h, hid, ins, ys, dys, dxs
    print(json.dumps({"crossover_70b_layer": rows,
                      "note": "per pass; unfused = one nf4s_dequant_batch_bf16 of the layer's 7 "
                              "weights + torch bf16 GEMMs (hipBLASLt); >1 means fused is faster"}),
          flush=True)


def bf16_gemm_reference(torch, dequant_gbs, layer_ms):
    """A plain bf16 GEMM (torch.matmul -> hipBLASLt) of the 70B gate shape, and
    the config-4 rate of an unfused path: dequantize each pass's weights to
    bf16 (at the measured dequant rate), then GEMMs at that plain rate."""
    m, n, k = GEMM_SHAPES["70b_gate"]
    g = torch.Generator(device="cuda").manual_seed(9)
    a = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    b = torch.randn(n, k, device="cuda", generator=g).to(torch.bfloat16)
    o = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    ms = timed(torch, lambda: torch.matmul(a, b.t(), out=o), 5, 2, name="bf16_reference")
    tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    res = {"op": "torch.matmul bf16 (hipBLASLt), M=8192 N=28672 K=8192", "tflops": round(tf, 1),
           "frac_of_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
    if dequant_gbs and layer_ms:
        fl_pass = sum(2.0 * 8192 * r * c for _, r, c in LAYER_70B)
        deq_ms = algorithmic_bytes_dq(LAYER_70B) / (dequant_gbs * 1e9) * 1e3
        unfused_ms = 3 * (deq_ms + fl_pass / (tf * 1e12) * 1e3)
        res["unfused_config4_tflops"] = round(3 * fl_pass / (unfused_ms * 1e-3) / 1e12, 1)
        # unfused time / fused time: above 1 the fused kernels are faster,
        # below 1 dequantize-then-hipBLASLt would be.
        res["fused_speedup_over_unfused"] = round(unfused_ms / layer_ms, 3)
    return res


def hbm_copy_ceiling(torch):
    """The box's measured HBM ceiling for a plain streaming copy: torch's
    device copy of 1 GiB (1 GiB read + 1 GiB written per call), far larger
    than the 256 MB Infinity Cache.  A reported ceiling beside the 8 TB/s
    nominal peak that `roofline.frac` is quoted against."""
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    ms = timed(torch, lambda: b.copy_(a), 10, 2, name="hbm_copy")
    gbs = 2.0 * n / (ms * 1e-3) / 1e9
    del a, b
    return {"op": "torch copy, 1 GiB each way", "gbs": round(gbs, 1),
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}


def copy_calibration(torch):
    """A plain device copy of exactly 1 GiB read + 1 GiB written (the known
    byte count that rocprofv3's FETCH_SIZE / WRITE_SIZE are scaled against)."""
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_each_way": n, "launches": 3}), flush=True)


def main():
    global WARM_S
    args = parse()
    WARM_S = args.warm_seconds
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU (every GPU box here has one); "
                                   "bench.py --gpus N with N > 1 is not supported"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(torch)
        return
    from aethelstream_amd import gemm, nf4
    if args.gemm_shape:
        bench_one_gemm(torch, nf4, gemm, args)
        return
    if args.crossover:
        bench_crossover(torch, nf4, gemm, args)
        return
    if args.workload == "quantize":
        # Config 1 alone (the program the quantize kernel trace runs): the
        # oracle's quantize of the matrix on one pinned core, then the device
        # quantize of the same matrix, checked bit for bit.
        with pinned_core() as pc:
            leg, x1, pk1, am1 = cpu_baseline_quantize(pc.core)
        print(json.dumps({"quantize_config1": bench_quantize_config1(torch, nf4, x1, pk1, am1,
                                                                     args),
                          "cpu_baseline_quantize_config1": leg}), flush=True)
        return
    if args.workload == "dequant-cold":
        # The cold-input leg alone (the program its counter runs profile).
        print(json.dumps({"dequant_cold": bench_dequant_cold(torch, nf4, args)}), flush=True)
        return

    line = {
        "metric": "NF4 dequant HBM GB/s (% peak); NF4-fused GEMM TFLOP/s at 7B/70B layer shapes",
        "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warm_seconds": args.warm_seconds, "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: torch.randn weights (sigma 0.02) quantized on device, "
                "randn activations",
        "config": {"workload": "config2: NF4 dequant to bf16 of one Llama-7B decoder layer "
                               "(q/k/v/o 4096x4096, gate/up 11008x4096, down 4096x11008), "
                               "block 64, double-quant uint8 absmax in groups of 256, one "
                               "grouped launch per step",
                   "elements": sum(r * c for _, r, c in LAYER_7B),
                   "algorithmic_bytes": algorithmic_bytes_dq(LAYER_7B)},
    }
    ws = None
    if args.workload in ("all", "dequant"):
        ws, ms = bench_dequant(torch, nf4, args)
        nbytes = algorithmic_bytes_dq(LAYER_7B)
        gbs = nbytes / (ms * 1e-3) / 1e9
        line["value"] = round(gbs, 2)
        line["ms_per_step"] = round(ms, 5)
        line["roofline"] = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                            "traffic": read_traffic()}
        line["dequant_cold"] = bench_dequant_cold(torch, nf4, args, ws)
        log("HBM copy ceiling")
        line["hbm_copy_ceiling"] = hbm_copy_ceiling(torch)
        log("PCIe-inclusive host-slice dequant")
        line["dequant_host_roundtrip"] = bench_dequant_host(torch, nf4, args)
    if args.workload in ("all", "gemm"):
        line["gemm"] = bench_gemm(torch, nf4, gemm, args)
        line["gemm"]["peak_tflops"] = BF16_PEAK_TFLOPS
        log("plain bf16 GEMM reference")
        line["gemm"]["bf16_gemm_reference"] = bf16_gemm_reference(
            torch, line.get("value"), line["gemm"]["config4_70b_layer"]["ms_per_layer_step"])
    if args.workload in ("all", "stream"):
        log(f"config 5: {args.stream_layers} streamed 70B layers")
        try:
            line["stream"] = bench_stream(torch, nf4, gemm, args.stream_layers)
        except Exception as e:  # reported, the rest of the line still prints
            line["stream"] = {"error": repr(e)}
    if not args.no_cpu_baseline and ws is not None:
        log("cpu baseline (oracle, 1 pinned core)")
        legs = {"host": host_facts()}
        with pinned_core() as pc:
            line["cpu_baseline"] = cpu_baseline_dequant(ws, args.cpu_seconds, pc.core)
            if args.workload == "all":
                legs["quantize_config1"], x1, pk1, am1 = cpu_baseline_quantize(pc.core)
                legs.update(cpu_baseline_gemm(pc.core))
        line["cpu_baseline_legs"] = legs
        if args.workload == "all":
            log("config 1: device quantize")
            line["quantize_config1"] = bench_quantize_config1(torch, nf4, x1, pk1, am1, args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
