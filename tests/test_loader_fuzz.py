"""Seeded fuzzing of the shard loader's host code (CPU) under AddressSanitizer
and UndefinedBehaviorSanitizer.

The loader parses files a user hands it: the shard index and layer registry
(JSON, index.rs:7-34) and the safetensors shards it maps (loader.rs:53-206).
This test builds nf4_loader.hip's host code with both sanitizers
(tests/fuzz/loader_driver.cpp walks open, param_info, staging_size,
load_layer, pack_layer and blob_tensor), derives mutated shard directories
from a valid fixture (index field values and types, JSON text, shard bytes and
truncations, registry entries), and requires a clean run: no memory error and
no undefined behaviour, whatever the loader reports for each case."""
import json
import os
import random
import shutil
import subprocess
from pathlib import Path

import pytest

from shard_fixture import build_cpu_shards

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
REPO = Path(__file__).resolve().parents[1]
CASES = 240

VALS = [-1, 0, 1, 2, 4, 63, 64, 65, 255, 256, 2**31 - 1, 2**31, 2**32, 2**62, 2**63 - 1,
        -2**63, 1.5, 1e30, "x", None, [], {}, True, "nf4", "fp16", "U8", "F16",
        "../layer_0.safetensors", "layer_1.safetensors", "", "a" * 5000]
FIELDS = ["file_path", "byte_offset", "byte_length", "shape", "dtype", "precision",
          "nf4_block_size", "nf4_absmax_offset", "nf4_absmax_length", "nf4_absmax_q_offset",
          "nf4_absmax_q_length", "nf4_absmax_scale_offset", "nf4_absmax_scale_length",
          "nf4_dq_group"]
SHAPES = [[], [0], [128, 128], [2**40, 2**40], [2**31, 4], [1] * 9, [3, 5], [2**62, 8]]


def _mutate_index(rng, idx):
    for _ in range(rng.randint(1, 4)):
        e = idx[rng.choice(list(idx))]
        f = rng.choice(FIELDS)
        r = rng.random()
        if r < 0.15:
            e.pop(f, None)
        elif f == "shape" and r < 0.6:
            e[f] = rng.choice(SHAPES)
        elif isinstance(e.get(f), int) and r < 0.7:
            e[f] += rng.choice([-8, -4, -1, 1, 2, 3, 4, 8, 64, 4096, -4096, 10**6, 2**62])
        else:
            e[f] = rng.choice(VALS)
    return idx


def _mutate_bytes(rng, b: bytearray) -> bytes:
    r = rng.random()
    if r < 0.4:
        del b[rng.randint(0, len(b)):]
    elif r < 0.8:
        for _ in range(rng.randint(1, 16)):
            b[rng.randrange(len(b))] = rng.randrange(256)
    else:
        b[rng.randrange(len(b)):] = rng.choice([b"{" * 100, b'"\\ud800"', b"1e999", b"\xff\xfe",
                                                 b'{"a":' * 70, b"99999999999999999999999"])
    return bytes(b)


def _cases(root: Path, rng):
    bases = [root / "plain", root / "dq"]
    build_cpu_shards(bases[0], n_layers=2, dim=128, double_quant=False)
    build_cpu_shards(bases[1], n_layers=2, dim=128, double_quant=True)
    dirs = list(bases)
    for i in range(CASES):
        d = root / f"c{i}"
        shutil.copytree(bases[i % 2], d)
        kind = rng.random()
        ip, rp = d / "shard_index.json", d / "layer_registry.json"
        if kind < 0.5:
            ip.write_text(json.dumps(_mutate_index(rng, json.loads(ip.read_text()))))
        elif kind < 0.7:
            p = d / rng.choice(["layer_0.safetensors", "layer_1.safetensors"])
            p.write_bytes(_mutate_bytes(rng, bytearray(p.read_bytes())))
        elif kind < 0.85:
            ip.write_bytes(_mutate_bytes(rng, bytearray(ip.read_bytes())))
        else:
            reg = json.loads(rp.read_text())
            reg[rng.choice(list(reg))] = rng.choice([None, 5, "missing.safetensors", ".", "..",
                                                     "shard_index.json", "a" * 300])
            rp.write_text(json.dumps(reg))
        dirs.append(d)
    return dirs


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_loader_host_code_under_sanitizers(tmp_path):
    exe = tmp_path / "loader_fuzz"
    csrc = REPO / "aethelstream_amd" / "csrc"
    cmd = [HIPCC, "-O1", "-g", "-std=c++17", "--offload-arch=gfx950", "-fno-gpu-rdc",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined",
           "-Xarch_host", "-fno-omit-frame-pointer",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           f"-I{REPO / 'include'}", f"-I{csrc}",
           str(REPO / "tests" / "fuzz" / "loader_driver.cpp"),
           str(REPO / "tests" / "fuzz" / "dequant_stub.cpp"),
           str(csrc / "nf4_loader.hip"), str(csrc / "nf4_abi.hip"), "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stderr[-2000:]
    dirs = _cases(tmp_path / "cases", random.Random(2024))
    run = subprocess.run([str(exe), *map(str, dirs)], capture_output=True, text=True,
                         timeout=600)
    out = run.stdout + run.stderr
    assert run.returncode == 0, out[-3000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-3000:]
    opened = int(out.split("opened ")[1].split()[0])
    assert opened >= CASES // 4          # the mutations leave many directories loadable
