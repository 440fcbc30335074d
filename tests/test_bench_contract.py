"""bench.py's contract on the CPU: the algorithmic byte count behind the
headline roofline, and the one-GPU guard (no GPU is touched)."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_algorithmic_bytes_of_the_7b_layer():
    # 0.5 (packed) + 1/64 (uint8 absmax) + 4/16384 (fp32 scale per 256 blocks)
    # + 2 (bf16 out) bytes per element over 202,375,168 elements.
    n = sum(r * c for _, r, c in bench.LAYER_7B)
    assert n == 202_375_168
    assert bench.algorithmic_bytes_dq(bench.LAYER_7B) == 509_149_440
    # A single 4096 x 4096 matrix: 8 M packed, 256 K codes, 1 K scales, 32 M out.
    assert bench.algorithmic_bytes_dq([("q", 4096, 4096)]) == (
        4096 * 4096 // 2 + 4096 * 4096 // 64 + 4 * (4096 * 4096 // 64 // 256) + 2 * 4096 * 4096)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]
