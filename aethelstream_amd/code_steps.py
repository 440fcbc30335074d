"""Step thresholds of the NF4 code rule, for the block-64 quantize kernels.

quantizer.py:40-41 (shard_engine/python/pipeline/quantizer.py) gives element
n the first index of the smallest fp32 distance |n - code_i|.  That rule is
monotone in n, so it equals a step function: code(n) = #{k : n >= S_k} with
S_k the smallest fp32 n whose code is >= k.  ``steps()`` finds the 15 S_k by
bisection over the fp32 values in [-1, 1], evaluating the rule in fp32 with
numpy; ``c_table()`` prints them as the kStepBits table of nf4_codec.hip.

    python -m aethelstream_amd.code_steps
"""
from __future__ import annotations

import numpy as np

# shard_engine/src/nf4.rs:6-23, as fp32 bit patterns.
CODE_BITS = [
    0xbf800000, 0xbf3239b1, 0xbf066b30, 0xbeca32a0,
    0xbe91a24d, 0xbe3d353f, 0xbdba7872, 0x00000000,
    0x3da2faff, 0x3e24cae3, 0x3e7c04dd, 0x3ead033a,
    0x3ee1a4b8, 0x3f1007ab, 0x3f3913b3, 0x3f800000,
]
_ONE = 0x3f800000


def _code(n: np.float32) -> int:
    codes = np.array(CODE_BITS, np.uint32).view(np.float32)
    d = np.abs(np.float32(n) - codes)        # fp32 subtraction, as torch does
    return int(np.argmin(d))                 # first minimum wins


def _value(t: int) -> np.float32:
    """The t-th fp32 value of [-1, 1] in ascending order (-0 skipped)."""
    b = (0x80000000 | (_ONE - t)) if t < _ONE else t - _ONE
    return np.array([b], np.uint32).view(np.float32)[0]


def steps() -> list[int]:
    """Bit patterns of S_1 .. S_15."""
    out = []
    for k in range(1, 16):
        lo, hi = 0, 2 * _ONE
        while lo < hi:
            mid = (lo + hi) // 2
            if _code(_value(mid)) >= k:
                hi = mid
            else:
                lo = mid + 1
        out.append(int(np.array([_value(lo)], np.float32).view(np.uint32)[0]))
    return out


def c_table() -> str:
    b = [f"0x{s:08x}u" for s in steps()]
    rows = [", ".join(b[i:i + 5]) + "," for i in range(0, 15, 5)]
    return "__constant__ uint32_t kStepBits[15] = {\n" + "\n".join(
        "    " + r for r in rows) + "\n};"


if __name__ == "__main__":
    print(c_table())
