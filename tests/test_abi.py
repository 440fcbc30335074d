"""The C-ABI library loads and exports every symbol include/nf4stream.h declares;
argument validation mirrors the reference's error rules.  CPU only: the calls
below are rejected before any kernel launch."""
import ctypes
import os
import re

import pytest

from aethelstream_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nf4stream.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(nf4s_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported():
    lib = _lib.load()
    syms = declared_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(lib, s), f"libnf4stream.so does not export {s}"
    # The ctypes table covers the header exactly.
    assert sorted(_lib.SIGNATURES) == syms


def test_abi_version_and_strerror():
    lib = _lib.load()
    hdr = open(HEADER).read()
    assert lib.nf4s_abi_version() == int(re.search(r"#define NF4S_ABI_VERSION (\d+)", hdr).group(1))
    assert lib.nf4s_strerror(0) == b"ok"
    assert b"nf4_absmax" in lib.nf4s_strerror(_lib.NF4S_ERR_ABSMAX_TOO_SMALL)
    assert b"nf4_packed" in lib.nf4s_strerror(_lib.NF4S_ERR_PACKED_TOO_SMALL)


def _desc(packed_len, absmax_len, bs, dq=False, scale_len=0, group=0):
    # Non-null dummy pointers: validation must reject before dereferencing.
    fake = 0x1000
    return _lib.Nf4sTensor(packed=fake, packed_len=packed_len,
                           absmax=None if dq else fake, absmax_q=fake if dq else None,
                           absmax_scale=fake if dq else None, absmax_len=absmax_len,
                           scale_len=scale_len, block_size=bs, dq_group=group)


def test_malformed_absmax_then_packed():
    # shard_engine/src/nf4.rs:46-57: absmax first, then packed; same text.
    lib = _lib.load()
    d = _desc(packed_len=8, absmax_len=1, bs=8)
    rc = lib.nf4s_dequant_f16(ctypes.byref(d), 16, 0x2000, None)
    assert rc == _lib.NF4S_ERR_ABSMAX_TOO_SMALL
    assert lib.nf4s_last_error_message() == b"absmax too small: 1 < 2"
    d = _desc(packed_len=3, absmax_len=4, bs=2)
    rc = lib.nf4s_dequant_bf16(ctypes.byref(d), 8, 0x2000, None)
    assert rc == _lib.NF4S_ERR_PACKED_TOO_SMALL
    assert lib.nf4s_last_error_message() == b"packed too small: 6 < 8"


def test_invalid_arguments():
    lib = _lib.load()
    assert lib.nf4s_dequant_bf16(None, 8, 0x2000, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    d = _desc(packed_len=4, absmax_len=1, bs=0)
    assert lib.nf4s_dequant_bf16(ctypes.byref(d), 8, 0x2000, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    d = _desc(packed_len=4, absmax_len=1, bs=64, dq=True, scale_len=0, group=256)
    assert lib.nf4s_dequant_bf16(ctypes.byref(d), 8, 0x2000, None) == _lib.NF4S_ERR_ABSMAX_TOO_SMALL
    assert lib.nf4s_quantize(None, 10, 64, None, None, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert lib.nf4s_quantize(0x1000, 10, 0, 0x1000, 0x1000, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert lib.nf4s_dq_encode(0x1000, 10, 0, 0x1000, 0x1000, None) == _lib.NF4S_ERR_INVALID_ARGUMENT


def test_wgrad_argument_rejection():
    """nf4s_gemm_wgrad validates before touching the device."""
    lib = _lib.load()
    f = lib.nf4s_gemm_wgrad
    assert f(None, 0x1000, 64, 64, 64, 0x1000, 0, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(0x1000, 0x1000, 64, 64, 64, None, 0, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(0x1000, 0x1000, 64, 0, 64, 0x1000, 0, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(0x1000, 0x1000, -1, 64, 64, 0x1000, 0, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(0x1000, 0x1000, 64, 12, 64, 0x1000, 0, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert f(0x1000, 0x1000, 64, 64, 20, 0x1000, 0, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert f(0x1008, 0x1000, 64, 64, 64, 0x1000, 0, None) == _lib.NF4S_ERR_MISALIGNED
    assert f(0x1000, 0x1000, 64, 64, 64, 0x1002, 0, None) == _lib.NF4S_ERR_MISALIGNED
    assert f(0x1000, 0x1000, 1 << 20, 1024, 64, 0x1000, 0, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE




def test_dgrad_workspace_size_query():
    """The split-K input-gradient workspace query allocates nothing and needs
    no kernel (256 CUs assumed without a GPU, the MI355X's)."""
    lib = _lib.load()
    f = lib.nf4s_gemm_dgrad_workspace_size
    out = ctypes.c_int64(-1)
    ns = (ctypes.c_int64 * 3)(8192, 1024, 1024)
    assert f(ns, 3, 256, 8192, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(ns, 0, 256, 8192, ctypes.byref(out)) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(ns, 5, 256, 8192, ctypes.byref(out)) == _lib.NF4S_ERR_INVALID_ARGUMENT
    # 70B d_h1 at 256 tokens: 64 tiles -> 4 slices of 256 x 256 fp32 per thread.
    assert f(ns, 3, 256, 8192, ctypes.byref(out)) == 0 and out.value == 64 * 4 * 256 * 256 * 4
    # 8192 tokens: 1024 tiles, whole rounds, no split.
    assert f(ns, 3, 8192, 8192, ctypes.byref(out)) == 0 and out.value == 0
    # n % 64 != 0 is the GEMM's own error; the query reports no split.
    bad = (ctypes.c_int64 * 1)(100)
    assert f(bad, 1, 256, 8192, ctypes.byref(out)) == 0 and out.value == 0

def test_wgrad_grouped_argument_rejection():
    """nf4s_gemm_wgrad_grouped validates every product before any launch."""
    lib = _lib.load()
    f = lib.nf4s_gemm_wgrad_grouped
    P = ctypes.c_void_p
    dys = (P * 5)(*([0x1000] * 5))
    dws = (P * 5)(*([0x1000] * 5))
    ns = (ctypes.c_int64 * 5)(64, 64, 64, 64, 64)
    assert f(dys, ns, dws, 0, 0x1000, 64, 64, 0, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(dys, ns, dws, 5, 0x1000, 64, 64, 0, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(None, ns, dws, 2, 0x1000, 64, 64, 0, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(dys, ns, dws, 2, 0x1000, 64, 20, 0, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    bad_n = (ctypes.c_int64 * 3)(64, 12, 64)
    assert f(dys, bad_n, dws, 3, 0x1000, 64, 64, 0, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    mis = (P * 3)(0x1000, 0x1000, 0x1008)
    assert f(mis, ns, dws, 3, 0x1000, 64, 64, 0, None) == _lib.NF4S_ERR_MISALIGNED
    nul = (P * 2)(0x1000, None)
    assert f(dys, ns, nul, 2, 0x1000, 64, 64, 0, None) == _lib.NF4S_ERR_INVALID_ARGUMENT

def test_fwd_workspace_size_query():
    """The split-K workspace query allocates nothing and needs no kernel.  On a
    host without a GPU the CU count reads as 256, the MI355X's."""
    lib = _lib.load()
    f = lib.nf4s_gemm_fwd_workspace_size
    out = ctypes.c_int64(-1)
    ns = (ctypes.c_int64 * 4)(1024, 1024, 1024, 1024)
    assert f(ns, 1, 8192, 8192, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(ns, 0, 8192, 8192, ctypes.byref(out)) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert f(ns, 5, 8192, 8192, ctypes.byref(out)) == _lib.NF4S_ERR_INVALID_ARGUMENT
    # k % 64 != 0 is the GEMM's own error; the query just reports no split.
    assert f(ns, 1, 8192, 96, ctypes.byref(out)) == 0 and out.value == 0
    if torch_has_gpu():
        return
    # 8192 x 1024 outputs = 128 tiles of 512 x 128: half a round of 256 CUs,
    # so two K slices of 256 x 256 fp32 partials (256 KiB) per tile.
    assert f(ns, 1, 8192, 8192, ctypes.byref(out)) == 0
    assert out.value == 128 * 2 * 256 * 1024
    # 8192 x 8192 = 1024 tiles: whole rounds, no split.
    ns[0] = 8192
    assert f(ns, 1, 8192, 8192, ctypes.byref(out)) == 0 and out.value == 0
    # A negative workspace size is rejected before any launch.
    assert lib.nf4s_gemm_fwd_grouped_ws(0x1000, None, ns, None, 1, 64, 64, None, -1,
                                        None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert lib.nf4s_gemm_fwd_grouped_ws(0x1000, None, ns, None, 1, 64, 64, 0x1008, 64,
                                        None) == _lib.NF4S_ERR_MISALIGNED
    # The no-allocation entry point checks count and sizes before it looks up
    # (and so loads) its static scratch: no GPU call is reached here.
    na = lib.nf4s_gemm_fwd_grouped_noalloc
    assert na(0x1000, None, ns, None, 0, 64, 64, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert na(0x1000, None, ns, None, 5, 64, 64, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert na(0x1000, None, None, None, 1, 64, 64, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert b"count must be 1..4" in lib.nf4s_last_error_message()


def torch_has_gpu():
    import torch
    return torch.cuda.is_available()


def test_python_mirror_raises_malformed_index():
    import torch
    from aethelstream_amd import nf4
    with pytest.raises(ValueError):
        nf4.dequant_nf4_into(torch.zeros(4, dtype=torch.uint8), torch.ones(1),
                             torch.zeros(8, dtype=torch.float16), 64)


def test_requantize_argument_rejection():
    # Rejected before any launch: wrong block size, non-power-of-two group.
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    assert lib.nf4s_quantize_dq(p, 128, 32, 256, p, p, p, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert lib.nf4s_quantize_dq(p, 128, 64, 3, p, p, p, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert lib.nf4s_quantize_dq_bf16(p, 128, 64, 16384, p, p, p, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert lib.nf4s_quantize_bf16(p, 128, 32, p, p, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert lib.nf4s_quantize_dq(p, -1, 64, 256, p, p, p, None) == _lib.NF4S_ERR_INVALID_ARGUMENT


def test_wgrad_rejects_offsets_past_2gib_in_the_last_step():
    # m = 1 with n = 2^25: dy itself is 64 MiB, but the last 32-token step
    # addresses rows up to 31, 2 GiB into dy, where 32-bit lane offsets wrap.
    lib = _lib.load()
    rc = lib.nf4s_gemm_wgrad(0x1000, 0x2000, 1, 1 << 25, 8, 0x3000, 0, None)
    assert rc == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert b"m rounded up to 32" in lib.nf4s_last_error_message()


def test_huge_sizes_are_rejected_not_wrapped():
    """Caller sizes whose products or tile counts would overflow are refused
    before any device work (checked division instead of wrapping products)."""
    lib = _lib.load()
    d = _desc(packed_len=1 << 62, absmax_len=1 << 56, bs=64)
    x, out = 0x1000, 0x2000
    f = lib.nf4s_gemm_fwd
    assert f(x, ctypes.byref(d), 64, 1 << 40, 64, out, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert b"beyond 2^39" in lib.nf4s_last_error_message()
    assert f(x, ctypes.byref(d), 1 << 62, 64, 64, out, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert lib.nf4s_gemm_dgrad(x, ctypes.byref(d), 64, 1 << 35, 1 << 35, out, None) == \
        _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert b"overflows 64 bits" in lib.nf4s_last_error_message()
    w = lib.nf4s_gemm_wgrad
    assert w(x, x, 1 << 62, 64, 8, out, 0, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert w(x, x, 64, 64, 1 << 45, out, 0, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert w(x, x, 0, 1 << 38, 1 << 38, out, 0, None) == _lib.NF4S_ERR_UNSUPPORTED_SHAPE
    assert b"overflows 64 bits" in lib.nf4s_last_error_message()
    # Descriptor checks at element counts near 2^63 (ceil divisions, not sums).
    big = (1 << 63) - 1
    d = _desc(packed_len=1 << 62, absmax_len=1 << 56, bs=64)
    assert lib.nf4s_dequant_bf16(ctypes.byref(d), big, out, None) == \
        _lib.NF4S_ERR_ABSMAX_TOO_SMALL
    d = _desc(packed_len=(1 << 62) - 1, absmax_len=1 << 62, bs=64)
    assert lib.nf4s_dequant_bf16(ctypes.byref(d), big, out, None) == \
        _lib.NF4S_ERR_PACKED_TOO_SMALL
    size = ctypes.c_int64(-1)
    ns = (ctypes.c_int64 * 1)(1 << 45)
    assert lib.nf4s_gemm_dgrad_workspace_size(ns, 1, 256, 8192, ctypes.byref(size)) == 0
    assert size.value == 0
    assert lib.nf4s_gemm_fwd_workspace_size(ns, 1, 1 << 62, 8192, ctypes.byref(size)) == 0
    assert size.value == 0
