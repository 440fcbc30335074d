"""aethelstream_amd: MI355X-native (gfx950) NF4 streamed-weight path.

Hand-written HIP kernels behind the C ABI of ``include/nf4stream.h``
(libnf4stream.so): NF4 quantize / double-quant / dequant and the
NF4-dequant-fused bf16 MFMA GEMM (forward X.W^T and input-gradient dY.W).
"""
from . import _lib  # noqa: F401
from .nf4 import (  # noqa: F401
    BLOCK_SIZE,
    DQ_GROUP,
    NF4_CODES,
    MalformedIndex,
    Nf4Result,
    Nf4Weight,
    ShardEngineError,
    check_fidelity,
    dequant,
    dequant_batch,
    dequant_nf4_alloc,
    dequant_nf4_into,
    dequantize_nf4,
    dq_encode,
    quantize_nf4,
    quantize_weight,
)

__version__ = "0.1.0"
