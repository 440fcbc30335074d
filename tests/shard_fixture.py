"""Builds small shard directories on the CPU (oracle quantizer + safetensors)
for the loader tests.  Test infrastructure only."""
import json
from pathlib import Path

import numpy as np

import oracle
from aethelstream_amd.shard import read_safetensors_offsets


def build_cpu_shards(root: Path, n_layers: int = 2, dim: int = 64, double_quant: bool = False):
    """Layer l holds an NF4 matrix `model.layers.l.q` [dim, dim] and an fp16
    vector `model.layers.l.norm` [dim]; returns (index, registry, tensors).
    With double_quant the matrix's absmax is stored as uint8 codes plus fp32
    scales (groups of 256 blocks), the index's double-quant fields."""
    from safetensors.numpy import save_file
    root.mkdir(parents=True, exist_ok=True)
    index, registry, tensors = {}, {}, {}
    for l in range(n_layers):
        w = oracle.gen_normal(100 + l, dim * dim, 0.02).reshape(dim, dim)
        norm = oracle.gen_normal(200 + l, dim, 1.0).astype(np.float16)
        packed, absmax = oracle.quantize_nf4(w)
        qn, nn = f"model.layers.{l}.q", f"model.layers.{l}.norm"
        fname = f"layer_{l}.safetensors"
        parts = {f"{qn}.__packed__": packed, f"{qn}.__shape__": np.array([dim, dim], np.int32),
                 nn: norm}
        if double_quant:
            q, sc = oracle.dq_encode(absmax, 256)
            parts[f"{qn}.__absmax_q__"] = q
            parts[f"{qn}.__absmax_scale__"] = sc
        else:
            parts[f"{qn}.__absmax__"] = absmax
        save_file(parts, str(root / fname))
        offs = read_safetensors_offsets(root / fname)
        ps, pe = offs[f"{qn}.__packed__"]
        index[qn] = {"file_path": fname, "byte_offset": ps, "byte_length": pe - ps,
                     "shape": [dim, dim], "dtype": "U8", "precision": "nf4",
                     "nf4_block_size": 64}
        if double_quant:
            qs, qe = offs[f"{qn}.__absmax_q__"]
            ss, se = offs[f"{qn}.__absmax_scale__"]
            index[qn].update(nf4_absmax_q_offset=qs, nf4_absmax_q_length=qe - qs,
                             nf4_absmax_scale_offset=ss, nf4_absmax_scale_length=se - ss,
                             nf4_dq_group=256)
        else:
            as_, ae = offs[f"{qn}.__absmax__"]
            index[qn].update(nf4_absmax_offset=as_, nf4_absmax_length=ae - as_)
        s, e = offs[nn]
        index[nn] = {"file_path": fname, "byte_offset": s, "byte_length": e - s,
                     "shape": [dim], "dtype": "F16", "precision": "fp16"}
        registry[str(l)] = fname
        tensors[qn] = (w, packed, absmax)
        tensors[nn] = norm
    write_index(root, index, registry)
    return index, registry, tensors


def write_index(root: Path, index: dict, registry: dict) -> None:
    with open(root / "shard_index.json", "w") as f:
        json.dump(index, f)
    with open(root / "layer_registry.json", "w") as f:
        json.dump(registry, f)
