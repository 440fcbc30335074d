"""Shard loader and on-disk format on the CPU: index parsing, load_layer, and
the reference's error rules (shard_engine/src/loader.rs:93-151,
error.rs:5-28, ffi.rs:33-43).  No kernel runs: every case below is decided
before any device work."""
import ctypes
import json
import struct

import pytest

from aethelstream_amd import _lib, shard
from shard_fixture import build_cpu_shards, write_index

GOLDEN_LEGACY = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                            "legacy_shard_index.json")


@pytest.fixture()
def shard_dir(tmp_path):
    index, registry, tensors = build_cpu_shards(tmp_path / "m")
    return tmp_path / "m", index, registry, tensors


def _load_f16_status(loader, name):
    """Calls load_param_f16 with a dummy device pointer: the checks must fail
    before the pointer is used."""
    return _lib.load().nf4s_loader_load_param_f16(loader._h, name.encode(), 0x1000, 1 << 20, None)


def test_param_info_and_pyo3_mirror(shard_dir):
    d, index, _, _ = shard_dir
    L = shard.PyShardLoader(str(d))
    assert L.param_shape("model.layers.0.q") == [64, 64]
    assert L.param_precision("model.layers.0.q") == "nf4"
    assert L.param_precision("model.layers.1.norm") == "fp16"
    info = shard.ShardLoader(d).param_info("model.layers.0.q")
    assert info.out_elems == 2 * index["model.layers.0.q"]["byte_length"]   # nf4.rs:103
    assert info.absmax_len == 64 * 64 // 64
    with pytest.raises(KeyError):
        L.param_shape("nope")


def test_load_layer_returns_safetensors_bytes(shard_dir):
    # shard_engine/tests/test_rust_roundtrip.py:38-47
    d, _, registry, _ = shard_dir
    L = shard.PyShardLoader(str(d))
    raw = L.load_layer(0)
    assert raw == (d / registry["0"]).read_bytes()
    header_len = struct.unpack("<Q", raw[:8])[0]
    assert header_len > 0 and len(raw) >= 8 + header_len
    buf = shard.ShardLoader(d).load_layer(1)
    assert buf.layer_index == 1 and buf.file_path.endswith(registry["1"])


def test_missing_layer_and_param(shard_dir):
    # test_rust_roundtrip.py:50-55 (ValueError or IOError); ffi.rs:33-43.
    d, _, _, _ = shard_dir
    L = shard.PyShardLoader(str(d))
    with pytest.raises((ValueError, IOError)):
        L.load_layer(9999)
    with pytest.raises(KeyError, match="not found in shard index"):
        L.load_param("model.layers.7.q")
    with pytest.raises(shard.LayerNotFound, match="layer index 9999 not found in layer registry"):
        shard.ShardLoader(d).load_layer(9999)


def test_open_errors(tmp_path):
    with pytest.raises(IOError, match="I/O error"):
        shard.PyShardLoader(str(tmp_path / "does_not_exist"))
    (tmp_path / "bad").mkdir()
    (tmp_path / "bad" / "shard_index.json").write_text("{ not json")
    (tmp_path / "bad" / "layer_registry.json").write_text("{}")
    with pytest.raises(shard.ShardJsonError, match="JSON parse error"):
        shard.ShardLoader(tmp_path / "bad")


def test_legacy_fixture_schema_is_rejected_like_index_store(tmp_path):
    # shard_engine/tests/fixtures/shard_index.json uses the legacy
    # {"file", "tensors"} schema that IndexStore cannot deserialize
    # (index.rs:7-34): a JSON error, not a crash.
    d = tmp_path / "legacy"
    d.mkdir()
    (d / "shard_index.json").write_text(open(GOLDEN_LEGACY).read())
    (d / "layer_registry.json").write_text("{}")
    with pytest.raises(shard.ShardJsonError, match="missing field `file_path`"):
        shard.ShardLoader(d)


def test_legacy_fixture_size_relations():
    # packed = n/2 bytes and absmax = 4*ceil(n/64) bytes: 8 packed bytes per
    # absmax byte when n % 64 == 0 (its NF4 entries).
    legacy = json.load(open(GOLDEN_LEGACY))
    nf4 = [v["tensors"] for v in legacy.values() if "packed" in v["tensors"]]
    assert len(nf4) == 43
    for t in nf4:
        pk = t["packed"]["end"] - t["packed"]["start"]
        am = t["absmax"]["end"] - t["absmax"]["start"]
        n = 2 * pk
        assert am == 4 * ((n + 63) // 64)


@pytest.mark.parametrize("mutation,match", [
    (lambda e: e.pop("nf4_absmax_offset"), "missing nf4_absmax_offset"),
    (lambda e: e.pop("nf4_absmax_length"), "missing nf4_absmax_length"),
    (lambda e: e.pop("nf4_block_size"), "missing nf4_block_size"),
    (lambda e: e.update(byte_length=10 ** 9), "packed data out of bounds"),
    (lambda e: e.update(nf4_absmax_length=10 ** 9), "absmax data out of bounds"),
    (lambda e: e.update(nf4_absmax_offset=e["nf4_absmax_offset"] + 2,
                        nf4_absmax_length=e["nf4_absmax_length"] - 4),
     "absmax offset .* is not 4-byte aligned"),
])
def test_malformed_nf4_entries(shard_dir, mutation, match):
    d, index, registry, _ = shard_dir
    e = dict(index["model.layers.0.q"])
    mutation(e)
    index = dict(index)
    index["model.layers.0.q"] = e
    write_index(d, index, registry)
    L = shard.ShardLoader(d)
    rc = _load_f16_status(L, "model.layers.0.q")
    assert rc == _lib.NF4S_ERR_MALFORMED_INDEX
    msg = _lib.load().nf4s_last_error_message().decode()
    assert msg.startswith("malformed index entry 'model.layers.0.q': ")
    import re
    assert re.search(match, msg), msg
