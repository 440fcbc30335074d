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


def _load_f16_status(loader, name, staging_bytes=1 << 20):
    """Calls load_param_f16 with dummy device pointers: the checks must fail
    before either pointer is used."""
    return _lib.load().nf4s_loader_load_param_f16(loader._h, name.encode(), 0x1000, 1 << 20,
                                                  0x2000, staging_bytes, None)


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


@pytest.mark.parametrize("field,value", [
    ("byte_offset", -8), ("byte_length", -1), ("nf4_absmax_offset", -8),
    ("nf4_absmax_length", -8), ("nf4_block_size", -64),
])
def test_negative_sizes_are_json_errors(shard_dir, field, value):
    # usize / Option<usize> fields (index.rs:7-34): serde rejects a negative
    # integer when IndexStore::load parses the index, before any access.
    d, index, registry, _ = shard_dir
    e = dict(index["model.layers.0.q"])
    e[field] = value
    index = dict(index)
    index["model.layers.0.q"] = e
    write_index(d, index, registry)
    with pytest.raises(shard.ShardJsonError, match=f"invalid value: integer `{value}`"):
        shard.ShardLoader(d)


def test_negative_offset_with_matching_length_does_not_wrap(shard_dir):
    # offset -8 + length 8 sums to 0 in unsigned arithmetic; the entry must
    # still be rejected (here already at parse time).
    d, index, registry, _ = shard_dir
    e = dict(index["model.layers.0.q"])
    e.update(nf4_absmax_offset=-8, nf4_absmax_length=8)
    index = dict(index)
    index["model.layers.0.q"] = e
    write_index(d, index, registry)
    with pytest.raises(shard.ShardJsonError):
        shard.ShardLoader(d)


def test_huge_offset_is_out_of_bounds(shard_dir):
    # An offset near 2^64 - 1 as unsigned must not wrap the bounds check.
    d, index, registry, _ = shard_dir
    e = dict(index["model.layers.0.q"])
    e.update(nf4_absmax_offset=(1 << 63) - 4, nf4_absmax_length=8)
    index = dict(index)
    index["model.layers.0.q"] = e
    write_index(d, index, registry)
    L = shard.ShardLoader(d)
    assert _load_f16_status(L, "model.layers.0.q") == _lib.NF4S_ERR_MALFORMED_INDEX
    assert "absmax data out of bounds" in _lib.load().nf4s_last_error_message().decode()


def test_staging_size_and_too_small_staging(shard_dir):
    d, index, _, _ = shard_dir
    L = shard.ShardLoader(d)
    n = ctypes.c_int64()
    _lib.check(_lib.load().nf4s_loader_staging_size(L._h, b"model.layers.0.q", ctypes.byref(n)))
    e = index["model.layers.0.q"]
    rnd = lambda x: (x + 255) // 256 * 256
    assert n.value == rnd(e["byte_length"]) + rnd(e["nf4_absmax_length"])
    _lib.check(_lib.load().nf4s_loader_staging_size(L._h, b"model.layers.0.norm",
                                                   ctypes.byref(n)))
    assert n.value == 0
    rc = _load_f16_status(L, "model.layers.0.q", staging_bytes=255)
    assert rc == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert "staging holds 255 bytes" in _lib.load().nf4s_last_error_message().decode()


def test_nf4_destination_capacity_checked(shard_dir):
    d, index, _, _ = shard_dir
    L = shard.ShardLoader(d)
    e = index["model.layers.0.q"]
    rc = _lib.load().nf4s_loader_load_param_nf4(L._h, b"model.layers.0.q", 0x1000,
                                                e["byte_length"] - 1, 0x2000, 1 << 20, None, 0,
                                                None)
    assert rc == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert "destination too small" in _lib.load().nf4s_last_error_message().decode()


def test_last_error_message_cleared_by_a_successful_call(shard_dir):
    d, _, _, _ = shard_dir
    lib = _lib.load()
    L = shard.ShardLoader(d)
    info = _lib.Nf4sParamInfo()
    assert lib.nf4s_loader_param_info(L._h, b"nope", ctypes.byref(info)) == \
        _lib.NF4S_ERR_PARAM_NOT_FOUND
    assert b"not found" in lib.nf4s_last_error_message()
    _lib.check(lib.nf4s_loader_param_info(L._h, b"model.layers.0.q", ctypes.byref(info)))
    assert lib.nf4s_last_error_message() == b""
    # The same for a call outside the loader (host-only validation path).
    assert lib.nf4s_gemm_fwd_workspace_size(None, 1, 1, 64, None) == _lib.NF4S_ERR_INVALID_ARGUMENT
    assert lib.nf4s_last_error_message() != b""
    ns = (ctypes.c_int64 * 1)(128)
    nb = ctypes.c_int64()
    _lib.check(lib.nf4s_gemm_fwd_workspace_size(ns, 1, 0, 64, ctypes.byref(nb)))
    assert lib.nf4s_last_error_message() == b""


@pytest.mark.parametrize("double_quant", [False, True])
def test_pack_layer_blob_bytes_and_descriptors(tmp_path, double_quant):
    # The blob a FlowCast pinned slot holds for a layer: each parameter's raw
    # payload parts at 256-byte boundaries, byte-equal to the shard's
    # tensors; descriptors rebased on any copy of the blob.
    d = tmp_path / "m"
    index, _, tensors = build_cpu_shards(d, n_layers=2, dim=128, double_quant=double_quant)
    L = shard.ShardLoader(d)
    names = ["model.layers.0.q", "model.layers.1.q"]
    ents, nb = L.pack_layer(names)
    assert nb % 256 == 0 and ents[0].packed_off == 0
    buf = (ctypes.c_uint8 * nb)()
    base = ctypes.addressof(buf)
    ents2, nb2 = L.pack_layer(names, base, nb)
    assert nb2 == nb
    raw = bytes(buf)
    from safetensors.numpy import load_file
    from aethelstream_amd import stream as st
    lay = st.BlobLayout(names, ents2, [[128, 128]] * 2, nb)
    for e, v, name, l in zip(ents2, lay.views(base), names, range(2)):
        for off in (e.packed_off, e.absmax_off, e.scale_off):
            assert off % 256 == 0
        f = load_file(str(d / f"layer_{l}.safetensors"))
        assert raw[e.packed_off:e.packed_off + e.packed_len] == f[f"{name}.__packed__"].tobytes()
        if double_quant:
            assert e.dq_group == 256 and e.absmax_len == 128 * 128 // 64
            assert raw[e.absmax_off:e.absmax_off + e.absmax_len] == \
                f[f"{name}.__absmax_q__"].tobytes()
            assert raw[e.scale_off:e.scale_off + 4 * e.scale_len] == \
                f[f"{name}.__absmax_scale__"].tobytes()
            assert v.desc.absmax is None and v.desc.absmax_q == base + e.absmax_off
            assert v.desc.absmax_scale == base + e.scale_off and v.desc.scale_len == 1
        else:
            assert e.dq_group == 0 and e.scale_len == 0
            assert raw[e.absmax_off:e.absmax_off + 4 * e.absmax_len] == \
                f[f"{name}.__absmax__"].tobytes()
            assert v.desc.absmax == base + e.absmax_off and v.desc.absmax_q is None
        assert v.desc.packed == base + e.packed_off and v.desc.packed_len == e.packed_len
    with pytest.raises(_lib.Nf4sError, match="blob holds 256 bytes"):
        L.pack_layer(names, base, 256)
    with pytest.raises(shard.MalformedIndexEntry, match="not nf4"):
        L.pack_layer(["model.layers.0.norm"])


@pytest.mark.parametrize("update,what", [
    ({"shape": [1 << 40, 1 << 40]}, "shape element count overflows 64 bits"),
    ({"byte_length": (1 << 63) - 1}, "byte_length"),
])
def test_param_info_sizes_do_not_overflow(shard_dir, update, what):
    # Products and doublings of index sizes are checked, not wrapped (found
    # by fuzzing the loader's host code under UBSan).
    d, index, registry, _ = shard_dir
    e = dict(index["model.layers.0.q"])
    e.update(update)
    index = dict(index)
    index["model.layers.0.q"] = e
    write_index(d, index, registry)
    L = shard.ShardLoader(d)
    info = _lib.Nf4sParamInfo()
    rc = _lib.load().nf4s_loader_param_info(L._h, b"model.layers.0.q", ctypes.byref(info))
    assert rc == _lib.NF4S_ERR_MALFORMED_INDEX
    assert what in _lib.load().nf4s_last_error_message().decode()


def test_staging_size_checks_the_entry_first(shard_dir):
    # Lengths near 2^63 used to be rounded and summed unchecked; the size
    # query now rejects an entry out of bounds of its file, as the load does.
    d, index, registry, _ = shard_dir
    e = dict(index["model.layers.0.q"])
    e.update(nf4_absmax_length=(1 << 63) - 1)
    index = dict(index)
    index["model.layers.0.q"] = e
    write_index(d, index, registry)
    L = shard.ShardLoader(d)
    n = ctypes.c_int64(7)
    rc = _lib.load().nf4s_loader_staging_size(L._h, b"model.layers.0.q", ctypes.byref(n))
    assert rc == _lib.NF4S_ERR_MALFORMED_INDEX and n.value == 0
    assert "absmax data out of bounds" in _lib.load().nf4s_last_error_message().decode()
