"""The 13 gguf-rs unit tests (crates/gguf-rs/src/lib.rs:334-573) ported to
the C++ reader of libstyx_hip.so (styx_gguf_inspect; no GPU needed), plus a
writer/reader round trip of styx_amd.gguf_io."""
from __future__ import annotations

import ctypes as C
import json
import struct

import numpy as np
import pytest


def inspect(path):
    from styx_amd import _lib
    lib = _lib.load()
    buf = C.create_string_buffer(1 << 20)
    rc = lib.styx_gguf_inspect(str(path).encode(), buf, len(buf))
    if rc != 0:
        raise ValueError(lib.styx_last_error().decode())
    return json.loads(buf.value.decode())


def u32(v): return struct.pack("<I", v)
def u64(v): return struct.pack("<Q", v)


def gstr(s: bytes): return u64(len(s)) + s


def header(version=3, tensors=0, kvs=0):
    return u32(0x46554747) + u32(version) + u64(tensors) + u64(kvs)


def open_bytes(tmp_path, tag, data: bytes):
    p = tmp_path / f"{tag}.gguf"
    p.write_bytes(data)
    return inspect(p)


def assert_invalid(tmp_path, tag, data, needle):
    with pytest.raises(ValueError) as e:
        open_bytes(tmp_path, tag, data)
    assert needle in str(e.value), (tag, str(e.value))


def test_gguf_parsing(tmp_path):
    """lib.rs:341-425: v3 image, 3 kvs, an f32 [4,2] and a q4_K [256,3] tensor."""
    b = header(3, 2, 3)
    b += gstr(b"general.name") + u32(8) + gstr(b"test")
    b += gstr(b"general.alignment") + u32(4) + u32(32)
    b += gstr(b"tokenizer.chat_template") + u32(8) + gstr(b"{{chat}}")
    b += gstr(b"t0") + u32(2) + u64(4) + u64(2) + u32(0) + u64(0)
    b += gstr(b"t1") + u32(2) + u64(256) + u64(3) + u32(12) + u64(16)
    g = open_bytes(tmp_path, "pos", b)
    assert g["version"] == 3 and len(g["tensors"]) == 2
    t0, t1 = g["tensors"]
    assert (t0["name"], t0["dims"], t0["type"], t0["offset"], t0["size_bytes"]) == ("t0", [4, 2], 0, 0, 32)
    assert (t1["name"], t1["dims"], t1["type"], t1["offset"], t1["size_bytes"]) == ("t1", [256, 3], 12, 16, 432)
    assert g["data_start"] == 256  # 228 aligned up to 32


def test_empty_file_is_rejected(tmp_path):
    with pytest.raises(ValueError):
        open_bytes(tmp_path, "empty", b"")


def test_bad_magic(tmp_path):
    b = bytearray(header())
    b[0] = ord("X")
    assert_invalid(tmp_path, "magic", bytes(b), "magic")


def test_unsupported_version(tmp_path):
    assert_invalid(tmp_path, "v1", header(1), "version")
    assert_invalid(tmp_path, "v99", header(99), "version")


def test_version_2_accepted(tmp_path):
    g = open_bytes(tmp_path, "v2", header(2))
    assert g["version"] == 2 and g["tensors"] == []


def test_truncated_metadata(tmp_path):
    with pytest.raises(ValueError):
        open_bytes(tmp_path, "trunc_meta", header(3, 0, 1))


def test_string_too_long(tmp_path):
    assert_invalid(tmp_path, "longstr", header(3, 0, 1) + u64(2**64 - 1), "String too long")


def test_invalid_utf8_string(tmp_path):
    assert_invalid(tmp_path, "utf8", header(3, 0, 1) + u64(4) + bytes([0xFF, 0xFE, 0xFD, 0xFC]), "UTF-8")


def test_unknown_metadata_value_type(tmp_path):
    assert_invalid(tmp_path, "valtype", header(3, 0, 1) + gstr(b"k") + u32(99), "value type")


def test_array_too_long(tmp_path):
    b = header(3, 0, 1) + gstr(b"k") + u32(9) + u32(4) + u64(2**64 - 1)
    assert_invalid(tmp_path, "longarr", b, "Array too long")


def test_unknown_tensor_ggml_type(tmp_path):
    b = header(3, 1, 0) + gstr(b"t") + u32(1) + u64(32) + u32(255) + u64(0)
    assert_invalid(tmp_path, "ggmltype", b, "type")


def test_dim_not_multiple_of_block_size(tmp_path):
    b = header(3, 1, 0) + gstr(b"t") + u32(1) + u64(100) + u32(12) + u64(0)
    with pytest.raises(ValueError):
        open_bytes(tmp_path, "blocksize", b)


def test_truncated_tensor_info(tmp_path):
    with pytest.raises(ValueError):
        open_bytes(tmp_path, "trunc_tensor", header(3, 1, 0) + gstr(b"t") + u32(2))


def test_writer_roundtrip(tmp_path):
    """styx_amd.gguf_io.write -> C++ reader: names, dims, types, offsets, sizes."""
    from styx_amd.gguf_io import write
    rng = np.random.default_rng(0)
    tens = [("a.weight", 0, [8, 3], rng.standard_normal(24).astype(np.float32).view(np.uint8)),
            ("b.weight", 8, [64, 5], rng.integers(0, 256, 5 * 2 * 34, dtype=np.uint8)),
            ("c.weight", 14, [256, 2, 3], rng.integers(0, 256, 6 * 210, dtype=np.uint8))]
    p = tmp_path / "w.gguf"
    write(p, {"general.architecture": "qwen3moe", "x.count": 7, "x.eps": 1e-6}, tens)
    g = inspect(p)
    assert g["data_start"] % 32 == 0
    raw = p.read_bytes()
    for (name, typ, dims, data), t in zip(tens, g["tensors"]):
        assert (t["name"], t["dims"], t["type"], t["size_bytes"]) == (name, dims, typ, len(data))
        start = g["data_start"] + t["offset"]
        assert raw[start:start + len(data)] == data.tobytes()
    assert set(g["metadata"]) == {"general.architecture", "x.count", "x.eps"}
