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


# ------------------------------------------- model-file checks (no GPU) ----

def tiny_qwen3moe(overrides=None, drop=()):
    """A 1-layer qwen3moe GGUF's tensor list (q8_0 matrices, f32 norms and
    router) with the dims its hparams imply; overrides maps a name to
    (type, dims) to plant a mistake."""
    hp = dict(n_layers=1, n_embd=256, n_heads=4, n_kv_heads=2, head_dim=64, n_expert=16,
              n_expert_used=2, n_ff_exp=64, n_vocab=64, rms_eps=1e-6, rope_base=1e6)
    H, qd, kvd, E, F, V = 256, 256, 128, 16, 64, 64
    spec = {"token_embd.weight": (8, [H, V]), "output.weight": (8, [H, V]),
            "output_norm.weight": (0, [H])}
    p = "blk.0."
    spec.update({p + "attn_norm.weight": (0, [H]), p + "attn_q_norm.weight": (0, [64]),
                 p + "attn_k_norm.weight": (0, [64]), p + "ffn_norm.weight": (0, [H]),
                 p + "attn_q.weight": (8, [H, qd]), p + "attn_k.weight": (8, [H, kvd]),
                 p + "attn_v.weight": (8, [H, kvd]), p + "attn_output.weight": (8, [qd, H]),
                 p + "ffn_gate_inp.weight": (0, [H, E]),
                 p + "ffn_gate_exps.weight": (8, [H, F, E]), p + "ffn_up_exps.weight": (8, [H, F, E]),
                 p + "ffn_down_exps.weight": (8, [F, H, E])})
    spec.update(overrides or {})
    tens = []
    for name, (typ, dims) in spec.items():
        if name in drop:
            continue
        n = int(np.prod(dims))
        nbytes = n * 4 if typ == 0 else n * 2 if typ == 1 else n // 32 * 34
        tens.append((name, typ, dims, np.zeros(nbytes, np.uint8)))
    return hp, tens


def check_file(path):
    from styx_amd import _lib
    lib = _lib.load()
    hp = _lib.MoeHparams()
    rc = lib.styx_moe_check_file(str(path).encode(), C.byref(hp))
    if rc != 0:
        raise ValueError(lib.styx_last_error().decode())
    return hp


def write_model(tmp_path, tag, hp, tens):
    from styx_amd.gguf_io import model_metadata, write
    p = tmp_path / f"{tag}.gguf"
    write(p, model_metadata(hp), tens)
    return p


def test_model_file_accepted(tmp_path):
    hp, tens = tiny_qwen3moe()
    got = check_file(write_model(tmp_path, "ok", hp, tens))
    assert (got.n_layers, got.n_embd, got.n_expert, got.n_vocab) == (1, 256, 16, 64)
    assert got.slab_bytes == 3 * 64 * 256 // 32 * 34


@pytest.mark.parametrize("name,typ,dims,needle", [
    ("blk.0.ffn_gate_inp.weight", 0, [256, 8], "dims"),        # short router
    ("output.weight", 8, [256, 32], "dims"),                   # short LM head
    ("output_norm.weight", 0, [128], "dims"),
    ("blk.0.attn_q_norm.weight", 0, [32], "dims"),
    ("blk.0.ffn_down_exps.weight", 8, [64, 256, 8], "dims"),
    ("blk.0.ffn_norm.weight", 8, [256], "expected f32"),
    ("blk.0.attn_q.weight", 0, [256, 256], "matrix type"),
    ("blk.0.ffn_gate_inp.bias", 0, [8], "dims"),               # optional tensor, wrong size
])
def test_model_file_shape_mismatch_rejected(tmp_path, name, typ, dims, needle):
    hp, tens = tiny_qwen3moe({name: (typ, dims)})
    with pytest.raises(ValueError) as e:
        check_file(write_model(tmp_path, "bad", hp, tens))
    assert needle in str(e.value) and name in str(e.value)


@pytest.mark.parametrize("typ", [0, 1])
def test_float_token_embd_accepted(tmp_path, typ):
    """MoeModel::load admits f32 and f16 embedding tables (moe.rs:1107-1112)
    as well as the quant types."""
    hp, tens = tiny_qwen3moe({"token_embd.weight": (typ, [256, 64])})
    got = check_file(write_model(tmp_path, f"embd{typ}", hp, tens))
    assert got.n_vocab == 64


def test_float_type_refused_for_other_matrices(tmp_path):
    """f32/f16 are for the embedding table only: an f16 attention matrix is
    refused before anything is uploaded, with the type named."""
    hp, tens = tiny_qwen3moe({"blk.0.attn_q.weight": (1, [256, 256])})
    with pytest.raises(ValueError, match="attn_q.weight: matrix type must be q8_0/q4_K/q5_K/q6_K"):
        check_file(write_model(tmp_path, "f16q", hp, tens))


def test_model_file_missing_tensor_rejected(tmp_path):
    hp, tens = tiny_qwen3moe(drop=("blk.0.ffn_gate_inp.weight",))
    with pytest.raises(ValueError, match="missing tensor blk.0.ffn_gate_inp.weight"):
        check_file(write_model(tmp_path, "miss", hp, tens))


def test_model_file_offset_near_2_64_rejected(tmp_path):
    """An offset that makes offset + size + data_start wrap past 2^64 is
    rejected, not taken as inside the file."""
    hp, tens = tiny_qwen3moe()
    p = write_model(tmp_path, "wrap", hp, tens)
    raw = bytearray(p.read_bytes())
    name = b"blk.0.ffn_gate_inp.weight"
    at = raw.index(struct.pack("<Q", len(name)) + name) + 8 + len(name)
    nd = struct.unpack_from("<I", raw, at)[0]
    off_at = at + 4 + 8 * nd + 4
    struct.pack_into("<Q", raw, off_at, (1 << 64) - 64)
    p.write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="past end of file"):
        check_file(p)


def test_dims_product_overflow_rejected(tmp_path):
    """Dims whose product passes 2^64 are rejected (the reference's u64
    product would wrap in a release build)."""
    b = header(3, 1, 0)
    b += gstr(b"big") + u32(3) + u64(1 << 32) + u64(1 << 32) + u64(1 << 8) + u32(0) + u64(0)
    assert_invalid(tmp_path, "ovf", b, "overflow")
    b = header(3, 1, 0)
    b += gstr(b"big") + u32(2) + u64(1 << 62) + u64(2) + u32(0) + u64(0)  # bytes = 2^63 * 4
    assert_invalid(tmp_path, "ovf2", b, "overflow")
