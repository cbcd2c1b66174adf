"""GGUF v3 writer and a minimal reader (crates/gguf-rs/src/lib.rs semantics:
little-endian header, typed metadata, tensor infos with offsets relative to
the 32-byte aligned data section)."""
from __future__ import annotations

import struct

import numpy as np

GGUF_MAGIC = 0x46554747
# metadata value types (lib.rs:151-167)
VT_U8, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STR, VT_ARR, VT_U64, VT_I64, VT_F64 = range(13)


def _str(b: bytearray, s: str) -> None:
    e = s.encode()
    b += struct.pack("<Q", len(e)) + e


def _val(b: bytearray, v) -> None:
    if isinstance(v, bool):
        b += struct.pack("<IB", VT_BOOL, int(v))
    elif isinstance(v, int):
        b += struct.pack("<II", VT_U32, v)
    elif isinstance(v, float):
        b += struct.pack("<If", VT_F32, v)
    elif isinstance(v, str):
        b += struct.pack("<I", VT_STR)
        _str(b, v)
    else:
        raise TypeError(f"unsupported metadata value {v!r}")


def write(path, metadata: dict, tensors: list, alignment: int = 32) -> None:
    """tensors: [(name, ggml_type, dims (GGUF order), bytes ndarray)]."""
    hdr = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(metadata)))
    for k, v in metadata.items():
        _str(hdr, k)
        _val(hdr, v)
    off = 0
    offsets = []
    for name, typ, dims, data in tensors:
        _str(hdr, name)
        hdr += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        hdr += struct.pack("<IQ", typ, off)
        offsets.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    pad = (-len(hdr)) % alignment
    with open(path, "wb") as f:
        f.write(hdr)
        f.write(b"\0" * pad)
        for (name, typ, dims, data), o in zip(tensors, offsets):
            raw = np.ascontiguousarray(data).view(np.uint8).tobytes()
            f.write(raw)
            f.write(b"\0" * ((-len(raw)) % alignment))


def model_metadata(hp: dict, arch: str = "qwen3moe") -> dict:
    """The metadata keys MoeModel::load reads (crates/model/src/moe.rs:550-590)."""
    return {
        "general.architecture": arch,
        "general.alignment": 32,
        f"{arch}.block_count": hp["n_layers"],
        f"{arch}.embedding_length": hp["n_embd"],
        f"{arch}.attention.head_count": hp["n_heads"],
        f"{arch}.attention.head_count_kv": hp["n_kv_heads"],
        f"{arch}.attention.key_length": hp["head_dim"],
        f"{arch}.expert_count": hp["n_expert"],
        f"{arch}.expert_used_count": hp["n_expert_used"],
        f"{arch}.expert_feed_forward_length": hp["n_ff_exp"],
        f"{arch}.attention.layer_norm_rms_epsilon": float(hp["rms_eps"]),
        f"{arch}.rope.freq_base": float(hp["rope_base"]),
    }
