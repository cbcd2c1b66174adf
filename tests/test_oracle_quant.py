"""Pins for the oracle's block decoders (oracle/styx_oracle.c) -- each check
is independent of the decoder's own formula: exhaustive sweeps against IEEE
arithmetic, structural special cases, and encoders written from the block
layout (crates/gguf-rs/src/lib.rs:242-332, crates/model/src/moe.rs:506-533,
the public ggml q5_K/q6_K layouts)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O

F16_SAMPLES = [0x3C00, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xBC00, 0x3555, 0x2E66, 0xC4D2, 0x1234]


def f16(bits: int) -> np.float32:
    return np.array([bits], np.uint16).view(np.float16).astype(np.float32)[0]


def test_f16_all_inputs():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    lib = O.lib()
    got = np.array([lib.styx_oracle_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_block_table_matches_gguf_rs():
    # crates/gguf-rs/src/lib.rs:242-332
    lib = O.lib()
    for t, el, by in [(0, 1, 4), (1, 1, 2), (8, 32, 34), (12, 256, 144), (13, 256, 176), (14, 256, 210)]:
        assert lib.styx_oracle_block_elems(t) == el and lib.styx_oracle_block_bytes(t) == by
    assert lib.styx_oracle_block_elems(99) == 0


def test_q8_0_exhaustive():
    """Every byte value under a set of f16 scales: y = f16(d) * int8(q) (lib.rs:103-113)."""
    q = np.arange(256, dtype=np.uint8).reshape(8, 32)
    for dbits in F16_SAMPLES:
        blocks = np.zeros((8, 34), np.uint8)
        blocks[:, 0] = dbits & 0xFF
        blocks[:, 1] = dbits >> 8
        blocks[:, 2:] = q
        got = O.dequant(8, blocks.ravel(), 256)
        ref = f16(dbits) * q.ravel().view(np.int8).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32)), hex(dbits)


def pack_k4_scales(sc, m):
    """Inverse of get_scale_min (moe.rs:513-522): 8 (sc, m) 6-bit pairs -> 12 bytes."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return s


def k4_block(d_bits, dmin_bits, sc, m, nibbles):
    """q4_K block from 256 4-bit values in element order."""
    b = np.zeros(144, np.uint8)
    b[0], b[1], b[2], b[3] = d_bits & 0xFF, d_bits >> 8, dmin_bits & 0xFF, dmin_bits >> 8
    b[4:16] = pack_k4_scales(sc, m)
    for c in range(4):
        for l in range(32):
            b[16 + 32 * c + l] = nibbles[64 * c + l] | (nibbles[64 * c + 32 + l] << 4)
    return b


@pytest.mark.parametrize("seed", range(20))
def test_q4_k_scale_min_brute_force(seed):
    """Distinct random (sc, m) per sub-block; d = dmin = 1: y = sc*q - m exactly."""
    rng = np.random.default_rng(seed)
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    got = O.dequant(12, k4_block(0x3C00, 0x3C00, sc, m, q), 256)
    j = np.arange(256) // 32
    assert np.array_equal(got, (sc[j] * q - m[j]).astype(np.float32))


def test_q4_k_nibble_placement():
    """One qs byte at 32c+l: low nibble -> element 64c+l, high -> 64c+32+l."""
    ones = np.ones(8, int)
    for c in range(4):
        for l in (0, 13, 31):
            b = k4_block(0x3C00, 0x3C00, ones, np.zeros(8, int), np.zeros(256, int))
            b[16 + 32 * c + l] = 0x21
            got = O.dequant(12, b, 256)
            want = np.zeros(256, np.float32)
            want[64 * c + l], want[64 * c + 32 + l] = 1, 2
            assert np.array_equal(got, want)


def test_q4_k_evaluation_order():
    """((d*sc)*q) - (dmin*m) in f32, the reference's order (moe.rs:527-528)."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        d_bits, dm_bits = int(rng.integers(0x2000, 0x3C00)), int(rng.integers(0x2000, 0x3C00))
        sc, m, q = rng.integers(1, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)
        got = O.dequant(12, k4_block(d_bits, dm_bits, sc, m, q), 256)
        j = np.arange(256) // 32
        d, dm = f16(d_bits), f16(dm_bits)
        ref = (d * sc[j].astype(np.float32)) * q.astype(np.float32) - dm * m[j].astype(np.float32)
        assert np.array_equal(got, ref.astype(np.float32))


def k5_block(k4: np.ndarray, qh: np.ndarray) -> np.ndarray:
    """q5_K block = q4_K header/scales + qh[32] + the same qs."""
    b = np.zeros(176, np.uint8)
    b[0:16] = k4[0:16]
    b[16:48] = qh
    b[48:176] = k4[16:144]
    return b


def test_q5_k_reduces_to_q4_k():
    rng = np.random.default_rng(5)
    for _ in range(20):
        k4 = rng.integers(0, 256, 144).astype(np.uint8)
        k4[1], k4[3] = (k4[1] & 0x83) | 0x30, (k4[3] & 0x83) | 0x30
        y4 = O.dequant(12, k4, 256)
        y5 = O.dequant(13, k5_block(k4, np.zeros(32, np.uint8)), 256)
        assert np.array_equal(y4, y5)


def test_q5_k_high_bit_placement():
    """qh[l] bit 2c -> element 64c+l gains 16*d*sc; bit 2c+1 -> element 64c+32+l."""
    sc, m = np.arange(1, 9), np.zeros(8, int)
    base = k4_block(0x3C00, 0x3C00, sc, m, np.zeros(256, int))
    y0 = O.dequant(13, k5_block(base, np.zeros(32, np.uint8)), 256)
    for bit in range(8):
        for l in (0, 17, 31):
            qh = np.zeros(32, np.uint8)
            qh[l] = 1 << bit
            y = O.dequant(13, k5_block(base, qh), 256)
            c, hi = bit // 2, bit % 2
            e = 64 * c + 32 * hi + l
            want = y0.copy()
            want[e] += 16 * sc[e // 32]
            assert np.array_equal(y, want), (bit, l)


def k6_block(q: np.ndarray, scales: np.ndarray, d_bits: int) -> np.ndarray:
    """q6_K encoder from the layout: 6-bit values q (0..63) in element order.
    Element 128n + 32i + l (i = 0..3, l = 0..31) keeps its low 4 bits in
    ql[64n + l + 32*(i&1)] (low nibble for i < 2, high for i >= 2) and its
    high 2 bits in qh[32n + l] bits 2i..2i+1; scales[j] covers values
    16j..16j+15; d (f16) at byte 208."""
    b = np.zeros(210, np.uint8)
    for n in range(2):
        for i in range(4):
            for l in range(32):
                v = int(q[128 * n + 32 * i + l])
                pos = 64 * n + l + 32 * (i & 1)
                b[pos] |= (v & 15) << (4 if i >= 2 else 0)
                b[128 + 32 * n + l] |= (v >> 4) << (2 * i)
    b[192:208] = scales.astype(np.int8).view(np.uint8)
    b[208], b[209] = d_bits & 0xFF, d_bits >> 8
    return b


@pytest.mark.parametrize("seed", range(10))
def test_q6_k_hand_built_blocks(seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 64, 256)
    sc = rng.integers(-128, 128, 16)
    got = O.dequant(14, k6_block(q, sc, 0x3C00), 256)
    want = (sc[np.arange(256) // 16] * (q - 32)).astype(np.float32)
    assert np.array_equal(got, want)
    # the scale factor lives at byte 208: d = 2 doubles every value
    got2 = O.dequant(14, k6_block(q, sc, 0x4000), 256)
    assert np.array_equal(got2, 2 * want)


def test_dequant_rejects_partial_blocks():
    with pytest.raises(ValueError):
        O.dequant(12, np.zeros(144, np.uint8), 100)
