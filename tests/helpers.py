"""Shared test helpers: LCG of the reference tests, relative errors, and
building an oracle model from the engine's exported tensors."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


class Lcg:
    """crates/vk-backend/tests/ops2.rs:29-38: s = s*1664525 + 1013904223."""

    def __init__(self, seed: int):
        self.s = seed & 0xFFFFFFFF

    def next(self) -> int:
        self.s = (self.s * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.s

    def f32(self) -> float:
        # (s >> 8) as f32 / 2^24 * 2 - 1, evaluated in f32
        return np.float32(np.float32(np.float32(self.next() >> 8) / np.float32(1 << 24)) * np.float32(2.0)) - np.float32(1.0)

    def f32s(self, n: int) -> np.ndarray:
        return np.array([self.f32() for _ in range(n)], np.float32)

    def bytes(self, n: int) -> np.ndarray:
        return np.array([(self.next() >> 16) & 0xFF for _ in range(n)], np.uint8)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def clamp_f16_exponents(blocks: np.ndarray, block_bytes: int, offsets) -> None:
    """kernels.rs:168-171: blk[o+1] = (blk[o+1] & 0x83) | 0x30 keeps f16 scales finite."""
    v = blocks.reshape(-1, block_bytes)
    for o in offsets:
        v[:, o + 1] = (v[:, o + 1] & 0x83) | 0x30


def model_hparams(m) -> dict:
    hp = m.hp
    return dict(n_layers=hp.n_layers, n_embd=hp.n_embd, n_heads=hp.n_heads,
                n_kv_heads=hp.n_kv_heads, head_dim=hp.head_dim, n_expert=hp.n_expert,
                n_expert_used=hp.n_expert_used, n_ff_exp=hp.n_ff_exp,
                n_ff_shexp=hp.n_ff_shexp, n_vocab=hp.n_vocab, rms_eps=hp.rms_eps,
                rope_base=hp.rope_base, norm_topk=hp.norm_topk)


def export_all(m) -> dict:
    return {n: m.export_tensor(n) for n in m.tensor_names()}


def oracle_from_model(m, n_ctx: int) -> O.OracleModel:
    return O.OracleModel(model_hparams(m), export_all(m), n_ctx)


class Tally:
    """Routed-id checks done and skipped as near-ties (k-th vs k+1-th logit
    within 1e-4 in the oracle): ids are compared bit for bit wherever the
    oracle's routing margin leaves no doubt, and the skips are counted so
    that a test can bound them."""

    def __init__(self):
        self.checked = self.skipped = 0

    def ids(self, gpu_ids, oracle_ids, margins, where):
        for l in range(gpu_ids.shape[0]):
            if margins[l] > 1e-4:
                assert np.array_equal(gpu_ids[l], oracle_ids[l].astype(np.uint32)), (where, l)
                self.checked += 1
            else:
                self.skipped += 1

    def bound(self, frac: float = 0.1):
        """At most frac of the (layer, step) pairs skipped, and at least one
        skip allowed however few pairs there are."""
        n = self.checked + self.skipped
        assert self.skipped <= max(1, int(frac * n)), (self.checked, self.skipped)
