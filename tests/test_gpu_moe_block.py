"""GPU tests of the fused MoE block (moe_block.hip): one persistent launch
per layer must give the results of the four separate kernels (router,
gate/up, down, reduce) -- the same routed ids, logits and per-layer
residuals within 1e-6 relative L2 (the same arithmetic; the compiler may
contract a multiply-add differently in the fused kernel) -- at the shapes of
the configs it serves, and stay exact across graph replays of the same
launch (each replay draws a new tag).  A layer's q/k/v matvec runs in the
tail of the previous layer's fused block when its weights are q8_0: the same
comparison covers it (the separate path launches every q/k/v itself)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    from styx_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def shapes():
    from styx_amd import SynthConfig
    from styx_amd import _lib as L
    return {
        # mixed q4_K/q5_K/q6_K per layer and role, E 32, k 4
        "mixed_small": SynthConfig(n_layers=3, n_embd=512, n_heads=8, n_kv_heads=2, head_dim=64,
                                   n_expert=32, n_expert_used=4, n_ff_exp=256, n_vocab=2048,
                                   exp_mix=True, seed=123),
        # q8_0 experts, F 768 (down with 3 units per lane)
        "q8_layer": SynthConfig(n_layers=1, n_embd=2048, n_heads=32, n_kv_heads=4, head_dim=128,
                                n_expert=128, n_expert_used=8, n_ff_exp=768, n_vocab=4096,
                                seed=0xA1),
        # E 512 (two-level ranking), k 10, shared expert as slot k
        "e512_shexp": SynthConfig(n_layers=2, n_embd=2048, n_heads=16, n_kv_heads=2,
                                  head_dim=128, n_expert=512, n_expert_used=10, n_ff_exp=512,
                                  n_ff_shexp=512, n_vocab=4096,
                                  exp_type=(L.Q4_K, L.Q4_K, L.Q6_K), seed=0x80B),
        # H 4096, F 1536 (down with 2 units per lane); the
        # folded q/k/v takes its limbs in two poll rounds
        "h4096": SynthConfig(n_layers=2, n_embd=4096, n_heads=64, n_kv_heads=4, head_dim=128,
                             n_expert=128, n_expert_used=8, n_ff_exp=1536, n_vocab=2048,
                             exp_type=(L.Q4_K, L.Q4_K, L.Q4_K), seed=0x235),
    }


@pytest.mark.parametrize("name", ["mixed_small", "q8_layer", "e512_shexp", "h4096"])
def test_fused_equals_separate_kernels(gpu, name):
    from styx_amd import MoeModel
    cfg = shapes()[name]
    fused = MoeModel.synth(gpu, cfg, n_ctx=32, record_hidden=True)
    sep = MoeModel.synth(gpu, cfg, n_ctx=32, record_hidden=True, fuse=False)
    # the fused kernel is the one that runs
    fused.set_timing(True)
    fused.forward_token(1)
    stats = fused.kernel_stats()
    fused.set_timing(False)
    assert "moe_block" in stats and "moe_gate_up" not in stats, sorted(stats)
    # q8_0 attention weights: only the first layer's q/k/v is a launch of its own
    assert stats["qkv"][0] == 1, stats["qkv"]
    sep.forward_token(1)
    for t in [7, cfg.n_vocab - 1, 300, 2]:
        la, lb = fused.forward_token(t), sep.forward_token(t)
        assert rel_l2(la, lb) < 1e-6, t
        ha, hb = fused.last_hidden(), sep.last_hidden()
        for l in range(ha.shape[0]):
            assert rel_l2(ha[l], hb[l]) < 1e-6, (t, l)
        assert np.array_equal(fused.last_expert_ids(), sep.last_expert_ids()), t
    fused.close()
    sep.close()


def test_qkv_fold_equals_unfolded(gpu):
    """The q/k/v folded into the block's tail is the separate q/k/v kernel's
    arithmetic: logits and residuals agree within 1e-6 relative L2 (the
    compiler may contract a multiply-add differently), fold on or off."""
    from styx_amd import MoeModel
    cfg = shapes()["e512_shexp"]
    a = MoeModel.synth(gpu, cfg, n_ctx=32, record_hidden=True)
    b = MoeModel.synth(gpu, cfg, n_ctx=32, record_hidden=True, fold_qkv=False)
    for t in [9, 4000, 12]:
        la, lb = a.forward_token(t), b.forward_token(t)
        assert rel_l2(la, lb) < 1e-6, t
        ha, hb = a.last_hidden(), b.last_hidden()
        for l in range(ha.shape[0]):
            assert rel_l2(ha[l], hb[l]) < 1e-6, (t, l)
        assert np.array_equal(a.last_expert_ids(), b.last_expert_ids()), t
    a.close()
    b.close()


def test_fused_replays_keep_results(gpu):
    """Graph replays of the fused launches (stage timing: every replay a new
    tag) leave the model exact: the next token equals a model that never
    replayed, and decode continues identically."""
    from styx_amd import MoeModel
    cfg = shapes()["mixed_small"]
    a = MoeModel.synth(gpu, cfg, n_ctx=64)
    b = MoeModel.synth(gpu, cfg, n_ctx=64)
    for t in [3, 4, 5]:
        a.forward_token(t)
        b.forward_token(t)
    us, n = a.time_stage("moe_block", 7)
    assert n == cfg.n_layers and us > 0
    la, lb = a.forward_token(6), b.forward_token(6)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert np.array_equal(a.decode(12), b.decode(12))
    a.close()
    b.close()
