"""GPU parity at BASELINE.json's full shapes, against the CPU oracle or the
all-in-HBM run (the parity bar: greedy tokens identical over 256 tokens,
per-layer hidden states within 1e-4 relative L2, top-k ids bit-exact,
placement invariance of scripts/verify.sh:57-78).

* the 48-layer 30B-A3B shape, 16-token prompt (seed 0xC0FFEE)
  then 256 greedy tokens: at every one of the 271 positions the logits, the
  49 residuals and the routed ids are compared with the oracle fed the same
  token, and the GPU's greedy token must be the oracle's argmax -- so the
  free-running streams are identical; the device-argmax graph path must
  then reproduce the same 256 tokens.
* the same shape with the Zipf(1.1) router bias, experts in
  pinned host memory under a 6 GiB HBM budget, cold slabs read in place or
  gathered into the arena: logits bit-identical to all-in-HBM, hot + cold
  = tokens x 48 x 8.
  The same routing and placement at 4 layers against the oracle.
* the 235B-A22B layer shape (H 4096, 64/4 heads, E 128 top-8,
  F 1536, q4_K experts; 2 of its 94 layers) at 512 and 32768 tokens of
  context: per-layer hidden states and logits against the oracle.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from helpers import Tally, oracle_from_model, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def gpu():
    from styx_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


@pytest.mark.timeout(900)
def test_config2_greedy_256_tokens_and_hidden_states(gpu):
    from oracle import oracle as O
    from styx_amd import CFG_30B_A3B, MoeModel
    from styx_amd.model import argmax_last
    O.set_threads(16)
    n_new = 256
    rng = np.random.default_rng(0xC0FFEE)
    prompt = rng.integers(0, CFG_30B_A3B.n_vocab, 16).astype(np.uint32).tolist()
    n_ctx = len(prompt) + n_new + 8
    m = MoeModel.synth(gpu, CFG_30B_A3B, n_ctx=n_ctx, record_hidden=True)
    orc = oracle_from_model(m, n_ctx)
    tally = Tally()
    worst_logit = worst_hidden = 0.0
    stream = []
    feed = list(prompt)
    pos = 0
    while len(stream) < n_new:
        t = feed[pos] if pos < len(prompt) else stream[-1]
        lg = m.forward_token(t)
        hid = m.last_hidden()
        ids = m.last_expert_ids()
        ol, oh, oids, margins = orc.forward(pos, t, want_hidden=True)
        e = rel_l2(lg, ol)
        assert e < TOL, ("logits", pos, e)
        worst_logit = max(worst_logit, e)
        for l in range(hid.shape[0]):
            e = rel_l2(hid[l], oh[l])
            assert e < TOL, ("hidden", pos, l, e)
            worst_hidden = max(worst_hidden, e)
        tally.ids(ids, oids, margins, pos)
        if pos >= len(prompt) - 1:
            g = argmax_last(lg)
            assert g == O.argmax(ol), ("greedy token", pos)
            stream.append(g)
        pos += 1
    pairs = tally.checked + tally.skipped
    print(f"\nconfigs[1]: {n_new} greedy tokens identical; {pos} positions; worst rel L2 "
          f"logits {worst_logit:.2e}, hidden {worst_hidden:.2e}; routed-id checks "
          f"{tally.checked} of {pairs} (step, layer) pairs, {tally.skipped} skipped as near-ties")
    assert tally.skipped <= 0.02 * pairs
    # the timed path: graph replays with the argmax on the device
    m.reset()
    toks, _, _ = m.generate(np.array(prompt, np.uint32), n_new)
    assert toks.tolist() == stream
    m.close()


def logits_run(m, prompt, n_new):
    """Prompt then n_new greedy tokens through forward_token: every step's
    logits, the token stream, and the (hot, cold) totals."""
    from styx_amd.model import argmax_last
    out, toks = [], []
    hot = cold = 0
    t = None
    for i in range(len(prompt) + n_new - 1):
        t = prompt[i] if i < len(prompt) else argmax_last(out[-1])
        out.append(m.forward_token(int(t)))
        if i >= len(prompt) - 1:
            toks.append(argmax_last(out[-1]))
        hc = m.last_hot_cold()
        assert (hc.sum(1) == m.hp.n_expert_used).all()
        hot += int(hc[:, 0].sum())
        cold += int(hc[:, 1].sum())
    return out, toks, hot, cold


@pytest.mark.timeout(600)
@pytest.mark.parametrize("arena", [False, True])
def test_config3_host_pinned_6gib_identical(gpu, tmp_path, arena):
    """Cold slabs read in place by the fused block (arena False) or gathered
    into the HBM arena by the separate kernels (True); the all-in-HBM model
    runs the same path with the same Zipf bias.  The hot set is the bias
    ranking (popularity CSV), 6 GiB of slabs."""
    from styx_amd import CFG_30B_A3B, MoeModel
    cfg = replace(CFG_30B_A3B, router_zipf_s=1.1)
    rng = np.random.default_rng(0xC0FFEE)
    prompt = rng.integers(0, cfg.n_vocab, 16).astype(np.uint32).tolist()
    n_new = 16
    ref = MoeModel.synth(gpu, cfg, n_ctx=64, fuse=not arena)
    want, want_toks, hot, cold = logits_run(ref, prompt, n_new)
    assert cold == 0
    rows = ["layer,expert,hits"]
    for l in range(cfg.n_layers):
        b = ref.export_tensor(f"blk.{l}.ffn_gate_inp.bias")[2].view(np.float32)
        rows += [f"{l},{e},{int(round(1e6 * np.exp(b[e])))}" for e in range(len(b))]
    hist = tmp_path / "zipf_hist.csv"
    hist.write_text("\n".join(rows) + "\n")
    ref.close()
    m = MoeModel.synth(gpu, cfg, n_ctx=64, fuse=not arena, expert_budget_mb=6144,
                       expert_hist=str(hist), arena=arena)
    assert m.hp.expert_bytes_host > 0 and 5.5 * 2**30 < m.hp.expert_bytes_hbm
    got, toks, hot, cold = logits_run(m, prompt, n_new)
    for i, (a, b) in enumerate(zip(want, got)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
    assert toks == want_toks
    steps = len(prompt) + n_new - 1
    assert hot + cold == steps * cfg.n_layers * cfg.n_expert_used
    print(f"\nconfigs[2] arena={arena}: {steps} tokens bit-identical to all-in-HBM; "
          f"hit rate {hot / (hot + cold):.3f}")
    assert 0.5 < hot / (hot + cold) < 1.0
    # the HUD of generate_moe.rs:87-119 over scripts/verify.sh:69-78's run:
    # 2 prompt + 32 generated tokens, 33 forwarded, 48 layers, k 8
    import re
    from styx_amd import generate_hud
    m.reset()
    _, hud = generate_hud(m, prompt[:2], 32)
    print("\n".join(hud))
    assert sum(int(v) for v in re.findall(r"\((\d+)\)", hud[0])) == 12672
    assert re.match(r"^hud: cold/layer \[[.0-9]{48}\]", hud[1])
    m.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("arena", [False, True])
def test_config3_zipf_host_pinned_against_oracle(gpu, tmp_path, arena):
    """configs[2]'s routing and placement at configs[1]'s layer shape on 4
    layers, against the oracle (the tests above hold the full-size run to
    the all-in-HBM one): Zipf(1.1) router bias, experts in pinned host
    memory under a 160 MiB HBM budget (about a tenth of the 512 (layer,
    expert) slabs hot, by the bias ranking), cold slabs read in place by the fused block or
    gathered into the arena; at every position each layer's residual and
    the logits within 1e-4 of the oracle with the same bias, routed ids
    identical outside counted near-ties, and both hot and cold slabs used."""
    from oracle import oracle as O
    from styx_amd import CFG_30B_A3B, MoeModel
    O.set_threads(16)
    cfg = replace(CFG_30B_A3B, n_layers=4, router_zipf_s=1.1)
    rng = np.random.default_rng(0x21BF)
    prompt = rng.integers(0, cfg.n_vocab, 6).astype(np.uint32).tolist()
    n_ctx = 32
    ref = MoeModel.synth(gpu, cfg, n_ctx=n_ctx)
    rows = ["layer,expert,hits"]
    for l in range(cfg.n_layers):
        b = ref.export_tensor(f"blk.{l}.ffn_gate_inp.bias")[2].view(np.float32)
        rows += [f"{l},{e},{int(round(1e6 * np.exp(b[e])))}" for e in range(len(b))]
    hist = tmp_path / "zipf_hist.csv"
    hist.write_text("\n".join(rows) + "\n")
    orc = oracle_from_model(ref, n_ctx)
    ref.close()
    m = MoeModel.synth(gpu, cfg, n_ctx=n_ctx, record_hidden=True, expert_budget_mb=160,
                       expert_hist=str(hist), arena=arena, fuse=not arena)
    assert m.hp.expert_bytes_host > 0 and m.hp.expert_bytes_hbm > 0
    tally = Tally()
    hot = cold = 0
    feed = list(prompt)
    for pos in range(len(prompt) + 6):
        t = feed[pos]
        lg = m.forward_token(t)
        hid = m.last_hidden()
        ol, oh, oids, margins = orc.forward(pos, t, want_hidden=True)
        assert rel_l2(lg, ol) < TOL, pos
        for l in range(hid.shape[0]):
            assert rel_l2(hid[l], oh[l]) < TOL, (pos, l)
        tally.ids(m.last_expert_ids(), oids, margins, pos)
        hc = m.last_hot_cold()
        hot += int(hc[:, 0].sum())
        cold += int(hc[:, 1].sum())
        if pos >= len(prompt) - 1:
            feed.append(int(np.argmax(ol)))
    tally.bound()
    print(f"\nconfigs[2] routing, 4 layers, arena={arena}: hit rate {hot / (hot + cold):.3f}, "
          f"ids checked {tally.checked}, near-ties skipped {tally.skipped}")
    assert hot > 0 and cold > 0
    m.close()


@pytest.mark.timeout(600)
def test_config4_context_512_and_32768(gpu):
    """64 q / 4 kv heads (gqa 16, the matrix-core attention), head_dim 128,
    H 4096, E 128 top-8, F 1536 q4_K: synthetic K/V contexts of 512 and
    32768 tokens (64 pages of 512 at the longer one), then two real
    tokens, each layer's residual and the logits within 1e-4 of the oracle
    reading the same K/V rows."""
    from oracle import oracle as O
    from styx_amd import MoeModel, SynthConfig
    from styx_amd import _lib as L
    O.set_threads(16)
    cfg = SynthConfig(n_layers=2, n_embd=4096, n_heads=64, n_kv_heads=4, head_dim=128,
                      n_expert=128, n_expert_used=8, n_ff_exp=1536, n_vocab=8192,
                      exp_type=(L.Q4_K, L.Q4_K, L.Q4_K), seed=0x235B)
    n_max = 32768
    m = MoeModel.synth(gpu, cfg, n_ctx=n_max + 8, record_hidden=True)
    orc = oracle_from_model(m, n_max + 8)
    kvd = cfg.n_kv_heads * cfg.head_dim
    kc = orc.kc.reshape(cfg.n_layers, n_max + 8, kvd)
    vc = orc.vc.reshape(cfg.n_layers, n_max + 8, kvd)
    tally = Tally()
    for n_t in (512, n_max):
        m.reset()
        m.fill_kv(n_t, seed=11, sigma=1.0)
        for l in range(cfg.n_layers):
            k, v = m.read_kv(l, 0, n_t)
            assert np.isfinite(k).all() and abs(float(k.std()) - 1.0) < 0.05
            kc[l, :n_t], vc[l, :n_t] = k, v
        for i, t in enumerate([17, 4000]):
            lg = m.forward_token(t)
            hid = m.last_hidden()
            ol, oh, oids, margins = orc.forward(n_t + i, t, want_hidden=True)
            assert rel_l2(lg, ol) < TOL, (n_t, i)
            for l in range(hid.shape[0]):
                assert rel_l2(hid[l], oh[l]) < TOL, (n_t, i, l)
            tally.ids(m.last_expert_ids(), oids, margins, (n_t, i))
    assert tally.checked >= 6
    m.close()
