"""The reference's own model formats end to end on the GPU: a GGUF file with
a q4_K token_embd (the table forward_token decodes, moe.rs:1824-1833),
K-quant attention (q4_K q/k/v, q6_K output projection), a q6_K LM head and
mixed q4_K/q5_K/q6_K experts -- the UD-Q4_K_XL-style mix -- written to
disk, loaded through styx_moe_load and decoded, against the oracle: logits
and every layer's residual within 1e-4 relative L2, routed ids identical
wherever the oracle's routing margin is not a near-tie (counted).  The same
with the f32 and f16 embedding tables MoeModel::load also admits
(moe.rs:1107-1112)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Tally, export_all, model_hparams, oracle_from_model, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    from styx_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def _cfg(**kw):
    from styx_amd import SynthConfig
    base = dict(n_layers=3, n_embd=512, n_heads=8, n_kv_heads=2, head_dim=64, n_expert=32,
                n_expert_used=4, n_ff_exp=256, n_vocab=2048, exp_mix=True, seed=321)
    base.update(kw)
    return SynthConfig(**base)


@pytest.mark.parametrize("embd", ["q4_K", "f16", "f32"])
def test_kquant_mix_through_gguf_load(gpu, tmp_path, embd):
    from styx_amd import MoeModel, _lib as L
    from styx_amd.gguf_io import model_metadata, write
    et = {"q4_K": L.Q4_K, "f16": L.F16, "f32": L.F32}[embd]
    # two synthetic models that differ only in their attention type: every
    # tensor is seeded by its name, so the f32 tensors and experts agree
    a = MoeModel.synth(gpu, _cfg(embd_type=et, attn_type=L.Q4_K, head_type=L.Q6_K), n_ctx=32)
    b = MoeModel.synth(gpu, _cfg(embd_type=et, attn_type=L.Q6_K, head_type=L.Q6_K), n_ctx=32)
    tens = export_all(a)
    tb = export_all(b)
    for name in tens:
        if name.endswith("attn_output.weight"):
            tens[name] = tb[name]
    hp = model_hparams(a)
    a.close()
    b.close()
    assert tens["token_embd.weight"][0] == et
    assert tens["blk.0.attn_q.weight"][0] == L.Q4_K
    assert tens["blk.0.attn_output.weight"][0] == L.Q6_K
    assert tens["output.weight"][0] == L.Q6_K
    path = tmp_path / "mix.gguf"
    write(path, model_metadata(hp), [(n, t, d, by) for n, (t, d, by) in tens.items()])
    m = MoeModel.load(gpu, str(path), n_ctx=32, record_hidden=True)
    assert m.export_tensor("token_embd.weight")[0] == et
    orc = oracle_from_model(m, 32)
    tally = Tally()
    for pos, t in enumerate([7, 1999, 640, 5, 1024, 77]):
        lg = m.forward_token(t)
        hid = m.last_hidden()
        ol, oh, oids, margins = orc.forward(pos, t, want_hidden=True)
        assert rel_l2(lg, ol) < 1e-4, pos
        for l in range(hid.shape[0]):
            assert rel_l2(hid[l], oh[l]) < 1e-4, (pos, l)
        tally.ids(m.last_expert_ids(), oids, margins, pos)
    tally.bound()
    m.close()
