"""Pins for the oracle's ops and its forward pass: the reference tests'
LCG known-answer setups (crates/vk-backend/tests/{kernels,ops2}.rs) checked
against f64 closed forms, invariants, brute force, and an independent numpy
f64 implementation of the decode step (crates/model/src/moe.rs:1780-2073)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Lcg, clamp_f16_exponents, rel_l2
from oracle import oracle as O

SKIP = 0xFFFFFFFF


def lcg_quant(seed, nbytes, block_bytes, f16_offsets):
    r = Lcg(seed)
    a = r.bytes(nbytes)
    clamp_f16_exponents(a, block_bytes, f16_offsets)
    return a, r


def sum_bound(t, a, rows, cols, x):
    """Forward error bound of a sequential f32 sum of `cols` products:
    |y - y_exact| <= cols * 2^-24 * sum_i |w_i x_i| (Higham, Accuracy and
    Stability, eq. 3.5, first order)."""
    w = O.dequant(t, a, rows * cols).reshape(rows, cols).astype(np.float64)
    return cols * 2.0 ** -24 * (np.abs(w) @ np.abs(x.astype(np.float64)))


def test_q4_k_matvec_kat():
    """kernels.rs:353-456: seed 0xdeadbeef, 64 rows x 512 cols, exponent clamp."""
    a, r = lcg_quant(0xDEADBEEF, 64 * 2 * 144, 144, (0, 2))
    x = r.f32s(512)
    y = O.matvec(12, a, 64, 512, x)
    y64 = O.matvec_f64(12, a, 64, 512, x)
    assert (np.abs(y - y64) <= sum_bound(12, a, 64, 512, x)).all()
    # the reference's own acceptance (relative 2e-2 against its CPU path)
    assert np.max(np.abs(y - y64) / np.maximum(np.abs(y64), 1e-3)) < 2e-2


def test_q8_0_matvec_kat():
    """ops2.rs:225-292: seed 0x51ce, 128 rows x 1024 cols."""
    a, r = lcg_quant(0x51CE, 128 * 32 * 34, 34, (0,))
    x = r.f32s(1024)
    y = O.matvec(8, a, 128, 1024, x)
    y64 = O.matvec_f64(8, a, 128, 1024, x)
    assert (np.abs(y - y64) <= sum_bound(8, a, 128, 1024, x)).all()
    assert np.max(np.abs(y - y64) / np.maximum(np.abs(y64), 1e-3)) < 1e-3  # reference: 1e-3


def test_matvec_f64_closed_form():
    """The f64 checker equals numpy's dot of the (pinned) dequantized rows."""
    rng = np.random.default_rng(1)
    for t, bb in ((8, 34), (12, 144), (13, 176), (14, 210)):
        be = 32 if t == 8 else 256
        a = rng.integers(0, 256, 16 * (512 // be) * bb).astype(np.uint8)
        clamp_f16_exponents(a, bb, (208,) if t == 14 else (0,) if t == 8 else (0, 2))
        x = rng.standard_normal(512).astype(np.float32)
        w = O.dequant(t, a, 16 * 512).reshape(16, 512).astype(np.float64)
        assert np.allclose(O.matvec_f64(t, a, 16, 512, x), w @ x.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_matvec_id_routing_kat():
    """kernels.rs:150-285: 8 q4_K experts of 32x512, ids [6,1,3,0] then
    [0,6,1,3]; each slot equals its expert's own matvec and the permuted
    routing permutes the outputs."""
    a, r = lcg_quant(0xCAFEF00D, 8 * 32 * 2 * 144, 144, (0, 2))
    x = r.f32s(512)
    stride = 32 * 2 * 144
    y1 = O.matvec_id(12, a, 32, 512, stride, [6, 1, 3, 0], x, 1)
    y2 = O.matvec_id(12, a, 32, 512, stride, [0, 6, 1, 3], x, 1)
    for s, e in enumerate([6, 1, 3, 0]):
        assert np.array_equal(y1[32 * s:32 * s + 32], O.matvec(12, a[e * stride:(e + 1) * stride], 32, 512, x))
    assert np.array_equal(y2[:32], y1[96:128]) and np.array_equal(y2[32:64], y1[:32])


def test_matvec_id_skip_and_ne11():
    rng = np.random.default_rng(2)
    a = rng.integers(0, 256, 4 * 8 * 34).astype(np.uint8)
    clamp_f16_exponents(a, 34, (0,))
    x = rng.standard_normal(3 * 32).astype(np.float32)
    sentinel = np.full(3 * 8, 7.0, np.float32)
    y = O.matvec_id(8, a, 8, 32, 8 * 34, [2, SKIP, 1], x, 3, y=sentinel.copy())
    assert (y[8:16] == 7.0).all()                       # SKIP slot untouched
    assert np.array_equal(y[16:24], O.matvec(8, a[8 * 34:16 * 34], 8, 32, x[64:96]))  # b = (s % ne11)


def test_rms_norm_kat_and_invariance():
    """kernels.rs:41-122: seed 0x12345678, 4 rows of 2048, eps 1e-6."""
    x = Lcg(0x12345678).f32s(2048 * 4)
    got = O.rms_norm(x, None, 2048, 4, 1e-6)
    xr = x.reshape(4, 2048).astype(np.float64)
    ref = xr / np.sqrt((xr ** 2).mean(1, keepdims=True) + 1e-6)
    assert np.max(np.abs(got.reshape(4, 2048) - ref)) < 1e-6  # reference: 1e-5
    # scale invariance, bit-exact for a power-of-two scale and eps = 0
    assert np.array_equal(O.rms_norm(4 * x, None, 2048, 4, 0.0), O.rms_norm(x, None, 2048, 4, 0.0))
    w = np.linspace(0.5, 1.5, 2048).astype(np.float32)
    assert np.allclose(O.rms_norm(x, w, 2048, 4, 1e-6).reshape(4, 2048), ref * w, atol=2e-6)


def test_swiglu_kat():
    """ops2.rs:296-348: seed 0x5119, gate = 4*lcg, up = lcg."""
    r = Lcg(0x5119)
    n = 3072 * 2
    g = (r.f32s(n) * np.float32(4.0)).astype(np.float32)
    u = r.f32s(n)
    got = O.swiglu(g, u)
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert np.max(np.abs(got - ref)) < 1e-6  # reference: 1e-5


def rope_complex(x, hd, nh, pos, base):
    """Rotation as complex multiplication by exp(i*pos*base^(-2i/hd))."""
    x = x.astype(np.float64).reshape(nh, hd)
    half = hd // 2
    z = x[:, :half] + 1j * x[:, half:]
    z = z * np.exp(1j * pos * base ** (-2.0 * np.arange(half) / hd))
    return np.concatenate([z.real, z.imag], 1).ravel()


def test_rope_kat_and_invariants():
    """ops2.rs:413-490: seed 0x40e0, head_dim 128, 4 heads, positions 0/5/17, base 1e6."""
    r = Lcg(0x40E0)
    x = r.f32s(128 * 4 * 3).reshape(3, 512)
    for t, pos in enumerate([0, 5, 17]):
        got = O.rope_neox(x[t], 128, 4, pos, 1e6)
        assert np.max(np.abs(got - rope_complex(x[t], 128, 4, pos, 1e6))) < 1e-6  # reference: 1e-4
        if pos == 0:
            assert np.array_equal(got, x[t])  # identity at position 0
        nrm = lambda v: np.hypot(v.reshape(4, 128)[:, :64], v.reshape(4, 128)[:, 64:])
        assert np.allclose(nrm(got), nrm(x[t]), rtol=1e-6)
    a = O.rope_neox(O.rope_neox(x[1], 128, 4, 300, 1e6), 128, 4, 77, 1e6)
    assert np.max(np.abs(a - O.rope_neox(x[1], 128, 4, 377, 1e6))) < 1e-5


def test_router_strided_closed_form():
    rng = np.random.default_rng(4)
    W = (0.02 * rng.standard_normal((128, 2048))).astype(np.float32)
    x = rng.standard_normal(2048).astype(np.float32)
    got = O.router_strided(W, x, 128, 2048)
    assert np.max(np.abs(got - W.astype(np.float64) @ x)) < 1e-5


def topk_brute(logits, k, renorm):
    order = sorted(range(len(logits)), key=lambda i: (-float(logits[i]), i))[:k]
    p = np.exp(logits.astype(np.float64) - logits.max())
    p /= p.sum()
    w = p[order]
    return order, (w / w.sum() if renorm else w)


@pytest.mark.parametrize("n,k", [(128, 8), (512, 10), (8, 8), (16, 1)])
def test_topk_brute_force(n, k):
    rng = np.random.default_rng(n + k)
    for trial in range(20):
        lg = rng.standard_normal(n).astype(np.float32)
        if trial % 3 == 0:  # ties: lowest index wins
            lg[rng.integers(0, n, n // 4)] = lg.max()
        for renorm in (True, False):
            w, ids = O.topk_softmax(lg, k, renorm)
            order, wref = topk_brute(lg, k, renorm)
            assert ids[:k].tolist() == order
            assert np.max(np.abs(w - wref)) < 1e-6
            if renorm:
                assert abs(w.astype(np.float64).sum() - 1) < 1e-6


def test_topk_id_rows_partition():
    """Rows 16/32/48 put every routed expert in exactly one of hot/arena/host
    (topk_softmax_f32.comp:4-17)."""
    rng = np.random.default_rng(8)
    E, k = 64, 8
    lg = rng.standard_normal(E).astype(np.float32)
    remap = np.full(E, SKIP, np.uint32)
    hot = rng.choice(E, 20, replace=False)
    remap[hot] = np.arange(20)
    pmap = np.full(E, SKIP, np.uint32)
    pre = rng.choice(E, 10, replace=False)
    pmap[pre] = 100 + np.arange(10)
    _, ids = O.topk_softmax(lg, k, True, remap, pmap)
    for s in range(k):
        e = ids[s]
        row = [ids[16 + s], ids[32 + s], ids[48 + s]]
        assert sum(v != -1 for v in row) == 1
        if remap[e] != SKIP:
            assert row[0] == remap[e]
        elif pmap[e] != SKIP:
            assert row[1] == pmap[e]
        else:
            assert row[2] == e


def test_moe_reduce_closed_form():
    rng = np.random.default_rng(9)
    d = rng.standard_normal(8 * 2048).astype(np.float32)
    w = rng.random(8).astype(np.float32)
    x = rng.standard_normal(2048).astype(np.float32)
    got = O.moe_reduce(d, w, 2048, 8, x)
    ref = x + (w.astype(np.float64)[:, None] * d.reshape(8, 2048)).sum(0)
    assert np.max(np.abs(got - ref)) < 1e-5


@pytest.mark.parametrize("n_t", [1, 7, 300])
def test_attention_online_vs_two_pass(n_t):
    rng = np.random.default_rng(n_t)
    nh, nkv, hd = 8, 2, 128
    kvd = nkv * hd
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = rng.standard_normal((n_t, kvd)).astype(np.float32)
    V = rng.standard_normal((n_t, kvd)).astype(np.float32)
    sc = 1 / np.sqrt(hd)
    got = O.attn_decode(q, K, V, n_t, hd, kvd, nh // nkv, nh, sc)
    ref = O.attn_decode_f64(q, K, V, n_t, hd, kvd, nh // nkv, nh, sc)
    assert rel_l2(got, ref) < 1e-6
    # textbook check of the f64 checker itself
    Kh = K.astype(np.float64).reshape(n_t, nkv, hd)
    Vh = V.astype(np.float64).reshape(n_t, nkv, hd)
    for h in range(nh):
        s = Kh[:, h // 4] @ q[h * hd:(h + 1) * hd].astype(np.float64) * sc
        p = np.exp(s - s.max())
        assert np.allclose(ref[h * hd:(h + 1) * hd], (p / p.sum()) @ Vh[:, h // 4], atol=1e-12)
    if n_t == 1:  # one token: the output is that token's V row
        assert np.array_equal(got.reshape(nh, hd), np.repeat(V.reshape(nkv, hd), 4, 0))
    perm = rng.permutation(n_t)  # attention is invariant to the order of the cache rows
    assert rel_l2(O.attn_decode(q, K[perm], V[perm], n_t, hd, kvd, 4, nh, sc), ref) < 1e-6


def test_gather_memcmp():
    rng = np.random.default_rng(10)
    import ctypes as C
    E, k, layer = 6, 3, 2
    slabs = [64, 48, 80]
    src = [rng.integers(0, 256, E * s, dtype=np.uint8) for s in slabs]
    dst = [np.zeros((layer + 1) * k * 80, np.uint8) for _ in range(3)]
    ids = np.array([4, SKIP, 0], np.uint32)
    S = (C.c_void_p * 3)(*[a.ctypes.data for a in src])
    D = (C.c_void_p * 3)(*[a.ctypes.data for a in dst])
    O.lib().styx_oracle_gather_slabs(S, (C.c_int64 * 3)(*slabs), D, (C.c_int64 * 3)(80, 80, 80),
                                     ids.ctypes.data, k, layer)
    for t in range(3):
        v = dst[t].reshape(-1, 80)
        assert np.array_equal(v[layer * k, :slabs[t]], src[t].reshape(E, -1)[4])
        assert not v[layer * k + 1].any()
        assert np.array_equal(v[layer * k + 2, :slabs[t]], src[t].reshape(E, -1)[0])
        assert not v[:layer * k].any()


def test_argmax_total_cmp_last():
    assert O.argmax(np.array([1, 3, 3, 2], np.float32)) == 2
    assert O.argmax(np.array([0.0, -0.0], np.float32)) == 0      # +0 > -0 under total_cmp
    assert O.argmax(np.array([-0.0, 0.0], np.float32)) == 1
    assert O.argmax(np.array([np.inf, np.nan, 1], np.float32)) == 1  # +NaN sorts above +inf
    assert O.argmax(np.array([-5, -5, -7], np.float32)) == 1


# ------------------------------------------------- forward-pass wiring -----

def quant_q8_0(w: np.ndarray) -> np.ndarray:
    """Simple q8_0 quantizer (block max / 127) for building a test model."""
    b = w.reshape(-1, 32).astype(np.float32)
    d = (np.abs(b).max(1) / 127).astype(np.float16)
    df = d.astype(np.float32)
    q = np.clip(np.rint(np.divide(b, df[:, None], out=np.zeros_like(b), where=df[:, None] > 0)), -127, 127)
    out = np.zeros((b.shape[0], 34), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.ravel()


def tiny_model(seed=0, shexp=False, bias=False):
    """Two-layer q8_0 model; shexp adds a shared expert of width 32 with its
    sigmoid gate row, bias a per-expert router bias -1.1*ln(rank) over a
    seeded rank permutation (the config-3 Zipf extension)."""
    rng = np.random.default_rng(seed)
    Fs = 32 if shexp else 0
    hp = dict(n_layers=2, n_embd=256, n_heads=4, n_kv_heads=2, head_dim=64, n_expert=8,
              n_expert_used=2, n_ff_exp=64, n_ff_shexp=Fs, n_vocab=96, rms_eps=1e-6,
              rope_base=1e4, norm_topk=1)
    H, qd, kvd, E, F, V = 256, 256, 128, 8, 64, 96
    T = {}

    def qmat(name, rows, cols, nmat=1, sigma=0.05):
        w = (sigma * rng.standard_normal(nmat * rows * cols)).astype(np.float32)
        T[name] = (8, [cols, rows] + ([nmat] if nmat > 1 else []), quant_q8_0(w))

    def f32(name, v):
        T[name] = (0, [len(v)], np.asarray(v, np.float32).view(np.uint8))

    qmat("token_embd.weight", V, H, sigma=1.0)
    qmat("output.weight", V, H)
    f32("output_norm.weight", 1 + 0.1 * rng.standard_normal(H))
    for l in range(2):
        p = f"blk.{l}."
        f32(p + "attn_norm.weight", 1 + 0.1 * rng.standard_normal(H))
        f32(p + "attn_q_norm.weight", 1 + 0.1 * rng.standard_normal(64))
        f32(p + "attn_k_norm.weight", 1 + 0.1 * rng.standard_normal(64))
        f32(p + "ffn_norm.weight", 1 + 0.1 * rng.standard_normal(H))
        qmat(p + "attn_q.weight", qd, H)
        qmat(p + "attn_k.weight", kvd, H)
        qmat(p + "attn_v.weight", kvd, H)
        qmat(p + "attn_output.weight", H, qd)
        f32(p + "ffn_gate_inp.weight", 0.1 * rng.standard_normal(E * H))
        qmat(p + "ffn_gate_exps.weight", F, H, E)
        qmat(p + "ffn_up_exps.weight", F, H, E)
        qmat(p + "ffn_down_exps.weight", H, F, E)
        if shexp:
            qmat(p + "ffn_gate_shexp.weight", Fs, H)
            qmat(p + "ffn_up_shexp.weight", Fs, H)
            qmat(p + "ffn_down_shexp.weight", H, Fs)
            f32(p + "ffn_gate_inp_shexp.weight", 0.1 * rng.standard_normal(H))
        if bias:
            f32(p + "ffn_gate_inp.bias", -1.1 * np.log(1 + rng.permutation(E)))
    return hp, T


def np_forward(hp, T, toks, use_bias=True):
    """Independent f64 decode of a token sequence (moe.rs:1842-2073 op order),
    plus the two extensions the oracle carries: a router bias added to the
    logits before top-k, and the shared expert
    x += sigmoid(ginp . xn) * down_sh(silu(gate_sh xn) * up_sh xn)
    (shaders/axpy_sig_f32.comp:2, moe.rs:127-151).  Returns per-token logits
    and the routed ids [token][layer][k]."""
    H, nh, nkv, hd, E, k, F = 256, 4, 2, 64, 8, 2, 64
    eps, base = hp["rms_eps"], hp["rope_base"]

    def deq(name):
        t, dims, data = T[name]
        if t == 0:
            return data.view(np.float32).astype(np.float64)
        n = int(np.prod(dims))
        return O.dequant(8, data, n).astype(np.float64).reshape(list(reversed(dims)))

    def rms(v, w):
        return v / np.sqrt((v * v).mean(-1, keepdims=True) + eps) * w

    def rope(v, pos):  # v [heads, hd]
        half = hd // 2
        th = pos * base ** (-2.0 * np.arange(half) / hd)
        c, s = np.cos(th), np.sin(th)
        return np.concatenate([v[:, :half] * c - v[:, half:] * s, v[:, :half] * s + v[:, half:] * c], 1)

    def silu(v):
        return v / (1 + np.exp(-v))

    emb = deq("token_embd.weight")
    Kc = [[] for _ in range(2)]
    Vc = [[] for _ in range(2)]
    out, routed = [], []
    for pos, tok in enumerate(toks):
        x = emb[tok].copy()
        rids = []
        for l in range(2):
            p = f"blk.{l}."
            xn = rms(x, deq(p + "attn_norm.weight"))
            q = (deq(p + "attn_q.weight") @ xn).reshape(nh, hd)
            kk = (deq(p + "attn_k.weight") @ xn).reshape(nkv, hd)
            vv = (deq(p + "attn_v.weight") @ xn).reshape(nkv, hd)
            q = rope(rms(q, deq(p + "attn_q_norm.weight")), pos)
            kk = rope(rms(kk, deq(p + "attn_k_norm.weight")), pos)
            Kc[l].append(kk)
            Vc[l].append(vv)
            Ks, Vs = np.stack(Kc[l]), np.stack(Vc[l])
            att = np.zeros((nh, hd))
            for h in range(nh):
                s = Ks[:, h // 2] @ q[h] / np.sqrt(hd)
                pr = np.exp(s - s.max())
                att[h] = (pr / pr.sum()) @ Vs[:, h // 2]
            x = x + deq(p + "attn_output.weight") @ att.ravel()
            xn = rms(x, deq(p + "ffn_norm.weight"))
            lg = deq(p + "ffn_gate_inp.weight").reshape(E, H) @ xn
            if use_bias and p + "ffn_gate_inp.bias" in T:
                lg = lg + deq(p + "ffn_gate_inp.bias")
            order = sorted(range(E), key=lambda i: (-lg[i], i))[:k]
            rids.append(order)
            pr = np.exp(lg - lg.max())
            pr /= pr.sum()
            w = pr[order] / pr[order].sum()
            G, U, D = deq(p + "ffn_gate_exps.weight"), deq(p + "ffn_up_exps.weight"), deq(p + "ffn_down_exps.weight")
            moe = np.zeros(H)
            for s_, e in enumerate(order):
                g, u = G[e] @ xn, U[e] @ xn
                moe += w[s_] * (D[e] @ (silu(g) * u))
            if p + "ffn_gate_shexp.weight" in T:
                hs = silu(deq(p + "ffn_gate_shexp.weight") @ xn) * (deq(p + "ffn_up_shexp.weight") @ xn)
                gate = 1 / (1 + np.exp(-(deq(p + "ffn_gate_inp_shexp.weight") @ xn)))
                moe += gate * (deq(p + "ffn_down_shexp.weight") @ hs)
            x = x + moe
        out.append(deq("output.weight") @ rms(x, deq("output_norm.weight")))
        routed.append(rids)
    return out, routed


def test_oracle_forward_matches_numpy_f64():
    hp, T = tiny_model(0)
    orc = O.OracleModel(hp, T, n_ctx=8)
    toks = [5, 60, 17, 90, 1]
    ref, _ = np_forward(hp, T, toks)
    for pos, t in enumerate(toks):
        lg, hid, ids, margins = orc.forward(pos, t, want_hidden=True)
        assert rel_l2(lg, ref[pos]) < 1e-5, pos


def test_oracle_forward_shared_expert_and_router_bias_match_numpy_f64():
    """The oracle's shared-expert branch (axpy_sig merge) and router-bias add
    (styx_oracle_moe_block) against the independent f64 forward.  The bias is
    strong enough to change the routed experts on some (token, layer), so a
    dropped or mis-signed bias fails the id check, and the shared expert
    moves the logits by far more than the tolerance, so a dropped branch, a
    wrong gate sign or gate input fails the logits check."""
    hp, T = tiny_model(3, shexp=True, bias=True)
    orc = O.OracleModel(hp, T, n_ctx=8)
    toks = [5, 60, 17, 90, 1, 33]
    ref, rids = np_forward(hp, T, toks)
    _, rids_nobias = np_forward(hp, T, toks, use_bias=False)
    assert rids != rids_nobias, "bias must change the routing somewhere"
    T_plain = {n: v for n, v in T.items() if "shexp" not in n}
    ref_plain, _ = np_forward(dict(hp, n_ff_shexp=0), T_plain, toks)
    assert min(rel_l2(a, b) for a, b in zip(ref, ref_plain)) > 1e-3
    for pos, t in enumerate(toks):
        lg, hid, ids, margins = orc.forward(pos, t, want_hidden=True)
        assert rel_l2(lg, ref[pos]) < 1e-5, pos
        for l in range(2):
            if margins[l] > 1e-4:
                assert ids[l].tolist() == rids[pos][l], (pos, l)


def test_axpy_sig_closed_form():
    """shaders/axpy_sig_f32.comp:7-11, d += sigmoid(g) * a, against f64 for
    gates across the sigmoid's range (saturated both ways, 0 -> 1/2)."""
    rng = np.random.default_rng(11)
    a = rng.standard_normal(300).astype(np.float32)
    d = rng.standard_normal(300).astype(np.float32)
    for g in [-100.0, -7.5, -1.0, 0.0, 0.3, 2.0, 15.0, 100.0]:
        got = O.axpy_sig(a, g, d).astype(np.float64)
        want = d.astype(np.float64) + a.astype(np.float64) / (1.0 + np.exp(-g))
        assert np.abs(got - want).max() <= 4e-7 * (np.abs(want) + np.abs(a)).max(), g
    assert np.array_equal(O.axpy_sig(a, 0.0, np.zeros_like(a)), a * np.float32(0.5))
    assert np.array_equal(O.axpy_sig(a, 200.0, d), d + a)
