"""GPU parity tests of the hot-path kernels against the CPU oracle, through
the C ABI (libstyx_hip.so).  Bit-exact for layout, dequant, ids and bytes;
floating point within the tolerance written in each test."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import rel_l2
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TYPES = [8, 12, 13, 14]  # q8_0, q4_K, q5_K, q6_K
BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


@pytest.fixture(scope="module")
def gpu():
    from styx_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def lib():
    from styx_amd import _lib
    return _lib.load()


def check(rc):
    from styx_amd import _lib
    _lib.check(rc)


def gen_quant(gpu, t, n, seed, sigma=0.02):
    """Seeded quant blocks generated on the device; returns (device buf, host bytes)."""
    nbytes = n // BLOCK[t][0] * BLOCK[t][1]
    b = gpu.buffer(nbytes)
    check(lib().styx_op_gen_quant(gpu.h, t, seed, C.c_float(sigma), b.ptr, n))
    return b, b.download()


def split(gpu, t, gguf_buf, rows, cols, nmat=1):
    from styx_amd.runtime import to_split
    return to_split(gpu, t, gguf_buf, rows, cols, nmat)


@pytest.mark.parametrize("t", TYPES)
def test_split_layout_roundtrip(gpu, t):
    from styx_amd.runtime import from_split
    rows, cols, nmat = 64, 512, 3
    b, host = gen_quant(gpu, t, rows * cols * nmat, seed=11 + t)
    s = split(gpu, t, b, rows, cols, nmat)
    back = from_split(gpu, t, s, rows, cols, nmat).download()
    assert np.array_equal(back, host)
    assert not np.array_equal(s.download(), host)  # it really is a permutation


@pytest.mark.parametrize("t", TYPES)
def test_dequant_bit_exact(gpu, t):
    rows, cols = 48, 768
    b, host = gen_quant(gpu, t, rows * cols, seed=21 + t, sigma=1.0)
    s = split(gpu, t, b, rows, cols)
    out = gpu.buffer(rows * cols * 4)
    check(lib().styx_op_dequant_rows(gpu.h, t, s.ptr, rows, cols, 0, rows, out.ptr))
    got = out.download(np.float32)
    ref = O.dequant(t, host, rows * cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("ncols", [512, 768, 2048, 4096, 8192])
def test_matvec_dense(gpu, t, ncols):
    if ncols % BLOCK[t][0]:
        pytest.skip("not a block multiple")
    rows = 200
    b, host = gen_quant(gpu, t, rows * ncols, seed=31 + t + ncols)
    s = split(gpu, t, b, rows, ncols)
    rng = np.random.default_rng(ncols + t)
    x = rng.standard_normal(ncols).astype(np.float32)
    xb, yb = gpu.from_numpy(x), gpu.buffer(rows * 4)
    check(lib().styx_op_matvec(gpu.h, t, s.ptr, rows, ncols, xb.ptr, None, C.c_float(0), yb.ptr, 0))
    got = yb.download(np.float32)
    ref = O.matvec_f64(t, host, rows, ncols, x)
    # activation limbs carry ~23 bits: f32-class error against the f64 dot
    assert rel_l2(got, ref) < 2e-6
    assert np.max(np.abs(got - ref)) < 1e-5 * np.abs(ref).max()


def test_matvec_dense_many_rows(gpu):
    """q8_0 rows of 2048 values, 40,960 of them: every workgroup takes 40
    rows, the walk that loads the activation limbs into LDS once per
    workgroup (as the LM head of configs[1] does)."""
    t, rows, ncols = 8, 40960, 2048
    b, host = gen_quant(gpu, t, rows * ncols, seed=77)
    s = split(gpu, t, b, rows, ncols)
    rng = np.random.default_rng(78)
    x = rng.standard_normal(ncols).astype(np.float32)
    xb, yb = gpu.from_numpy(x), gpu.buffer(rows * 4)
    check(lib().styx_op_matvec(gpu.h, t, s.ptr, rows, ncols, xb.ptr, None, C.c_float(0), yb.ptr, 0))
    got = yb.download(np.float32)
    ref = O.matvec_f64(t, host, rows, ncols, x)
    assert rel_l2(got, ref) < 2e-6
    assert np.max(np.abs(got - ref)) < 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("t", [8, 14])
def test_matvec_norm_add(gpu, t):
    rows, ncols, eps = 96, 2048, 1e-6
    b, host = gen_quant(gpu, t, rows * ncols, seed=41 + t)
    s = split(gpu, t, b, rows, ncols)
    rng = np.random.default_rng(5)
    x = rng.standard_normal(ncols).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(ncols)).astype(np.float32)
    y0 = rng.standard_normal(rows).astype(np.float32)
    xb, wb, yb = gpu.from_numpy(x), gpu.from_numpy(w), gpu.from_numpy(y0)
    check(lib().styx_op_matvec(gpu.h, t, s.ptr, rows, ncols, xb.ptr, wb.ptr, C.c_float(eps),
                               yb.ptr, 1))
    xn = O.rms_norm(x, w, ncols, 1, eps)
    ref = y0.astype(np.float64) + O.matvec_f64(t, host, rows, ncols, xn)
    assert rel_l2(yb.download(np.float32), ref) < 2e-6


def _router_case(gpu, E, H, k, seed, bias=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(H).astype(np.float32)
    nw = np.ones(H, np.float32)
    W = (0.02 * rng.standard_normal((E, H))).astype(np.float32)
    bv = (-1.1 * np.log(rng.permutation(E) + 1)).astype(np.float32) if bias else None
    bufs = dict(x=gpu.from_numpy(x), nw=gpu.from_numpy(nw), W=gpu.from_numpy(W),
                xn=gpu.buffer(H * 4), lg=gpu.buffer(E * 4), w=gpu.buffer(64), ids=gpu.buffer(256))
    bb = gpu.from_numpy(bv) if bias else None
    check(lib().styx_op_router_topk(gpu.h, bufs["x"].ptr, bufs["nw"].ptr, C.c_float(1e-6),
                                    bufs["W"].ptr, bb.ptr if bb else None, E, H, k, 1, None, None,
                                    0, 0, bufs["xn"].ptr, bufs["lg"].ptr, bufs["w"].ptr,
                                    bufs["ids"].ptr))
    gpu.sync()
    return x, W, bv, {n: b for n, b in bufs.items()}


@pytest.mark.parametrize("E,H,k", [(128, 2048, 8), (512, 2048, 10), (128, 4096, 8), (16, 512, 4)])
def test_router_topk(gpu, E, H, k):
    for seed in range(3):
        x, W, _, b = _router_case(gpu, E, H, k, seed)
        xn_ref = O.rms_norm(x, np.ones(H, np.float32), H, 1, 1e-6)
        xn = b["xn"].download(np.float32)
        assert rel_l2(xn, xn_ref) < 1e-6
        lg = b["lg"].download(np.float32)
        lg_ref = W.astype(np.float64) @ xn_ref.astype(np.float64)
        assert np.max(np.abs(lg - lg_ref)) < 1e-5
        # top-k on identical logits is bit-exact against the oracle
        w_ref, ids_ref = O.topk_softmax(lg, k, True)
        ids = b["ids"].download(np.int32)
        assert np.array_equal(ids[:k], ids_ref[:k])
        assert np.array_equal(ids[16:16 + k], ids_ref[:k])       # identity remap: hot = e
        assert (ids[32:32 + k] == -1).all() and (ids[48:48 + k] == -1).all()
        w = b["w"].download(np.float32)[:k]
        assert np.max(np.abs(w - w_ref)) < 1e-6
        assert abs(float(w.sum()) - 1.0) < 1e-5


def test_router_bias(gpu):
    E, H, k = 128, 2048, 8
    x, W, bv, b = _router_case(gpu, E, H, k, 3, bias=True)
    xn_ref = O.rms_norm(x, np.ones(H, np.float32), H, 1, 1e-6)
    lg_ref = W.astype(np.float64) @ xn_ref.astype(np.float64) + bv
    lg = b["lg"].download(np.float32)
    assert np.max(np.abs(lg - lg_ref)) < 1e-5


def test_topk_softmax_rows(gpu):
    """Hot/arena/host id rows with a remap and pmap (topk_softmax_f32.comp:4-17)."""
    rng = np.random.default_rng(9)
    E, k = 64, 6
    logits = rng.standard_normal(E).astype(np.float32)
    logits[10] = logits[20] = np.float32(5.0)  # a tie: lowest index first
    remap = np.full(E, 0xFFFFFFFF, np.uint32)
    remap[[10, 3, 7]] = [0, 1, 2]
    pmap = np.full(E, 0xFFFFFFFF, np.uint32)
    pmap[20] = 17
    lb, rb, pb = gpu.from_numpy(logits), gpu.from_numpy(remap), gpu.from_numpy(pmap)
    wb, ib = gpu.buffer(64), gpu.buffer(256)
    check(lib().styx_op_topk_softmax(gpu.h, lb.ptr, E, k, 1, rb.ptr, pb.ptr, 0, 0, wb.ptr, ib.ptr))
    gpu.sync()
    w_ref, ids_ref = O.topk_softmax(logits, k, True, remap, pmap)
    ids = ib.download(np.int32)
    for row in (0, 16, 32, 48):
        assert np.array_equal(ids[row:row + k], ids_ref[row:row + k]), row
    assert ids[0] == 10 and ids[1] == 20
    assert np.max(np.abs(wb.download(np.float32)[:k] - w_ref)) < 1e-6


def _expert_block(gpu, types, H, F, E, k, seed):
    tg, tu, td = types
    bufs = {}
    host = {}
    for name, t, rows, cols in (("g", tg, F, H), ("u", tu, F, H), ("d", td, H, F)):
        b, hb = gen_quant(gpu, t, E * rows * cols, seed=seed * 10 + len(bufs))
        bufs[name] = split(gpu, t, b, rows, cols, E)
        host[name] = hb
    return bufs, host


@pytest.mark.parametrize("types,H,F,E,k", [
    ((8, 8, 8), 2048, 768, 128, 8),
    ((12, 13, 14), 2048, 768, 128, 8),
    ((13, 14, 12), 2048, 768, 32, 8),
    ((14, 12, 13), 2048, 768, 32, 8),
    ((12, 12, 14), 2048, 512, 64, 10),
    ((12, 12, 12), 4096, 1536, 16, 8),
])
def test_moe_block(gpu, types, H, F, E, k):
    """router+topk -> gate/up -> swiglu+down+reduce against the oracle MoE block."""
    from styx_amd._lib import ExpertSrc
    tg, tu, td = types
    bufs, host = _expert_block(gpu, types, H, F, E, k, seed=H + F + E)
    rng = np.random.default_rng(E)
    x = rng.standard_normal(H).astype(np.float32)
    nw = (1 + 0.05 * rng.standard_normal(H)).astype(np.float32)
    W = (0.02 * rng.standard_normal((E, H))).astype(np.float32)
    xb, nwb, Wb = gpu.from_numpy(x), gpu.from_numpy(nw), gpu.from_numpy(W)
    xn, lg, wts, ids = gpu.buffer(H * 4), gpu.buffer(E * 4), gpu.buffer(64), gpu.buffer(256)
    check(lib().styx_op_router_topk(gpu.h, xb.ptr, nwb.ptr, C.c_float(1e-6), Wb.ptr, None, E, H, k,
                                    1, None, None, 0, 0, xn.ptr, lg.ptr, wts.ptr, ids.ptr))
    slab = {n: b.nbytes // E for n, b in bufs.items()}
    src = {n: ExpertSrc(hot=bufs[n].ptr, hot_slab=slab[n]) for n in bufs}
    gu = gpu.buffer(2 * k * F * 4)
    check(lib().styx_op_moe_gate_up(gpu.h, tg, tu, C.byref(src["g"]), C.byref(src["u"]), ids.ptr,
                                    xn.ptr, gu.ptr, H, F, k))
    check(lib().styx_op_moe_down_reduce(gpu.h, td, C.byref(src["d"]), ids.ptr, wts.ptr, gu.ptr,
                                        xb.ptr, H, F, k))
    gpu.sync()
    # oracle on the same routing
    xn_ref = O.rms_norm(x, nw, H, 1, 1e-6)
    lgh = lg.download(np.float32)
    w_ref, ids_ref = O.topk_softmax(lgh, k, True)
    idh = ids.download(np.int32)
    assert np.array_equal(idh[:k], ids_ref[:k])
    sel = ids_ref[:k].astype(np.uint32)
    g = O.matvec_id(tg, host["g"], F, H, slab["g"], sel, xn_ref, 1)
    u = O.matvec_id(tu, host["u"], F, H, slab["u"], sel, xn_ref, 1)
    gu_h = gu.download(np.float32).reshape(2, k * F)
    assert rel_l2(gu_h[0], g) < 1e-5 and rel_l2(gu_h[1], u) < 1e-5
    h = O.swiglu(g, u)
    d = O.matvec_id(td, host["d"], H, F, slab["d"], sel, h, k)
    x_ref = O.moe_reduce(d, w_ref, H, k, x)
    assert rel_l2(xb.download(np.float32) - x, x_ref - x) < 1e-5
    # a second call accumulates again into the residual
    check(lib().styx_op_moe_down_reduce(gpu.h, td, C.byref(src["d"]), ids.ptr, wts.ptr, gu.ptr,
                                        xb.ptr, H, F, k))
    gpu.sync()
    x2_ref = O.moe_reduce(d, w_ref, H, k, x_ref)
    assert rel_l2(xb.download(np.float32) - x, x2_ref - x) < 1e-5


def _norm_rope_ref(v, w, hd, nh, pos, base, eps=1e-6):
    v = O.rms_norm(v, w, hd, nh, eps) if w is not None else v
    return O.rope_neox(v, hd, nh, pos, base)


@pytest.mark.parametrize("nh,nkv,hd,n_steps,page,max_chunks",
                         [(32, 4, 128, 70, 512, 4), (64, 4, 128, 40, 32, 4), (8, 8, 64, 33, 64, 4),
                          (32, 4, 128, 70, 512, 2), (64, 4, 128, 40, 32, 1),
                          (16, 8, 256, 50, 64, 3)])
def test_attention_paged(gpu, nh, nkv, hd, n_steps, page, max_chunks):
    """Fused norm+rope+append+split-context attention over a scrambled page
    table.  With few chunks the per-chunk span grows past the minimum of 32
    tokens (max(32, ceil16(n_t / max_chunks))), so waves walk several tiles."""
    rng = np.random.default_rng(nh + hd + max_chunks)
    kvd = nkv * hd
    n_ctx = 128
    chunk = 32
    npages = max(1, -(-n_ctx // page))
    pt = rng.permutation(npages).astype(np.int32)   # logical -> physical, scrambled
    kpool, vpool = gpu.zeros(npages * page * kvd * 4), gpu.zeros(npages * page * kvd * 4)
    base = 1e6
    rope = np.empty((n_ctx, hd // 2, 2), np.float64)
    lib().styx_rope_table(C.c_float(base), hd, n_ctx, rope.ctypes.data)
    invb, ptb = gpu.from_numpy(rope), gpu.from_numpy(pt)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    qnb, knb = gpu.from_numpy(qn), gpu.from_numpy(kn)
    part = gpu.buffer(lib().styx_op_attn_part_floats(nh, nkv, hd, max_chunks) * 4)
    out = gpu.buffer(nh * hd * 4)
    K = np.zeros((n_ctx, kvd), np.float32)
    Vv = np.zeros((n_ctx, kvd), np.float32)
    scale = 1.0 / np.sqrt(hd)
    for pos in range(n_steps):
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k = rng.standard_normal(kvd).astype(np.float32)
        v = rng.standard_normal(kvd).astype(np.float32)
        qb, kb, vb, posb = gpu.from_numpy(q), gpu.from_numpy(k), gpu.from_numpy(v), gpu.from_numpy(np.array([pos], np.int32))
        check(lib().styx_op_attn_decode(gpu.h, qb.ptr, kb.ptr, vb.ptr, qnb.ptr, knb.ptr,
                                        C.c_float(1e-6), invb.ptr, kpool.ptr, vpool.ptr, ptb.ptr,
                                        page, posb.ptr, out.ptr, part.ptr, nh, nkv, hd, chunk,
                                        max_chunks, C.c_float(scale)))
        gpu.sync()
        qr = _norm_rope_ref(q, qn, hd, nh, pos, base)
        K[pos] = _norm_rope_ref(k, kn, hd, nkv, pos, base)
        Vv[pos] = v
        ref = O.attn_decode_f64(qr, K, Vv, pos + 1, hd, kvd, nh // nkv, nh, scale)
        got = out.download(np.float32)
        assert rel_l2(got, ref) < 2e-6, pos
    # the cache holds the appended rows at their paged addresses
    kp = kpool.download(np.float32).reshape(npages, page, kvd)
    vp = vpool.download(np.float32).reshape(npages, page, kvd)
    for t in range(n_steps):
        # K went through RMSNorm (its sum order differs from the oracle's) and rope
        np.testing.assert_allclose(kp[pt[t // page], t % page], K[t], rtol=2e-6, atol=2e-6)
        assert np.array_equal(vp[pt[t // page], t % page], Vv[t]), t


@pytest.mark.parametrize("nh,nkv,n_t", [(32, 4, 3001), (64, 4, 8001)])
def test_attention_many_chunks(gpu, nh, nkv, n_t):
    """One decode step after a long context written straight into the paged
    pools: about a hundred chunks per kv head (94 for the VALU kernel's
    32-token chunks, 126 for the matrix-core kernel's 64), so the combine
    kernel merges two batches per half wave and drops the grid's chunks past
    the context (the grid is 128 chunks)."""
    rng = np.random.default_rng(n_t)
    hd, page, chunk, max_chunks = 128, 512, 32, 128
    kvd = nkv * hd
    npages = -(-n_t // page)
    pt = rng.permutation(npages).astype(np.int32)
    K = rng.standard_normal((n_t, kvd)).astype(np.float32)
    Vv = rng.standard_normal((n_t, kvd)).astype(np.float32)
    kp = np.zeros((npages, page, kvd), np.float32)
    vp = np.zeros((npages, page, kvd), np.float32)
    pos = n_t - 1
    for t in range(pos):
        kp[pt[t // page], t % page] = K[t]
        vp[pt[t // page], t % page] = Vv[t]
    kpool, vpool = gpu.from_numpy(kp), gpu.from_numpy(vp)
    base = 1e6
    rope = np.empty((n_t, hd // 2, 2), np.float64)
    lib().styx_rope_table(C.c_float(base), hd, n_t, rope.ctypes.data)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(kvd).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    part = gpu.buffer(lib().styx_op_attn_part_floats(nh, nkv, hd, max_chunks) * 4)
    out = gpu.buffer(nh * hd * 4)
    bufs = [gpu.from_numpy(x) for x in (q, k, v, rope, pt, np.array([pos], np.int32))]
    qb, kb, vb, invb, ptb, posb = bufs
    scale = 1.0 / np.sqrt(hd)
    check(lib().styx_op_attn_decode(gpu.h, qb.ptr, kb.ptr, vb.ptr, None, None, C.c_float(1e-6),
                                    invb.ptr, kpool.ptr, vpool.ptr, ptb.ptr, page, posb.ptr,
                                    out.ptr, part.ptr, nh, nkv, hd, chunk, max_chunks,
                                    C.c_float(scale)))
    gpu.sync()
    qr = O.rope_neox(q, hd, nh, pos, base)
    K[pos] = O.rope_neox(k, hd, nkv, pos, base)
    Vv[pos] = v
    ref = O.attn_decode_f64(qr, K, Vv, n_t, hd, kvd, nh // nkv, nh, scale)
    assert rel_l2(out.download(np.float32), ref) < 2e-6


def test_gather_slabs(gpu):
    rng = np.random.default_rng(2)
    E, k, layer = 12, 4, 3
    slabs = [1 << 12, 3 << 10, 5 << 9]
    srcs = [gpu.from_numpy(rng.integers(0, 256, E * s, dtype=np.uint8)) for s in slabs]
    dsl = [max(slabs)] * 3
    dsts = [gpu.zeros((layer + 1) * k * d) for d in dsl]
    ids = np.array([7, 0xFFFFFFFF, 2, 11], np.uint32)
    idb = gpu.from_numpy(ids)
    S = (C.c_void_p * 3)(*[b.ptr for b in srcs])
    D = (C.c_void_p * 3)(*[b.ptr for b in dsts])
    check(lib().styx_op_gather_slabs(gpu.h, S, (C.c_int64 * 3)(*slabs), D, (C.c_int64 * 3)(*dsl),
                                     idb.ptr, k, layer))
    gpu.sync()
    for t in range(3):
        hs = srcs[t].download().reshape(E, slabs[t])
        hd = dsts[t].download().reshape(-1, dsl[t])
        for s in range(k):
            slot = layer * k + s
            if ids[s] == 0xFFFFFFFF:
                assert not hd[slot].any()
            else:
                assert np.array_equal(hd[slot, :slabs[t]], hs[ids[s]])
                assert not hd[slot, slabs[t]:].any()
        assert not hd[:layer * k].any()


def test_argmax_ties_last(gpu):
    rng = np.random.default_rng(4)
    for n in (1, 1000, 151936):
        v = rng.standard_normal(n).astype(np.float32)
        if n > 10:
            v[[5, n // 2, n - 3]] = v.max() + 1  # ties: the last index wins
        vb, ob, sv, si = gpu.from_numpy(v), gpu.buffer(4), gpu.buffer(256), gpu.buffer(256)
        check(lib().styx_op_argmax(gpu.h, vb.ptr, n, ob.ptr, sv.ptr, si.ptr))
        gpu.sync()
        assert int(ob.download(np.uint32)[0]) == O.argmax(v)
