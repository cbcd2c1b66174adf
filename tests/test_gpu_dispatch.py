"""GPU tests of the drop-in dispatch level of the boundary: the reference's
pipeline names, binding order and push-constant bytes through
styx_kernel_get + styx_batch_dispatch + styx_batch_submit (the
Gpu::create_pipeline / Batch surface of crates/vk-backend/src/lib.rs), with
the reference tests' own seeds, shapes and tolerances where a reference test
exists (crates/vk-backend/tests/{kernels,ops2}.rs), checked against the CPU
oracle.  Quant weights are in GGUF block layout, as the reference uploads
them."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from helpers import Lcg, clamp_f16_exponents, rel_l2
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SKIP = 0xFFFFFFFF
BLK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
F16_AT = {8: (0,), 12: (0, 2), 13: (0, 2), 14: (208,)}
NAME = {8: "q8_0", 12: "q4_k", 13: "q5_k", 14: "q6_k"}


@pytest.fixture(scope="module")
def gpu():
    from styx_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def run(gpu, name, binds, push: bytes, grid, spec=()):
    from styx_amd.runtime import Batch, Kernel
    k = Kernel(gpu, name, list(spec))
    b = Batch(gpu)
    b.begin()
    b.dispatch(k, binds, push, grid)
    b.submit()
    b.free()
    k.free()


def f32buf(gpu, a):
    return gpu.from_numpy(np.ascontiguousarray(a, np.float32))


def sum_bound(t, a, rows, cols, x):
    """|y - y_exact| <= cols * 2^-24 * sum |w x| for any f32 summation order
    of the dot product (Higham, Accuracy and Stability, eq. 3.5)."""
    w = O.dequant(t, a, rows * cols).reshape(rows, cols).astype(np.float64)
    return cols * 2.0 ** -24 * (np.abs(w) @ np.abs(x.astype(np.float64)))


def mmv_id_push(ncols, nrows, be, k, ne11=1, batch_stride_a=None):
    # MatVecIdPush (ops.rs:123-136), as moe.rs:1576-1589 fills it
    return struct.pack("<12I", ncols, ncols // be, ncols, nrows,
                       batch_stride_a if batch_stride_a is not None else nrows * ncols,
                       ncols, k * nrows, 0, k, ne11, 0, 1)


def test_mul_mat_vec_id_q4_k_routing(gpu):
    """kernels.rs:150-285: 8 q4_K experts of 32 x 512 (LCG 0xcafef00d, f16
    exponents clamped), ids [6,1,3,0], grid (32, 4); each slot within the
    reference's 2e-2 relative and the f32 forward-error bound of its
    expert's f64 matvec; routing [0,6,1,3] permutes the slots exactly."""
    r = Lcg(0xCAFEF00D)
    a = r.bytes(8 * 32 * 2 * 144)
    clamp_f16_exponents(a, 144, (0, 2))
    x = r.f32s(512)
    ebytes = 32 * 2 * 144
    ba, bx, bd = gpu.from_numpy(a), f32buf(gpu, x), gpu.zeros(4 * 32 * 4)
    f0, f1 = gpu.zeros(16), gpu.zeros(16)
    ids = gpu.from_numpy(np.array([6, 1, 3, 0], np.int32))
    push = mmv_id_push(512, 32, 256, 4)
    run(gpu, "mul_mat_vec_id_q4_k_f32_f32", [ba, bx, bd, f0, f1, ids], push, (32, 4, 1),
        [(0, 32), (1, 1), (2, 1)])
    got = bd.download(np.float32)
    for s, e in enumerate([6, 1, 3, 0]):
        w = a[e * ebytes:(e + 1) * ebytes]
        y64 = O.matvec_f64(12, w, 32, 512, x)
        g = got[32 * s:32 * s + 32].astype(np.float64)
        assert (np.abs(g - y64) <= sum_bound(12, w, 32, 512, x)).all(), s
        assert np.max(np.abs(g - y64) / np.maximum(np.abs(y64), 1e-3)) < 2e-2
    ids.upload(np.array([0, 6, 1, 3], np.int32))
    run(gpu, "mul_mat_vec_id_q4_k_f32_f32", [ba, bx, bd, f0, f1, ids], push, (32, 4, 1),
        [(0, 32), (1, 1), (2, 1)])
    got2 = bd.download(np.float32)
    assert np.array_equal(got2[:32], got[96:128]) and np.array_equal(got2[32:64], got[:32])


@pytest.mark.parametrize("t", [8, 13, 14])
def test_mul_mat_vec_id_other_types_skip_and_ne11(gpu, t):
    """The q8_0 / q5_K / q6_K expert pipelines (no reference test covers q5_K
    and q6_K: parity against the oracle's public-format decoders), with a
    SKIP slot left untouched and ne11 = k (slot s reads x[s], the down
    projection's binding, moe.rs:2039-2048)."""
    be, bb = BLK[t]
    E, rows, cols, k = 6, 48, 512, 3
    rng = np.random.default_rng(40 + t)
    a = rng.integers(0, 256, E * rows * (cols // be) * bb).astype(np.uint8)
    clamp_f16_exponents(a, bb, F16_AT[t])
    x = rng.standard_normal(k * cols).astype(np.float32)
    sentinel = np.full(k * rows, 7.0, np.float32)
    ba, bx, bd = gpu.from_numpy(a), f32buf(gpu, x), f32buf(gpu, sentinel)
    f0, f1 = gpu.zeros(16), gpu.zeros(16)
    idl = [4, SKIP, 1]
    ids = gpu.from_numpy(np.array(idl, np.uint32))
    run(gpu, f"mul_mat_vec_id_{NAME[t]}_f32_f32", [ba, bx, bd, f0, f1, ids],
        mmv_id_push(cols, rows, be, k, ne11=k), (rows, k, 1))
    got = bd.download(np.float32)
    ebytes = rows * (cols // be) * bb
    assert (got[rows:2 * rows] == 7.0).all()
    for s, e in enumerate(idl):
        if e == SKIP:
            continue
        w = a[e * ebytes:(e + 1) * ebytes]
        xs = x[s * cols:(s + 1) * cols]
        y64 = O.matvec_f64(t, w, rows, cols, xs)
        assert (np.abs(got[s * rows:(s + 1) * rows] - y64) <= sum_bound(t, w, rows, cols, xs)).all()


def test_mul_mat_vec_id_out_of_range_expert_is_skipped(gpu):
    """An id naming a matrix past the weight binding is skipped like SKIP
    (the slot keeps its contents) instead of reading past the buffer."""
    t, rows, cols = 8, 16, 64
    a = np.random.default_rng(3).integers(0, 256, 2 * rows * 2 * 34).astype(np.uint8)
    clamp_f16_exponents(a, 34, (0,))
    x = np.ones(cols, np.float32)
    bd = f32buf(gpu, np.full(2 * rows, 5.0, np.float32))
    ids = gpu.from_numpy(np.array([1, 9], np.int32))
    run(gpu, "mul_mat_vec_id_q8_0_f32_f32",
        [gpu.from_numpy(a), f32buf(gpu, x), bd, gpu.zeros(16), gpu.zeros(16), ids],
        mmv_id_push(cols, rows, 32, 2), (rows, 2, 1))
    got = bd.download(np.float32)
    assert (got[rows:] == 5.0).all()
    assert np.allclose(got[:rows], O.matvec_f64(8, a[rows * 68:], rows, cols, x), rtol=1e-5, atol=1e-5)


def test_mul_mat_vec_q8_0(gpu):
    """ops2.rs:225-292: LCG 0x51ce, 128 x 1024 q8_0, MatVecPush::simple with
    block stride, grid (128, 1, 1); reference tolerance 1e-3 relative, and
    the f32 forward-error bound."""
    r = Lcg(0x51CE)
    a = r.bytes(128 * 32 * 34)
    clamp_f16_exponents(a, 34, (0,))
    x = r.f32s(1024)
    bd = gpu.zeros(128 * 4)
    push = struct.pack("<13I", 1024, 32, 1024, 128, 128 * 1024, 1024, 128, 0, 0, 1, 1, 1, 1)
    run(gpu, "mul_mat_vec_q8_0_f32_f32", [gpu.from_numpy(a), f32buf(gpu, x), bd, gpu.zeros(16),
                                          gpu.zeros(16)], push, (128, 1, 1),
        [(0, 32), (1, 1), (2, 1)])
    got = bd.download(np.float32).astype(np.float64)
    y64 = O.matvec_f64(8, a, 128, 1024, x)
    assert (np.abs(got - y64) <= sum_bound(8, a, 128, 1024, x)).all()
    assert np.max(np.abs(got - y64) / np.maximum(np.abs(y64), 1e-3)) < 1e-3


def test_rms_norm(gpu):
    """kernels.rs:41-122: LCG 0x12345678, 4 rows of 2048, eps 1e-6,
    do_multiply = 0 (spec (1, 0)); reference tolerance 1e-5 absolute."""
    x = Lcg(0x12345678).f32s(2048 * 4)
    dims = lambda n0, n1: [n0, n1, 1, 1, 1, n0, n0 * n1, n0 * n1]
    push = struct.pack("<25I", 2048 * 4, *dims(2048, 4), *dims(2048, 1), *dims(2048, 4)) + \
        struct.pack("<I2fi", 0, 1e-6, 0.0, 0)
    bd = gpu.zeros(2048 * 4 * 4)
    run(gpu, "rms_norm_f32", [f32buf(gpu, x), f32buf(gpu, np.ones(2048)), bd], push, (4, 1, 1),
        [(1, 0)])
    got = bd.download(np.float32).reshape(4, 2048)
    xr = x.reshape(4, 2048).astype(np.float64)
    ref = xr / np.sqrt((xr ** 2).mean(1, keepdims=True) + 1e-6)
    assert np.max(np.abs(got - ref)) < 1e-5
    assert np.max(np.abs(got - O.rms_norm(x, None, 2048, 4, 1e-6).reshape(4, 2048))) < 1e-6


def test_swiglu(gpu):
    """ops2.rs:296-348: LCG 0x5119, gate = 4 * lcg, up = lcg, n = 3072 x 2,
    GluPush::split, grid ceil(n / 512); reference tolerance 1e-5."""
    r = Lcg(0x5119)
    n = 3072 * 2
    g = (r.f32s(n) * np.float32(4.0)).astype(np.float32)
    u = r.f32s(n)
    push = struct.pack("<27I", n, *([0] * 26))  # n first; the other fields are strides
    bd = gpu.zeros(n * 4)
    run(gpu, "swiglu_f32", [f32buf(gpu, g), f32buf(gpu, u), bd], push, ((n + 511) // 512, 1, 1))
    got = bd.download(np.float32)
    gd = g.astype(np.float64)
    assert np.max(np.abs(got - gd / (1 + np.exp(-gd)) * u)) < 1e-5
    assert np.max(np.abs(got - O.swiglu(g, u))) < 1e-6


def test_topk_softmax(gpu):
    """topk_softmax_f32 (shaders/topk_softmax_f32.comp) with its five
    bindings: ids bit-exact against the oracle including the hot / arena /
    host rows, weights within 1e-6 relative; tied logits keep the lower
    index."""
    rng = np.random.default_rng(5)
    E, k = 128, 8
    lg = rng.standard_normal(E).astype(np.float32)
    lg[17] = lg[90] = np.float32(lg.max() + 0.5)          # a tie at the top
    remap = np.full(E, SKIP, np.uint32)
    remap[::3] = np.arange(len(remap[::3]))
    pmap = np.full(E, SKIP, np.uint32)
    pmap[1::3] = 40 + np.arange(len(pmap[1::3]))
    bw, bi = gpu.zeros(64), gpu.from_numpy(np.full(64, -7, np.int32))
    run(gpu, "topk_softmax_f32", [f32buf(gpu, lg), bw, bi, gpu.from_numpy(remap),
                                  gpu.from_numpy(pmap)], struct.pack("<3I", E, k, 1), (1, 1, 1))
    w_ref, ids_ref = O.topk_softmax(lg, k, True, remap, pmap)
    ids = bi.download(np.int32)
    for row in (0, 16, 32, 48):
        assert np.array_equal(ids[row:row + k], ids_ref[row:row + k]), row
    assert ids[0] == 17 and ids[1] == 90
    assert rel_l2(bw.download(np.float32, k), w_ref) < 1e-6


def test_moe_reduce_add_axpy_sig(gpu):
    """moe_reduce_f32 (x += sum_s w_s d_s, s ascending), add_flat_f32 and
    axpy_sig_f32 (shaders/*.comp) against the oracle: the reduce bit for
    bit (same order, no contraction), the sigmoid merge within 2 ulp."""
    rng = np.random.default_rng(6)
    ne, k = 2048, 8
    d = rng.standard_normal(k * ne).astype(np.float32)
    w = rng.random(k).astype(np.float32)
    x = rng.standard_normal(ne).astype(np.float32)
    bx = f32buf(gpu, x)
    run(gpu, "moe_reduce_f32", [f32buf(gpu, d), f32buf(gpu, w), bx], struct.pack("<2I", ne, k),
        ((ne + 255) // 256, 1, 1))
    assert np.array_equal(bx.download(np.float32), O.moe_reduce(d, w, ne, k, x))
    a, b = d[:ne], d[ne:2 * ne]
    bo = gpu.zeros(ne * 4)
    run(gpu, "add_flat_f32", [f32buf(gpu, a), f32buf(gpu, b), bo], struct.pack("<I", ne),
        ((ne + 255) // 256, 1, 1))
    assert np.array_equal(bo.download(np.float32), a + b)
    for g0 in (-3.0, 0.0, 1.7):
        bd = f32buf(gpu, x)
        run(gpu, "axpy_sig_f32", [f32buf(gpu, a), f32buf(gpu, np.array([g0])), bd],
            struct.pack("<I", ne), ((ne + 255) // 256, 1, 1))
        ref = O.axpy_sig(a, g0, x)
        assert np.max(np.abs(bd.download(np.float32) - ref)) <= 2 * np.spacing(np.abs(ref).max())


def test_matvec_strided(gpu):
    """matvec_strided_f32 (the router, shaders/matvec_strided_f32.comp): the
    shader's 32 lane-strided partials and halving tree, as the oracle
    restates them; against the oracle within 1 ulp-scale and f64 within
    the forward-error bound."""
    rng = np.random.default_rng(7)
    E, H = 128, 2048
    W = (0.02 * rng.standard_normal(E * H)).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    bd = gpu.zeros(E * 4)
    run(gpu, "matvec_strided_f32", [f32buf(gpu, W), f32buf(gpu, x), bd], struct.pack("<2I", H, H),
        (E, 1, 1))
    got = bd.download(np.float32)
    ref = O.router_strided(W, x, E, H)
    assert np.max(np.abs(got - ref)) <= 4 * np.spacing(np.abs(ref).max())
    Wd = W.reshape(E, H).astype(np.float64)
    bound = H * 2.0 ** -24 * (np.abs(Wd) @ np.abs(x.astype(np.float64)))
    assert (np.abs(got - Wd @ x.astype(np.float64)) <= bound).all()


@pytest.mark.parametrize("n_t,gqa", [(1, 8), (37, 8), (300, 16)])
def test_attn_decode(gpu, n_t, gqa):
    """attn_decode_f32 (shaders/attn_decode_f32.comp:31-79), one workgroup
    per query head over contiguous f32 K/V rows: against the oracle's f32
    restatement and the f64 two-pass softmax within 1e-5 relative; n_t = 1
    returns the V row."""
    rng = np.random.default_rng(n_t)
    hd, nkv = 128, 4
    nh, kvd = nkv * gqa, nkv * 128
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = rng.standard_normal(n_t * kvd).astype(np.float32)
    V = rng.standard_normal(n_t * kvd).astype(np.float32)
    scale = np.float32(1 / np.sqrt(hd))
    bo = gpu.zeros(nh * hd * 4)
    run(gpu, "attn_decode_f32", [f32buf(gpu, q), f32buf(gpu, K), f32buf(gpu, V), bo],
        struct.pack("<4If", n_t, hd, kvd, gqa, scale), (nh, 1, 1))
    got = bo.download(np.float32)
    assert rel_l2(got, O.attn_decode(q, K, V, n_t, hd, kvd, gqa, nh, scale)) < 1e-6
    assert rel_l2(got, O.attn_decode_f64(q, K, V, n_t, hd, kvd, gqa, nh, float(scale))) < 1e-5
    if n_t == 1:
        for h in range(nh):
            kv = (h // gqa) * hd
            assert np.allclose(got[h * hd:(h + 1) * hd], V[kv:kv + hd], rtol=1e-6)


def test_gather_slabs(gpu):
    """gather_slabs_f32 (shaders/gather_slabs_f32.comp:40-86): slab e of each
    tensor to arena slot layer*k+s, byte-exact against the oracle; SKIP
    slots and every other arena slot untouched."""
    rng = np.random.default_rng(8)
    E, k, layer = 12, 4, 2
    slabs = [4096, 4608, 6144]
    dst_slab = 6144
    src = [rng.integers(0, 256, E * s, dtype=np.uint8) for s in slabs]
    arena0 = [rng.integers(0, 256, (layer + 1) * k * dst_slab, dtype=np.uint8) for _ in range(3)]
    ids = np.array([7, SKIP, 0, 11], np.uint32)
    bsrc = [gpu.from_numpy(a) for a in src]
    bdst = [gpu.from_numpy(a) for a in arena0]
    push = struct.pack("<9I", *[dst_slab // 16] * 3, *[s // 16 for s in slabs], layer, k, 0)
    run(gpu, "gather_slabs_f32", bsrc + bdst + [gpu.from_numpy(ids)], push, (k, 1, 1))
    import ctypes as C
    want = [a.copy() for a in arena0]
    O.lib().styx_oracle_gather_slabs((C.c_void_p * 3)(*[a.ctypes.data for a in src]),
                                     (C.c_int64 * 3)(*slabs),
                                     (C.c_void_p * 3)(*[a.ctypes.data for a in want]),
                                     (C.c_int64 * 3)(dst_slab, dst_slab, dst_slab),
                                     ids.ctypes.data, k, layer)
    for t in range(3):
        got = bdst[t].download()
        assert np.array_equal(got, want[t]), t
        assert not np.array_equal(got, arena0[t])


def test_dispatch_rejects_reach_past_binding(gpu):
    """Push constants or a grid that would read or write past a binding are
    refused on the host (nothing is launched): a matvec whose rows exceed
    the weight buffer, a reduce longer than its output."""
    from styx_amd import _lib as L
    a = np.zeros(16 * 2 * 34, np.uint8)
    push = struct.pack("<13I", 64, 2, 64, 32, 32 * 64, 64, 32, 0, 0, 1, 1, 1, 1)  # 32 rows, 16 stored
    with pytest.raises(L.StyxError, match="reach past"):
        run(gpu, "mul_mat_vec_q8_0_f32_f32", [gpu.from_numpy(a), gpu.zeros(256), gpu.zeros(128),
                                              gpu.zeros(16), gpu.zeros(16)], push, (32, 1, 1))
    with pytest.raises(L.StyxError, match="reach past"):
        run(gpu, "moe_reduce_f32", [gpu.zeros(8 * 1024 * 4), gpu.zeros(32), gpu.zeros(512 * 4)],
            struct.pack("<2I", 1024, 8), (4, 1, 1))


def test_async_batch_and_timeline(gpu):
    """The M7b-B surface (lib.rs:233-333, moe.rs:2093,2370-2375): an async
    batch gathers slabs on its own stream and signals a timeline; the main
    batch waits for that value, then adds the gathered slab to a vector.
    The result equals the serial order's; the timeline reaches each
    signalled value; signal values must increase; a wait for a value no one
    signalled and submit_async on a plain batch are refused."""
    from styx_amd import StyxError
    from styx_amd.runtime import Batch, Kernel, Timeline
    rng = np.random.default_rng(12)
    E, k, slab = 4, 1, 1 << 20  # one 1 MiB slab per tensor
    # finite f32 values as bytes (the add must not meet NaN payloads)
    src = [rng.standard_normal(E * slab // 4).astype(np.float32).view(np.uint8) for _ in range(3)]
    bsrc = [gpu.from_numpy(a) for a in src]
    bdst = [gpu.zeros(k * slab) for _ in range(3)]
    other = rng.standard_normal(slab // 4).astype(np.float32)
    bo, bsum = f32buf(gpu, other), gpu.zeros(slab)
    t = Timeline(gpu)
    gk = Kernel(gpu, "gather_slabs_f32", [])
    ak = Kernel(gpu, "add_flat_f32", [])
    ab, mb = Batch(gpu, is_async=True), Batch(gpu)
    ne = slab // 4
    for rnd, e in enumerate([3, 1]):
        ids = gpu.from_numpy(np.array([e], np.uint32))
        ab.begin()
        ab.dispatch(gk, bsrc + bdst + [ids],
                    struct.pack("<9I", *[slab // 16] * 6, 0, k, 0), (k, 1, 1))
        ab.submit_async(t, rnd + 1)
        mb.begin()
        mb.dispatch(ak, [bdst[0], bo, bsum], struct.pack("<I", ne), ((ne + 255) // 256, 1, 1))
        mb.submit_wait_sem(t, rnd + 1)
        ab.wait_idle()
        assert t.value() == rnd + 1
        want = src[0][e * slab:(e + 1) * slab].view(np.float32) + other
        got = bsum.download(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rnd
        for i in range(3):
            assert np.array_equal(bdst[i].download(), src[i][e * slab:(e + 1) * slab])
    ab.begin()
    ab.dispatch(gk, bsrc + bdst + [gpu.from_numpy(np.array([0], np.uint32))],
                struct.pack("<9I", *[slab // 16] * 6, 0, k, 0), (k, 1, 1))
    with pytest.raises(StyxError):
        ab.submit_async(t, 2)  # not above the last signalled value
    mb.begin()
    mb.dispatch(ak, [bdst[0], bo, bsum], struct.pack("<I", ne), ((ne + 255) // 256, 1, 1))
    with pytest.raises(StyxError):
        mb.submit_wait_sem(t, 9)  # never signalled
    with pytest.raises(StyxError):
        mb.submit_async(t, 9)  # a plain batch has no async stream
    for o in (ab, mb, gk, ak, t):
        o.free()


def rope_push(head_dim, n_heads, n_tokens, base):
    # RopePush::neox (ops.rs:413-439): 116 bytes
    ts = np.float32(np.float64(base) ** (-2.0 / head_dim))
    return struct.pack("<3I4f2ffI4i3I3I3I3I2I", 2, n_heads * n_tokens, head_dim, 1.0, base, 0.0,
                       1.0, 0.0, 0.0, ts, 0, 0, 0, 0, 0, 0, 0, 0, head_dim, n_heads, n_tokens,
                       head_dim, head_dim * n_heads, head_dim * n_heads * n_tokens, head_dim,
                       head_dim * n_heads, head_dim * n_heads * n_tokens, 0, 0)


def test_rope_neox(gpu):
    """rope_neox_f32 (ops2.rs:413-490): head_dim 128, 4 heads, 3 tokens at
    positions [0, 5, 17], base 1e6, LCG 0x40e0 inputs; against the test's
    f64 CPU formula within its 1e-4 (and within 1e-6 here), position 0 the
    identity bit for bit; the rotation composes: rotating by 5 then by 12
    equals rotating by 17 (1e-6)."""
    hd, nh, nt = 128, 4, 3
    pos = np.array([0, 5, 17], np.int32)
    x = Lcg(0x40E0).f32s(hd * nh * nt)
    half = hd // 2
    ts = np.float64(1e6) ** (-2.0 / hd)
    th = pos[:, None].astype(np.float64) * ts ** np.arange(half, dtype=np.float64)[None, :]
    xr = x.reshape(nt, nh, hd).astype(np.float64)
    c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    want = np.concatenate([xr[..., :half] * c - xr[..., half:] * s,
                           xr[..., :half] * s + xr[..., half:] * c], -1).astype(np.float32).ravel()
    bo = gpu.zeros(x.nbytes)
    binds = [f32buf(gpu, x), gpu.from_numpy(pos), gpu.zeros(16), bo, gpu.zeros(16)]
    run(gpu, "rope_neox_f32", binds, rope_push(hd, nh, nt, 1e6), (nh * nt, 1, 1))
    got = bo.download(np.float32)
    assert np.max(np.abs(got - want)) < 1e-6
    assert np.array_equal(got[:hd * nh].view(np.uint32), x[:hd * nh].view(np.uint32))
    # composition through single dispatches of one token each
    # (Gpu::dispatch_sync, lib.rs:1415)
    from styx_amd.runtime import Kernel, dispatch_sync
    k = Kernel(gpu, "rope_neox_f32", [])
    y = x[:hd * nh]
    b1, b2 = gpu.zeros(y.nbytes), gpu.zeros(y.nbytes)
    one = rope_push(hd, nh, 1, 1e6)
    dispatch_sync(gpu, k, [f32buf(gpu, y), gpu.from_numpy(np.array([5], np.int32)),
                           gpu.zeros(16), b1, gpu.zeros(16)], one, (nh, 1, 1))
    dispatch_sync(gpu, k, [b1, gpu.from_numpy(np.array([12], np.int32)), gpu.zeros(16), b2,
                           gpu.zeros(16)], one, (nh, 1, 1))
    dispatch_sync(gpu, k, [f32buf(gpu, y), gpu.from_numpy(np.array([17], np.int32)),
                           gpu.zeros(16), b1, gpu.zeros(16)], one, (nh, 1, 1))
    assert np.max(np.abs(b2.download(np.float32) - b1.download(np.float32))) < 1e-6
    k.free()


def unary_push(ne, src0, dst, misalign):
    # UnaryPush (ops.rs:253-273): 120 bytes; the fastdiv words are unused here
    return struct.pack("<I8I8II4f8I", ne, *src0, *dst, misalign, 0, 0, 0, 0, *([0] * 8))


def test_cpy_contig_and_strided(gpu):
    """cpy_f32_f32 with UnaryPush::contig_copy into a KV row at a binding
    offset (moe.rs:1935-1943: the KV append), and strided_copy(n, stride,
    off): exact copies, everything else untouched."""
    rng = np.random.default_rng(21)
    kvd, pos = 512, 3
    src = rng.standard_normal(kvd).astype(np.float32)
    cache0 = rng.standard_normal(8 * kvd).astype(np.float32)
    bc = f32buf(gpu, cache0)
    run(gpu, "cpy_f32_f32", [f32buf(gpu, src), (bc, pos * kvd * 4, 2**64 - 1)],
        unary_push(kvd, [kvd, 1, 1, 1, 1, kvd, kvd, kvd], [kvd, 1, 1, 1, 1, kvd, kvd, kvd], 0),
        ((kvd + 511) // 512, 1, 1))
    want = cache0.copy()
    want[pos * kvd:(pos + 1) * kvd] = src
    assert np.array_equal(bc.download(np.float32), want)
    n, stride, off = 100, 3, 7
    d0 = np.full(off + n * stride + 5, -1.0, np.float32)
    bd = f32buf(gpu, d0)
    run(gpu, "cpy_f32_f32", [f32buf(gpu, src[:n]), bd],
        unary_push(n, [n, 1, 1, 1, 1, n, n, n],
                   [n, 1, 1, 1, stride, n * stride, n * stride, n * stride], off), (1, 1, 1))
    want = d0.copy()
    want[off:off + n * stride:stride] = src[:n]
    assert np.array_equal(bd.download(np.float32), want)


# ------------------------------------------------------------ fused names --
# The fused kernels registered under their own names (moe_gate_up_silu_{t},
# moe_down_reduce_{t}, router_topk, attn_decode_paged), dispatched through
# styx_batch_dispatch with their push blocks (include/styx_hip.h), checked
# against the oracle's MoE block and attention.  Quant weights in the split
# layout (styx_op_to_split), as the fused path reads them.

def _push(cls, **kw) -> bytes:
    import ctypes
    from styx_amd import _lib as L
    p = getattr(L, cls)(**kw)
    return ctypes.string_at(ctypes.addressof(p), ctypes.sizeof(p))


def _experts(gpu, t, E, rows, cols, seed):
    """E seeded slabs of type t: (split-layout device buffer, GGUF host bytes)."""
    import ctypes
    from styx_amd import _lib as L
    from styx_amd.runtime import to_split
    be, bb = BLK[t]
    b = gpu.buffer(E * rows * cols // be * bb)
    L.check(gpu.lib.styx_op_gen_quant(gpu.h, t, seed, ctypes.c_float(0.02), b.ptr, E * rows * cols))
    host = b.download()
    sp = to_split(gpu, t, b, rows, cols, E)
    b.free()
    return sp, host


@pytest.mark.parametrize("types,H,F,E,k", [((12, 13, 14), 2048, 768, 32, 8),
                                           ((8, 8, 8), 1024, 512, 16, 4),
                                           ((12, 12, 14), 2048, 512, 64, 10)])
def test_fused_moe_block_dispatch(gpu, types, H, F, E, k):
    """router_topk -> moe_gate_up_silu_{t} -> moe_down_reduce_{t} as three
    dispatches of one batch (moe.rs:1975-2062 in three calls) against the
    oracle: ids bit-exact, h and the updated residual within 1e-5 relative
    L2; a SKIP id leaves its h row untouched; two down launches over
    disjoint id rows (hot then cold) add what one launch over all slots adds."""
    from styx_amd.runtime import Batch, Kernel
    tg, tu, td = types
    rng = np.random.default_rng(H + F + E)
    x = rng.standard_normal(H).astype(np.float32)
    nw = (1 + 0.05 * rng.standard_normal(H)).astype(np.float32)
    W = (0.02 * rng.standard_normal((E, H))).astype(np.float32)
    gsp, gh = _experts(gpu, tg, E, F, H, 11 * E + 1)
    usp, uh = _experts(gpu, tu, E, F, H, 11 * E + 2)
    dsp, dh = _experts(gpu, td, E, H, F, 11 * E + 3)
    xb, nwb, Wb = f32buf(gpu, x), f32buf(gpu, nw), f32buf(gpu, W)
    xn, lg, wts, ids = gpu.buffer(H * 4), gpu.buffer(E * 4), gpu.buffer(64), gpu.buffer(256)
    sentinel = np.full(k * F, 3.0, np.float32)
    hb = f32buf(gpu, sentinel)
    dummy = gpu.zeros(256)
    kr = Kernel(gpu, "router_topk", [])
    kg = Kernel(gpu, f"moe_gate_up_silu_{NAME[tg]}", [])
    kd = Kernel(gpu, f"moe_down_reduce_{NAME[td]}", [])
    b = Batch(gpu)
    b.begin()
    b.dispatch(kr, [xb, nwb, Wb, dummy, dummy, dummy, xn, lg, wts, ids],
               _push("PushRouterTopk", E=E, H=H, k=k, renorm=1, arena_mode=0, layer=0, eps=1e-6,
                     flags=0), (1, 1, 1))
    b.dispatch(kg, [gsp, usp, xn, (ids, 0, 4 * k), hb],
               _push("PushGateUpSilu", H=H, F=F, k=k, type_up=tu, n_slabs=E), (1, 1, 1))
    b.submit()
    # oracle on the same routing
    xn_ref = O.rms_norm(x, nw, H, 1, 1e-6)
    w_ref, ids_ref = O.topk_softmax(lg.download(np.float32), k, True)
    idh = ids.download(np.int32)
    assert np.array_equal(idh[:k], ids_ref[:k]) and np.array_equal(idh[16:16 + k], ids_ref[:k])
    sel = ids_ref[:k].astype(np.uint32)
    g = O.matvec_id(tg, gh, F, H, len(gh) // E, sel, xn_ref, 1)
    u = O.matvec_id(tu, uh, F, H, len(uh) // E, sel, xn_ref, 1)
    h_ref = O.swiglu(g, u)
    h = hb.download(np.float32)
    assert rel_l2(h, h_ref) < 1e-5
    d = O.matvec_id(td, dh, H, F, len(dh) // E, sel, h_ref, k)
    x_ref = O.moe_reduce(d, w_ref, H, k, x)
    b.begin()
    b.dispatch(kd, [dsp, hb, (ids, 0, 4 * k), wts, xb],
               _push("PushDownReduce", H=H, F=F, k=k, n_slabs=E), (1, 1, 1))
    b.submit()
    assert rel_l2(xb.download(np.float32) - x, x_ref - x) < 1e-5
    # hot / cold split over disjoint id rows adds the same
    half = k // 2
    hot = np.where(np.arange(k) < half, idh[:k], -1).astype(np.int32)
    cold = np.where(np.arange(k) >= half, idh[:k], -1).astype(np.int32)
    hotb, coldb = gpu.from_numpy(hot), gpu.from_numpy(cold)
    xb.upload(x)
    b.begin()
    for rowb in (hotb, coldb):
        b.dispatch(kd, [dsp, hb, rowb, wts, xb],
                   _push("PushDownReduce", H=H, F=F, k=k, n_slabs=E), (1, 1, 1))
    b.submit()
    assert rel_l2(xb.download(np.float32) - x, x_ref - x) < 1e-5
    # a SKIP (and an id past n_slabs) leaves h untouched
    skip = idh[:k].copy()
    skip[1] = -1
    skip[k - 1] = E + 5
    sb = gpu.from_numpy(skip.astype(np.int32))
    hb.upload(sentinel)
    b.begin()
    b.dispatch(kg, [gsp, usp, xn, sb, hb],
               _push("PushGateUpSilu", H=H, F=F, k=k, type_up=tu, n_slabs=E), (1, 1, 1))
    b.submit()
    h2 = hb.download(np.float32).reshape(k, F)
    assert (h2[1] == 3.0).all() and (h2[k - 1] == 3.0).all()
    assert rel_l2(h2[0], h_ref.reshape(k, F)[0]) < 1e-5
    b.free()
    for kk in (kr, kg, kd):
        kk.free()


@pytest.mark.parametrize("paged", [False, True])
def test_fused_attn_decode_paged(gpu, paged):
    """attn_decode_paged (moe.rs:1875-1964 in one dispatch: q/k norm, rope,
    K/V append at pos, split-context attention) over the reference's
    contiguous caches or a scrambled page table, 40 positions, against the
    f64 oracle at 2e-6 relative L2; the appended rows land at their
    addresses."""
    import ctypes
    from styx_amd.runtime import Batch, Kernel
    nh, nkv, hd, n_steps, page, max_chunks = 32, 4, 128, 40, 16, 4
    rng = np.random.default_rng(77 + paged)
    kvd, n_ctx, base = nkv * hd, 64, 1e6
    npages = n_ctx // page
    pt = rng.permutation(npages).astype(np.int32)
    kpool, vpool = gpu.zeros(n_ctx * kvd * 4), gpu.zeros(n_ctx * kvd * 4)
    rope = np.empty((n_ctx, hd // 2, 2), np.float64)
    gpu.lib.styx_rope_table(ctypes.c_float(base), hd, n_ctx, rope.ctypes.data)
    ropeb, ptb = gpu.from_numpy(rope), gpu.from_numpy(pt)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    qnb, knb = f32buf(gpu, qn), f32buf(gpu, kn)
    part = gpu.buffer(gpu.lib.styx_op_attn_part_floats(nh, nkv, hd, max_chunks) * 4)
    out = gpu.buffer(nh * hd * 4)
    kern = Kernel(gpu, "attn_decode_paged", [])
    b = Batch(gpu)
    K = np.zeros((n_ctx, kvd), np.float32)
    V = np.zeros((n_ctx, kvd), np.float32)
    scale = 1.0 / np.sqrt(hd)

    def nr(v, w, n, pos):
        return O.rope_neox(O.rms_norm(v, w, hd, n, 1e-6), hd, n, pos, base)
    for pos in range(n_steps):
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k = rng.standard_normal(kvd).astype(np.float32)
        v = rng.standard_normal(kvd).astype(np.float32)
        b.begin()
        b.dispatch(kern, [f32buf(gpu, q), f32buf(gpu, k), f32buf(gpu, v), qnb, knb, ropeb, kpool,
                          vpool, ptb, out, part],
                   _push("PushAttnPaged", eps=1e-6, page_tokens=page, nh=nh, nkv=nkv, hd=hd,
                         chunk=16, max_chunks=max_chunks, scale=scale,
                         flags=3 | (4 if paged else 0), pos=pos), (1, 1, 1))
        b.submit()
        K[pos] = nr(k, kn, nkv, pos)
        V[pos] = v
        ref = O.attn_decode_f64(nr(q, qn, nh, pos), K, V, pos + 1, hd, kvd, nh // nkv, nh, scale)
        assert rel_l2(out.download(np.float32), ref) < 2e-6, pos
    kp = kpool.download(np.float32).reshape(n_ctx, kvd)
    vp = vpool.download(np.float32).reshape(n_ctx, kvd)
    for t in range(n_steps):
        row = pt[t // page] * page + t % page if paged else t
        np.testing.assert_allclose(kp[row], K[t], rtol=2e-6, atol=2e-6)
        assert np.array_equal(vp[row], V[t]), t
    b.free()
    kern.free()


def test_fused_attn_page_entries_clamped_to_pool(gpu):
    """A page-table entry past the pool reads (and appends to) the pool's
    last page instead of memory outside it: the result equals the table
    with that entry replaced by the last page."""
    import ctypes
    from styx_amd.runtime import Batch, Kernel
    nh, nkv, hd, page = 8, 2, 64, 16
    kvd, n_ctx, base = nkv * hd, 32, 1e6
    rng = np.random.default_rng(5)
    rope = np.empty((n_ctx, hd // 2, 2), np.float64)
    gpu.lib.styx_rope_table(ctypes.c_float(base), hd, n_ctx, rope.ctypes.data)
    ropeb = gpu.from_numpy(rope)
    q, k, v = (rng.standard_normal(n).astype(np.float32) for n in (nh * hd, kvd, kvd))
    pools = rng.standard_normal(n_ctx * kvd).astype(np.float32)
    kern = Kernel(gpu, "attn_decode_paged", [])
    outs = []
    for table in ([0, 2 ** 31 - 1], [0, 1]):
        kp, vp = f32buf(gpu, pools), f32buf(gpu, pools[::-1].copy())
        out, part = gpu.buffer(nh * hd * 4), gpu.buffer(
            gpu.lib.styx_op_attn_part_floats(nh, nkv, hd, 2) * 4)
        b = Batch(gpu)
        b.begin()
        b.dispatch(kern, [f32buf(gpu, q), f32buf(gpu, k), f32buf(gpu, v), gpu.zeros(256),
                          gpu.zeros(256), ropeb, kp, vp, gpu.from_numpy(np.array(table, np.int32)),
                          out, part],
                   _push("PushAttnPaged", eps=1e-6, page_tokens=page, nh=nh, nkv=nkv, hd=hd,
                         chunk=16, max_chunks=2, scale=0.125, flags=4, pos=20), (1, 1, 1))
        b.submit()
        b.free()
        outs.append(out.download(np.float32))
    assert np.array_equal(outs[0], outs[1])
    kern.free()


def test_fused_rejects_reach_past_binding(gpu):
    """A fused dispatch whose push block implies more bytes than a binding
    makes visible is refused before anything launches."""
    from styx_amd import _lib as L
    from styx_amd.runtime import Batch, Kernel
    H, E, k = 512, 16, 4
    small = gpu.zeros(64)
    big = gpu.zeros(E * H * 4)
    kr = Kernel(gpu, "router_topk", [])
    b = Batch(gpu)
    b.begin()
    b.dispatch(kr, [small, big, big, big, big, big, big, big, big, big],
               _push("PushRouterTopk", E=E, H=H, k=k, renorm=1, arena_mode=0, layer=0, eps=1e-6,
                     flags=0), (1, 1, 1))
    with pytest.raises(L.StyxError) as ei:
        b.submit()
    assert ei.value.status == -1
    b.free()
    kr.free()
