"""styx_op_attn_decode_noalloc (no counterpart in the reference: the
attention op for callers that cannot allocate) against styx_op_attn_decode
with a caller-allocated workspace, through the C ABI: two calls in a row,
the second smaller (fewer heads, a shorter context, fewer chunks), outputs
and appended K/V rows bit-identical (same kernels, same arithmetic); a
request past the static array is refused before anything is launched."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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


def one_call(gpu, rng, nh, nkv, hd, n_t, page, max_chunks):
    """Attention for the token at position n_t - 1 over n_t - 1 seeded
    context rows plus the appended one, through the workspace entry and the
    no-allocation entry on identical buffers: [(out, K pool, V pool)] x 2."""
    kvd = nkv * hd
    n_ctx = n_t + 16
    npages = -(-n_ctx // page)
    pt = np.random.default_rng(n_t).permutation(npages).astype(np.int32)
    kp = rng.standard_normal(npages * page * kvd).astype(np.float32)
    vp = rng.standard_normal(npages * page * kvd).astype(np.float32)
    rope = np.empty((n_ctx, hd // 2, 2), np.float64)
    lib().styx_rope_table(C.c_float(1e6), hd, n_ctx, rope.ctypes.data)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(kvd).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    res = []
    for use_noalloc in (False, True):
        b = [gpu.from_numpy(a) for a in (q, k, v, qn, kn, rope, kp, vp, pt,
                                         np.array([n_t - 1], np.int32))]
        out = gpu.buffer(nh * hd * 4)
        args = [gpu.h, b[0].ptr, b[1].ptr, b[2].ptr, b[3].ptr, b[4].ptr, C.c_float(1e-6), b[5].ptr,
                b[6].ptr, b[7].ptr, b[8].ptr, page, b[9].ptr, out.ptr]
        tail = [nh, nkv, hd, 16, max_chunks, C.c_float(1 / np.sqrt(hd))]
        if use_noalloc:
            check(lib().styx_op_attn_decode_noalloc(*args, *tail))
        else:
            part = gpu.buffer(lib().styx_op_attn_part_floats(nh, nkv, hd, max_chunks) * 4)
            check(lib().styx_op_attn_decode(*args, part.ptr, *tail))
        gpu.sync()
        res.append((out.download(np.float32), b[6].download(np.float32), b[7].download(np.float32)))
    return res


def test_noalloc_matches_workspace_entry_twice(gpu):
    rng = np.random.default_rng(0xA11)
    # first: gqa 16 (matrix-core kernel), 700 tokens over 64-token pages,
    # 64 chunks; second, smaller: gqa 8, 45 tokens, 4 chunks
    for nh, nkv, hd, n_t, page, mc in [(64, 4, 128, 700, 64, 64), (32, 4, 128, 45, 32, 4)]:
        (o_ref, k_ref, v_ref), (o_na, k_na, v_na) = one_call(gpu, rng, nh, nkv, hd, n_t, page, mc)
        assert np.isfinite(o_ref).all() and np.abs(o_ref).max() > 0
        assert np.array_equal(o_na.view(np.uint32), o_ref.view(np.uint32)), (nh, n_t)
        assert np.array_equal(k_na, k_ref) and np.array_equal(v_na, v_ref), (nh, n_t)


def test_noalloc_rejects_partials_past_the_static_array(gpu):
    nh, nkv, hd = 64, 8, 256
    mc = 4096  # 8 * 4096 * 8 * 258 floats, past 2 Mi
    assert lib().styx_op_attn_part_floats(nh, nkv, hd, mc) > (2 << 20)
    z = gpu.zeros(64)
    rc = lib().styx_op_attn_decode_noalloc(gpu.h, z.ptr, z.ptr, z.ptr, None, None, C.c_float(1e-6),
                                           z.ptr, z.ptr, z.ptr, z.ptr, 512, z.ptr, z.ptr, nh, nkv,
                                           hd, 16, mc, C.c_float(0.1))
    assert rc == -1  # STYX_E_INVALID
    assert "exceed the static scratch" in lib().styx_last_error().decode()
