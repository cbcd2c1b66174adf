"""The C-ABI library loads and exports every entry point include/styx_hip.h
declares; the product package never reaches into the oracle; without the
library the package fails loudly (no CPU fallback).  No GPU needed."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def declared_functions() -> list[str]:
    hdr = (ROOT / "include" / "styx_hip.h").read_text()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    return sorted(set(re.findall(r"\b(styx_[a-z0-9_]+)\s*\(", hdr)))


def test_exports_every_declared_symbol():
    from styx_amd import _lib
    lib = C.CDLL(str(_lib.LIB_PATH))
    names = declared_functions()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python bindings cover all of them
    assert set(names) <= set(_lib.EXPORTED), set(names) - set(_lib.EXPORTED)


def test_gpu_calls_fail_cleanly_without_device():
    """On a machine without the GPU, device entry points return an error
    status with a message instead of aborting."""
    from styx_amd import _lib
    lib = _lib.load()
    h = C.c_void_p()
    rc = lib.styx_gpu_new(0, C.byref(h))
    if rc == 0:  # running on the GPU box
        lib.styx_gpu_free(h)
        return
    assert rc < 0 and lib.styx_last_error().decode()


def test_kernel_names_cover_reference_pipelines():
    from styx_amd import _lib
    names = _lib.load().styx_kernel_names().decode().split(",")
    for n in ("topk_softmax_f32", "moe_reduce_f32", "gather_slabs_f32", "attn_decode_f32",
              "matvec_strided_f32", "add_flat_f32", "axpy_sig_f32", "swiglu_f32",
              "rms_norm_f32", "mul_mat_vec_id_q4_k_f32_f32", "mul_mat_vec_q8_0_f32_f32"):
        assert n in names


def test_product_never_imports_oracle():
    for p in (ROOT / "styx_amd").rglob("*.py"):
        src = p.read_text()
        assert "oracle" not in re.sub(r'""".*?"""|#.*', "", src, flags=re.S), p
    for p in (ROOT / "styx_amd" / "csrc").iterdir():
        assert "styx_oracle" not in p.read_text(), p


def test_missing_library_fails_loudly(tmp_path):
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from styx_amd import _lib\n"
            "try:\n    _lib.load(%r)\nexcept RuntimeError as e:\n    print('refused', e)\n") % (
        str(ROOT), str(tmp_path / "nope.so"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True)
    assert "refused" in out.stdout and "no fallback" in out.stdout


def test_rope_table_matches_oracle_rotation():
    """styx_rope_table (host, no GPU) holds the f64 (cos, sin) the oracle's
    rope_neox evaluates (ops2.rs:426-442): rotating with the table in f64 and
    rounding to f32 reproduces the oracle bit for bit."""
    import numpy as np
    from oracle import oracle as O
    from styx_amd._lib import load
    lib = load
    hd, n_pos, base = 128, 300, 1e6
    tab = np.empty((n_pos, hd // 2, 2), np.float64)
    lib().styx_rope_table(C.c_float(base), hd, n_pos, tab.ctypes.data)
    assert np.array_equal(tab[0, :, 0], np.ones(hd // 2)) and not tab[0, :, 1].any()
    assert np.allclose(tab[..., 0] ** 2 + tab[..., 1] ** 2, 1.0, atol=1e-15)
    rng = np.random.default_rng(4)
    for pos in (1, 17, 299):
        x = rng.standard_normal(2 * hd).astype(np.float32)
        half = hd // 2
        got = np.empty_like(x)
        for h in range(2):
            x0 = x[h * hd:h * hd + half].astype(np.float64)
            x1 = x[h * hd + half:(h + 1) * hd].astype(np.float64)
            c, s = tab[pos, :, 0], tab[pos, :, 1]
            got[h * hd:h * hd + half] = (x0 * c - x1 * s).astype(np.float32)
            got[h * hd + half:(h + 1) * hd] = (x0 * s + x1 * c).astype(np.float32)
        assert np.array_equal(got, O.rope_neox(x, hd, 2, pos, base))
