"""ctypes loader of the CPU oracle (libstyx_oracle.so, built by oracle/Makefile).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the parity checker or the timed CPU baseline.
The product path (styx_amd / libstyx_hip.so) never loads it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libstyx_oracle.so"
SKIP = 0xFFFFFFFF


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


class Mat(C.Structure):
    _fields_ = [("type", C.c_int), ("nrows", C.c_int), ("ncols", C.c_int), ("data", C.c_void_p)]


class Layer(C.Structure):
    _fields_ = [
        ("attn_norm", C.c_void_p), ("q_norm", C.c_void_p), ("k_norm", C.c_void_p),
        ("ffn_norm", C.c_void_p), ("wq", Mat), ("wk", Mat), ("wv", Mat), ("wo", Mat),
        ("router", C.c_void_p), ("router_bias", C.c_void_p),
        ("gate_exps", Mat), ("up_exps", Mat), ("down_exps", Mat),
        ("gate_sh", Mat), ("up_sh", Mat), ("down_sh", Mat), ("gate_inp_sh", C.c_void_p),
    ]


class Model(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("n_embd", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("n_expert", C.c_int),
        ("n_expert_used", C.c_int), ("n_ff_exp", C.c_int), ("n_ff_sh", C.c_int),
        ("n_vocab", C.c_int), ("n_ctx", C.c_int), ("rms_eps", C.c_float),
        ("rope_base", C.c_float), ("norm_topk", C.c_int), ("layers", C.POINTER(Layer)),
        ("output_norm", C.c_void_p), ("output", Mat), ("token_embd", Mat),
        ("kcache", C.c_void_p), ("vcache", C.c_void_p),
    ]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
        vp, i, i64, f = C.c_void_p, C.c_int, C.c_int64, C.c_float
        sigs = {
            "styx_oracle_set_threads": (None, [i]),
            "styx_oracle_f16_to_f32": (f, [C.c_uint16]),
            "styx_oracle_dequant": (i, [i, vp, i64, vp]),
            "styx_oracle_matvec": (i, [i, vp, i, i, vp, vp]),
            "styx_oracle_matvec_f64": (i, [i, vp, i, i, vp, vp]),
            "styx_oracle_matvec_id": (i, [i, vp, i, i, i64, vp, i, vp, i, vp]),
            "styx_oracle_rms_norm": (None, [vp, vp, i, i, f, vp]),
            "styx_oracle_router_strided": (None, [vp, vp, i, i, i, vp]),
            "styx_oracle_topk_softmax": (None, [vp, i, i, i, vp, vp, vp, vp]),
            "styx_oracle_swiglu": (None, [vp, vp, i, vp]),
            "styx_oracle_moe_reduce": (None, [vp, vp, i, i, vp]),
            "styx_oracle_axpy_sig": (None, [vp, f, i, vp]),
            "styx_oracle_rope_neox": (None, [vp, i, i, i, f]),
            "styx_oracle_attn_decode": (None, [vp, vp, vp, i, i, i, i, i, f, vp]),
            "styx_oracle_attn_decode_f64": (None, [vp, vp, vp, i, i, i, i, i, C.c_double, vp]),
            "styx_oracle_moe_block": (i, [vp, i, vp, vp, vp, vp, vp]),
            "styx_oracle_forward": (i, [vp, i, C.c_uint32, vp, vp, vp, vp]),
            "styx_oracle_argmax": (C.c_uint32, [vp, i]),
            "styx_oracle_gather_slabs": (None, [vp, vp, vp, vp, vp, i, i]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(_lib, name)
            fn.restype, fn.argtypes = res, args
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def set_threads(n: int) -> None:
    lib().styx_oracle_set_threads(n)


def dequant(type_: int, blocks: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    rc = lib().styx_oracle_dequant(C.c_int(type_), _p(np.ascontiguousarray(blocks)), C.c_int64(n),
                                   _p(out))
    if rc:
        raise ValueError("dequant: bad type/size")
    return out


def matvec(type_: int, w: np.ndarray, nrows: int, ncols: int, x: np.ndarray) -> np.ndarray:
    y = np.empty(nrows, np.float32)
    rc = lib().styx_oracle_matvec(C.c_int(type_), _p(np.ascontiguousarray(w)), nrows, ncols,
                                  _p(np.ascontiguousarray(x, np.float32)), _p(y))
    if rc:
        raise ValueError("matvec: bad type/size")
    return y


def matvec_f64(type_: int, w: np.ndarray, nrows: int, ncols: int, x: np.ndarray) -> np.ndarray:
    y = np.empty(nrows, np.float64)
    rc = lib().styx_oracle_matvec_f64(C.c_int(type_), _p(np.ascontiguousarray(w)), nrows, ncols,
                                      _p(np.ascontiguousarray(x, np.float32)), _p(y))
    if rc:
        raise ValueError("matvec_f64: bad type/size")
    return y


def matvec_id(type_, w, nrows, ncols, expert_stride, ids, x, ne11, y=None):
    ids = np.ascontiguousarray(ids, np.uint32)
    if y is None:
        y = np.zeros(len(ids) * nrows, np.float32)
    rc = lib().styx_oracle_matvec_id(C.c_int(type_), _p(np.ascontiguousarray(w)), nrows, ncols,
                                     C.c_int64(expert_stride), _p(ids), len(ids),
                                     _p(np.ascontiguousarray(x, np.float32)), ne11, _p(y))
    if rc:
        raise ValueError("matvec_id failed")
    return y


def rms_norm(x, w, ncols, nrows, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().styx_oracle_rms_norm(_p(x), _p(None if w is None else np.ascontiguousarray(w, np.float32)),
                               ncols, nrows, C.c_float(eps), _p(out))
    return out


def router_strided(W, x, nrows, ncols):
    out = np.empty(nrows, np.float32)
    lib().styx_oracle_router_strided(_p(np.ascontiguousarray(W, np.float32)),
                                     _p(np.ascontiguousarray(x, np.float32)), nrows, ncols, ncols,
                                     _p(out))
    return out


def topk_softmax(logits, k, renorm=True, remap=None, pmap=None):
    logits = np.ascontiguousarray(logits, np.float32)
    w = np.empty(k, np.float32)
    ids = np.full(64, -1, np.int32)
    r = None if remap is None else np.ascontiguousarray(remap, np.uint32)
    pm = None if pmap is None else np.ascontiguousarray(pmap, np.uint32)
    lib().styx_oracle_topk_softmax(_p(logits), len(logits), k, int(renorm), _p(r), _p(pm), _p(w),
                                   _p(ids))
    return w, ids


def swiglu(g, u):
    g = np.ascontiguousarray(g, np.float32)
    out = np.empty_like(g)
    lib().styx_oracle_swiglu(_p(g), _p(np.ascontiguousarray(u, np.float32)), len(g), _p(out))
    return out


def moe_reduce(d, w, ne, k, x):
    x = np.array(x, np.float32, copy=True)
    lib().styx_oracle_moe_reduce(_p(np.ascontiguousarray(d, np.float32)),
                                 _p(np.ascontiguousarray(w, np.float32)), ne, k, _p(x))
    return x


def axpy_sig(a, g0, d):
    """d + sigmoid(g0) * a (shaders/axpy_sig_f32.comp:7-11); returns a new array."""
    d = np.array(d, np.float32, copy=True)
    a = np.ascontiguousarray(a, np.float32)
    lib().styx_oracle_axpy_sig(_p(a), C.c_float(g0), len(d), _p(d))
    return d


def rope_neox(x, hd, nh, pos, base):
    x = np.array(x, np.float32, copy=True)
    lib().styx_oracle_rope_neox(_p(x), hd, nh, pos, C.c_float(base))
    return x


def attn_decode(q, K, V, n_t, hd, kv_dim, gqa, n_heads, scale):
    out = np.empty(n_heads * hd, np.float32)
    lib().styx_oracle_attn_decode(_p(np.ascontiguousarray(q, np.float32)),
                                  _p(np.ascontiguousarray(K, np.float32)),
                                  _p(np.ascontiguousarray(V, np.float32)), n_t, hd, kv_dim, gqa,
                                  n_heads, C.c_float(scale), _p(out))
    return out


def attn_decode_f64(q, K, V, n_t, hd, kv_dim, gqa, n_heads, scale):
    out = np.empty(n_heads * hd, np.float64)
    lib().styx_oracle_attn_decode_f64(_p(np.ascontiguousarray(q, np.float32)),
                                      _p(np.ascontiguousarray(K, np.float32)),
                                      _p(np.ascontiguousarray(V, np.float32)), n_t, hd, kv_dim,
                                      gqa, n_heads, C.c_double(scale), _p(out))
    return out


def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().styx_oracle_argmax(_p(v), len(v)))


def f16_to_f32(h: int) -> float:
    return float(lib().styx_oracle_f16_to_f32(C.c_uint16(h)))


class OracleModel:
    """Holds numpy copies of a model's GGUF-layout tensors and runs the
    oracle's forward pass (styx_oracle_forward)."""

    def __init__(self, hp: dict, tensors: dict, n_ctx: int):
        self.hp, self.t, self.n_ctx = hp, tensors, n_ctx
        L = hp["n_layers"]
        kvd = hp["n_kv_heads"] * hp["head_dim"]
        self.kc = np.zeros(L * n_ctx * kvd, np.float32)
        self.vc = np.zeros(L * n_ctx * kvd, np.float32)
        self.layers = (Layer * L)()
        self._keep = []

        def f32(name):
            if name not in tensors:
                return None
            a = np.ascontiguousarray(tensors[name][2]).view(np.float32)
            self._keep.append(a)
            return a.ctypes.data

        def mat(name, per_expert=False):
            m = Mat()
            if name not in tensors:
                return m
            typ, dims, data = tensors[name]
            data = np.ascontiguousarray(data)
            self._keep.append(data)
            m.type, m.ncols, m.nrows, m.data = typ, dims[0], dims[1], data.ctypes.data
            return m

        for l in range(L):
            p = f"blk.{l}."
            ly = self.layers[l]
            ly.attn_norm = f32(p + "attn_norm.weight")
            ly.q_norm = f32(p + "attn_q_norm.weight")
            ly.k_norm = f32(p + "attn_k_norm.weight")
            ly.ffn_norm = f32(p + "ffn_norm.weight")
            ly.wq, ly.wk, ly.wv = mat(p + "attn_q.weight"), mat(p + "attn_k.weight"), mat(p + "attn_v.weight")
            ly.wo = mat(p + "attn_output.weight")
            ly.router = f32(p + "ffn_gate_inp.weight")
            ly.router_bias = f32(p + "ffn_gate_inp.bias")
            ly.gate_exps = mat(p + "ffn_gate_exps.weight")
            ly.up_exps = mat(p + "ffn_up_exps.weight")
            ly.down_exps = mat(p + "ffn_down_exps.weight")
            ly.gate_sh = mat(p + "ffn_gate_shexp.weight")
            ly.up_sh = mat(p + "ffn_up_shexp.weight")
            ly.down_sh = mat(p + "ffn_down_shexp.weight")
            ly.gate_inp_sh = f32(p + "ffn_gate_inp_shexp.weight")
        m = Model()
        for k in ("n_layers", "n_embd", "n_heads", "n_kv_heads", "head_dim", "n_expert",
                  "n_expert_used", "n_ff_exp", "n_vocab"):
            setattr(m, k, int(hp[k]))
        m.n_ff_sh = int(hp.get("n_ff_shexp", 0))
        m.n_ctx = n_ctx
        m.rms_eps, m.rope_base, m.norm_topk = hp["rms_eps"], hp["rope_base"], int(hp.get("norm_topk", 1))
        m.layers = self.layers
        m.output_norm = f32("output_norm.weight")
        m.output = mat("output.weight")
        m.token_embd = mat("token_embd.weight")
        m.kcache, m.vcache = self.kc.ctypes.data, self.vc.ctypes.data
        self.m = m

    def forward(self, pos: int, token: int, want_hidden=False):
        hp = self.hp
        logits = np.empty(hp["n_vocab"], np.float32)
        hidden = np.empty((hp["n_layers"] + 1, hp["n_embd"]), np.float32) if want_hidden else None
        ids = np.empty((hp["n_layers"], hp["n_expert_used"]), np.int32)
        margins = np.empty(hp["n_layers"], np.float32)
        rc = lib().styx_oracle_forward(C.addressof(self.m), pos, C.c_uint32(token), _p(logits),
                                       _p(hidden), _p(ids), _p(margins))
        if rc:
            raise RuntimeError(f"oracle forward failed ({rc})")
        return logits, hidden, ids, margins

    def moe_block(self, layer: int, x: np.ndarray):
        hp = self.hp
        x = np.array(x, np.float32, copy=True)
        xn = np.empty(hp["n_embd"], np.float32)
        lg = np.empty(hp["n_expert"], np.float32)
        ids = np.empty(hp["n_expert_used"], np.int32)
        w = np.empty(hp["n_expert_used"], np.float32)
        rc = lib().styx_oracle_moe_block(C.addressof(self.m), layer, _p(x), _p(xn), _p(lg), _p(ids), _p(w))
        if rc:
            raise RuntimeError(f"oracle moe_block failed ({rc})")
        return x, xn, lg, ids, w
