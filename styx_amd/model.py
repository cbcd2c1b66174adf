"""MoeModel: Python mirror of the engine API of crates/model/src/moe.rs
(load, forward_token, last_expert_ids, last_hot_cold, reset, hp, slab_bytes)
and of the generate_moe driver, over libstyx_hip.so's styx_moe_* entry
points."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib as L
from .runtime import Gpu


@dataclass
class SynthConfig:
    """Seeded synthetic qwen3moe model (weights generated in HBM)."""
    n_layers: int = 48
    n_embd: int = 2048
    n_heads: int = 32
    n_kv_heads: int = 4
    head_dim: int = 128
    n_expert: int = 128
    n_expert_used: int = 8
    n_ff_exp: int = 768
    n_ff_shexp: int = 0
    n_vocab: int = 151936
    rms_eps: float = 1e-6
    rope_base: float = 1e6
    attn_type: int = L.Q8_0
    embd_type: int = L.Q8_0
    head_type: int = L.Q8_0
    exp_type: tuple = (L.Q8_0, L.Q8_0, L.Q8_0)
    exp_mix: bool = False  # type(l, role) = [q4_K, q5_K, q6_K][(l + role) % 3]
    sigma: float = 0.02
    seed: int = 0x5157594D
    router_zipf_s: float = 0.0

    def to_c(self) -> L.MoeSynthCfg:
        c = L.MoeSynthCfg()
        for f in ("n_layers", "n_embd", "n_heads", "n_kv_heads", "head_dim", "n_expert",
                  "n_expert_used", "n_ff_exp", "n_ff_shexp", "n_vocab", "attn_type",
                  "embd_type", "head_type"):
            setattr(c, f, int(getattr(self, f)))
        c.rms_eps, c.rope_base, c.sigma = self.rms_eps, self.rope_base, self.sigma
        c.exp_type[:] = [int(t) for t in self.exp_type]
        c.exp_mix, c.seed, c.router_zipf_s = int(self.exp_mix), int(self.seed), self.router_zipf_s
        return c


# the 48-layer Qwen3-30B-A3B shape, mixed K-quant experts.
CFG_30B_A3B = SynthConfig(exp_mix=True)
# one qwen3moe layer, all q8_0 (vocab kept small: only the MoE block matters).
CFG_LAYER_Q8 = SynthConfig(n_layers=1, n_vocab=4096)


def make_opts(n_ctx=4096, use_graph=True, expert_budget_mb=-1, expert_hist=None, arena=True,
              repin_interval=0, repin_max=2, record_hidden=False, time_kernels=False,
              fuse=True, fold_qkv=True, max_polls=0):
    o = L.MoeOpts()
    o.n_ctx, o.use_graph, o.expert_budget_mb = n_ctx, int(use_graph), expert_budget_mb
    o._hist = expert_hist.encode() if expert_hist else None
    o.expert_hist = o._hist
    o.arena, o.repin_interval, o.repin_max = int(arena), repin_interval, repin_max
    o.record_hidden, o.time_kernels = int(record_hidden), int(time_kernels)
    o.no_fuse = 0 if fuse else 1
    o.no_fold_qkv = 0 if fold_qkv else 1
    o.max_polls = max_polls
    return o


class MoeModel:
    """MoeModel (moe.rs:373-499)."""

    def __init__(self, gpu: Gpu, handle: C.c_void_p):
        self.gpu, self.lib, self.h = gpu, gpu.lib, handle
        hp = L.MoeHparams()
        L.check(self.lib.styx_moe_get_hparams(self.h, C.byref(hp)))
        self.hp = hp

    @classmethod
    def load(cls, gpu: Gpu, path: str, **opts) -> "MoeModel":
        """MoeModel::load (moe.rs:536)."""
        o = make_opts(**opts)
        h = C.c_void_p()
        L.check(gpu.lib.styx_moe_load(gpu.h, str(path).encode(), C.byref(o), C.byref(h)))
        return cls(gpu, h)

    @classmethod
    def synth(cls, gpu: Gpu, cfg: SynthConfig, **opts) -> "MoeModel":
        o = make_opts(**opts)
        c = cfg.to_c()
        h = C.c_void_p()
        L.check(gpu.lib.styx_moe_synth(gpu.h, C.byref(c), C.byref(o), C.byref(h)))
        return cls(gpu, h)

    @property
    def slab_bytes(self) -> int:
        return int(self.hp.slab_bytes)

    @property
    def n_ctx_max(self) -> int:
        return int(self.hp.n_ctx)

    def forward_token(self, token: int, want_logits: bool = True) -> np.ndarray | None:
        """MoeModel::forward_token (moe.rs:1780)."""
        out = np.empty(self.hp.n_vocab, np.float32) if want_logits else None
        L.check(self.lib.styx_moe_forward_token(self.h, int(token),
                                                out.ctypes.data if want_logits else None))
        return out

    def generate(self, prompt, n_predict: int):
        """generate_moe.rs:44-67: returns (tokens, prefill_s, decode_s)."""
        p = np.ascontiguousarray(np.asarray(prompt, np.uint32))
        out = np.empty(n_predict, np.uint32)
        ps, ds = C.c_double(), C.c_double()
        L.check(self.lib.styx_moe_generate(self.h, p.ctypes.data, len(p), n_predict,
                                           out.ctypes.data, C.byref(ps), C.byref(ds)))
        return out, ps.value, ds.value

    def decode(self, n_steps: int) -> np.ndarray:
        """Greedy-decode n_steps more tokens from the current state."""
        out = np.empty(max(n_steps, 1), np.uint32)
        L.check(self.lib.styx_moe_decode(self.h, n_steps, out.ctypes.data))
        return out[:n_steps]

    def set_timing(self, on: bool) -> None:
        L.check(self.lib.styx_moe_set_timing(self.h, int(on)))

    def time_stage(self, stage: str, reps: int = 20) -> tuple[float, int]:
        """(mean us per graph replay, kernels per replay) of one stage's
        launches over every layer (styx_moe_time_stage)."""
        us, n = C.c_double(), C.c_int()
        L.check(self.lib.styx_moe_time_stage(self.h, stage.encode(), reps, C.byref(us), C.byref(n)))
        return us.value, n.value

    def moe_block_trace(self) -> tuple[np.ndarray, float] | None:
        """Phase stamps of the fused MoE block from the last timed token:
        ([n_layers][nwg][16] ticks, ticks per us), or None without it."""
        nwg, tpu = C.c_int(), C.c_double()
        L.check(self.lib.styx_moe_moe_block_trace(self.h, None, 0, C.byref(nwg), None))
        if nwg.value == 0:
            return None
        out = np.zeros((self.hp.n_layers, nwg.value, 16), np.uint64)
        L.check(self.lib.styx_moe_moe_block_trace(self.h, out.ctypes.data, out.size, C.byref(nwg),
                                                 C.byref(tpu)))
        return out, tpu.value

    def set_wait_limit(self, max_polls: int):
        """Wait bound of the fused launches for the following tokens."""
        L.check(self.lib.styx_moe_set_wait_limit(self.h, max_polls))

    def unfused_fallbacks(self) -> int:
        """Times a fused launch gave up and the model went over to the
        separate kernels."""
        hp = L.MoeHparams()
        L.check(self.lib.styx_moe_get_hparams(self.h, C.byref(hp)))
        return hp.unfused_fallbacks

    def attn_trace(self) -> tuple[np.ndarray, float] | None:
        """Phase stamps of the attention launches from the last timed token:
        ([n_layers][nwg][8] ticks, ticks per us), or None."""
        nwg, tpu = C.c_int(), C.c_double()
        L.check(self.lib.styx_moe_attn_trace(self.h, None, 0, C.byref(nwg), None))
        if nwg.value == 0:
            return None
        out = np.zeros((self.hp.n_layers, nwg.value, 8), np.uint64)
        L.check(self.lib.styx_moe_attn_trace(self.h, out.ctypes.data, out.size, C.byref(nwg),
                                            C.byref(tpu)))
        return out, tpu.value

    def last_expert_ids(self) -> np.ndarray:
        """moe.rs:2387-2402: [n_layers][k]."""
        out = np.empty((self.hp.n_layers, self.hp.n_expert_used), np.uint32)
        L.check(self.lib.styx_moe_last_expert_ids(self.h, out.ctypes.data))
        return out

    def last_hot_cold(self) -> np.ndarray:
        """moe.rs:1512-1521: [n_layers][2] (hot, cold)."""
        out = np.empty((self.hp.n_layers, 2), np.uint32)
        L.check(self.lib.styx_moe_last_hot_cold(self.h, out.ctypes.data))
        return out

    def last_hidden(self) -> np.ndarray:
        out = np.empty((self.hp.n_layers + 1, self.hp.n_embd), np.float32)
        L.check(self.lib.styx_moe_last_hidden(self.h, out.ctypes.data))
        return out

    def reset(self) -> None:
        L.check(self.lib.styx_moe_reset(self.h))

    def fill_kv(self, n_t: int, seed: int = 0x4B56, sigma: float = 1.0) -> None:
        """Synthetic context: K/V rows [0, n_t) ~ N(0, sigma); the next token
        is forwarded at position n_t."""
        L.check(self.lib.styx_moe_fill_kv(self.h, int(n_t), int(seed), float(sigma)))

    def read_kv(self, layer: int, t0: int, n: int):
        kvd = self.hp.n_kv_heads * self.hp.head_dim
        k = np.empty((n, kvd), np.float32)
        v = np.empty((n, kvd), np.float32)
        L.check(self.lib.styx_moe_read_kv(self.h, layer, t0, n, k.ctypes.data, v.ctypes.data))
        return k, v

    @property
    def repin_swaps(self) -> int:
        return int(self.lib.styx_moe_repin_swaps(self.h))

    def tensor_names(self) -> list[str]:
        buf = C.create_string_buffer(1 << 20)
        L.check(self.lib.styx_moe_tensor_names(self.h, buf, len(buf)))
        return [s for s in buf.value.decode().split("\n") if s]

    def export_tensor(self, name: str):
        """(ggml_type, gguf_dims, bytes or f32 array) of one tensor, GGUF layout."""
        size, typ, nd = C.c_uint64(), C.c_int(), C.c_int()
        dims = (C.c_int64 * 4)()
        L.check(self.lib.styx_moe_export_tensor(self.h, name.encode(), None, 0, C.byref(size),
                                                C.byref(typ), C.byref(dims), C.byref(nd)))
        data = np.empty(size.value, np.uint8)
        L.check(self.lib.styx_moe_export_tensor(self.h, name.encode(), data.ctypes.data,
                                                size.value, None, None, None, None))
        return typ.value, [int(dims[i]) for i in range(nd.value)], data

    def kernel_stats(self) -> dict:
        arr = (L.KernelStat * 64)()
        n = C.c_int()
        L.check(self.lib.styx_moe_kernel_stats(self.h, arr, 64, C.byref(n)))
        return {arr[i].name.decode(): (arr[i].launches, arr[i].total_ms, arr[i].bytes)
                for i in range(min(n.value, 64))}

    def kernel_stats_reset(self) -> None:
        L.check(self.lib.styx_moe_kernel_stats_reset(self.h))

    def close(self) -> None:
        if self.h:
            self.lib.styx_moe_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class Hud:
    """The residency HUD of generate_moe.rs:87-119: per-token (hot, cold)
    routed-slot counts folded into totals and a per-layer cold count, then
    the reference's summary lines (hot/cold shares, cold PCIe bytes, the
    per-layer cold heatmap, repin swaps)."""

    def __init__(self, n_layers: int, k: int, slab_bytes: int):
        self.k, self.slab_bytes = k, slab_bytes
        self.hot = self.cold = 0
        self.cold_by_layer = np.zeros(n_layers, np.int64)

    def tick(self, hot_cold: np.ndarray) -> None:
        """hud_tick: fold one token's MoeModel.last_hot_cold() ([L][2])."""
        hc = np.asarray(hot_cold, np.int64)
        self.hot += int(hc[:, 0].sum())
        self.cold += int(hc[:, 1].sum())
        self.cold_by_layer += hc[:, 1]

    def lines(self, n_tok: int, repin_swaps: int = 0) -> list[str]:
        """The summary after n_tok forwarded tokens (prompt + generated - 1)."""
        total = max(self.hot + self.cold, 1)
        streamed = self.cold * self.slab_bytes
        out = [f"hud: hot {100.0 * self.hot / total:.1f}% ({self.hot}) | "
               f"cold {100.0 * self.cold / total:.1f}% ({self.cold}) | "
               f"cold PCIe ~{streamed / 2**30:.2f} GiB total, "
               f"~{streamed / max(n_tok, 1) / 2**20:.1f} MiB/tok"]
        glyphs = ""
        for c in self.cold_by_layer:
            f = c / max(n_tok * self.k, 1)
            glyphs += "." if f == 0 else str(min(int(f * 10.0), 9))
        out.append(f"hud: cold/layer [{glyphs}] (.=0%, 9=90%+ of k={self.k} slots)")
        if repin_swaps > 0:
            out.append(f"hud: repin {repin_swaps} slab swaps "
                       f"(~{repin_swaps * self.slab_bytes / 2**30:.2f} GiB copied)")
        return out


def generate_hud(m: MoeModel, prompt, n_predict: int) -> tuple[list[int], list[str]]:
    """generate_moe.rs:44-119 with MOE_HUD: token-at-a-time prefill, greedy
    argmax on the host (ties to the last index), a HUD tick after every
    forward_token call (prompt and generated tokens alike; the last
    generated token is not forwarded).  Returns (tokens, HUD lines)."""
    hud = Hud(m.hp.n_layers, m.hp.n_expert_used, m.slab_bytes)
    logits = None
    for t in prompt:
        logits = m.forward_token(int(t))
        hud.tick(m.last_hot_cold())
    nxt = argmax_last(logits)
    out = [nxt]
    for _ in range(1, n_predict):
        logits = m.forward_token(nxt)
        hud.tick(m.last_hot_cold())
        nxt = argmax_last(logits)
        out.append(nxt)
    n_tok = len(prompt) + len(out) - 1
    return out, hud.lines(n_tok, m.repin_swaps)


def argmax_last(v: np.ndarray) -> int:
    """generate_moe.rs:29: max_by(total_cmp) -> the LAST maximal index."""
    b = v.astype(np.float32).view(np.int32).astype(np.int64)
    key = b ^ ((b >> 31) & 0x7FFFFFFF)
    m = key.max()
    return int(np.nonzero(key == m)[0][-1])
