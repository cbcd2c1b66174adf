"""ctypes bindings of libstyx_hip.so (include/styx_hip.h).

The library is built in-tree by ``python -m styx_amd.build``.  Loading fails
loudly when it is missing: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libstyx_hip.so"

STYX_OK = 0
F32, F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14
SKIP = 0xFFFFFFFF
BUF_DEVICE, BUF_HOST_PINNED = 0, 1

BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
TYPE_NAMES = {F32: "f32", F16: "f16", Q8_0: "q8_0", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K"}


class StyxError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"styx status {status}: {msg}")
        self.status = status


class MoeOpts(C.Structure):
    _fields_ = [
        ("n_ctx", C.c_int),
        ("use_graph", C.c_int),
        ("expert_budget_mb", C.c_int64),
        ("expert_hist", C.c_char_p),
        ("arena", C.c_int),
        ("repin_interval", C.c_int),
        ("repin_max", C.c_int),
        ("record_hidden", C.c_int),
        ("time_kernels", C.c_int),
        ("no_fuse", C.c_int),
        ("no_fold_qkv", C.c_int),
        ("max_polls", C.c_int),
    ]


class MoeHparams(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("n_embd", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("n_expert", C.c_int),
        ("n_expert_used", C.c_int), ("n_ff_exp", C.c_int), ("n_ff_shexp", C.c_int),
        ("n_vocab", C.c_int), ("n_ctx", C.c_int), ("rms_eps", C.c_float),
        ("rope_base", C.c_float), ("norm_topk", C.c_int), ("slab_bytes", C.c_uint64),
        ("expert_bytes_hbm", C.c_uint64), ("expert_bytes_host", C.c_uint64),
        ("unfused_fallbacks", C.c_int),
    ]


class MoeSynthCfg(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("n_embd", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("n_expert", C.c_int),
        ("n_expert_used", C.c_int), ("n_ff_exp", C.c_int), ("n_ff_shexp", C.c_int),
        ("n_vocab", C.c_int), ("rms_eps", C.c_float), ("rope_base", C.c_float),
        ("attn_type", C.c_int), ("embd_type", C.c_int), ("head_type", C.c_int),
        ("exp_type", C.c_int * 3), ("exp_mix", C.c_int), ("sigma", C.c_float),
        ("seed", C.c_uint64), ("router_zipf_s", C.c_float),
    ]


class ExpertSrc(C.Structure):
    _fields_ = [
        ("hot", C.c_void_p), ("hot_slab", C.c_int64),
        ("arena", C.c_void_p), ("arena_slab", C.c_int64),
        ("host", C.c_void_p), ("host_slab", C.c_int64),
    ]


class KernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 32), ("launches", C.c_uint64), ("total_ms", C.c_double),
                ("bytes", C.c_double)]


class Binding(C.Structure):
    _fields_ = [("buf", C.c_void_p), ("offset", C.c_uint64), ("range", C.c_uint64)]


# push blocks of the fused dispatch kernels (include/styx_hip.h)
class PushRouterTopk(C.Structure):
    _fields_ = [("E", C.c_uint32), ("H", C.c_uint32), ("k", C.c_uint32), ("renorm", C.c_uint32),
                ("arena_mode", C.c_uint32), ("layer", C.c_uint32), ("eps", C.c_float),
                ("flags", C.c_uint32)]


class PushGateUpSilu(C.Structure):
    _fields_ = [("H", C.c_uint32), ("F", C.c_uint32), ("k", C.c_uint32), ("type_up", C.c_uint32),
                ("n_slabs", C.c_uint32), ("slab_gate", C.c_uint32), ("slab_up", C.c_uint32)]


class PushDownReduce(C.Structure):
    _fields_ = [("H", C.c_uint32), ("F", C.c_uint32), ("k", C.c_uint32), ("n_slabs", C.c_uint32),
                ("slab_down", C.c_uint32)]


class PushAttnPaged(C.Structure):
    _fields_ = [("eps", C.c_float), ("page_tokens", C.c_uint32), ("nh", C.c_uint32),
                ("nkv", C.c_uint32), ("hd", C.c_uint32), ("chunk", C.c_uint32),
                ("max_chunks", C.c_uint32), ("scale", C.c_float), ("flags", C.c_uint32),
                ("pos", C.c_uint32)]


vp, i32, i64, u32, u64, f32p = C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_uint64, C.c_void_p

# name: (restype, argtypes)
_SIGS = {
    "styx_last_error": (C.c_char_p, []),
    "styx_gpu_new": (i32, [i32, C.POINTER(vp)]),
    "styx_gpu_free": (None, [vp]),
    "styx_gpu_hbm_bytes": (u64, [vp]),
    "styx_gpu_name": (C.c_char_p, [vp]),
    "styx_gpu_sync": (i32, [vp]),
    "styx_buf_new": (i32, [vp, u64, i32, C.POINTER(vp)]),
    "styx_buf_free": (None, [vp]),
    "styx_buf_size": (u64, [vp]),
    "styx_buf_device_ptr": (vp, [vp]),
    "styx_upload": (i32, [vp, vp, u64, vp, u64]),
    "styx_download": (i32, [vp, vp, u64, vp, u64]),
    "styx_copy_region": (i32, [vp, vp, u64, vp, u64, u64]),
    "styx_kernel_get": (i32, [vp, C.c_char_p, vp, i32, C.POINTER(vp)]),
    "styx_kernel_free": (None, [vp]),
    "styx_kernel_names": (C.c_char_p, []),
    "styx_batch_new": (i32, [vp, C.POINTER(vp)]),
    "styx_batch_free": (None, [vp]),
    "styx_batch_begin": (i32, [vp]),
    "styx_batch_dispatch": (i32, [vp, vp, vp, i32, vp, u32, u32, u32, u32, i32]),
    "styx_batch_submit": (i32, [vp]),
    "styx_dispatch_sync": (i32, [vp, vp, vp, i32, vp, u32, u32, u32, u32]),
    "styx_batch_new_async": (i32, [vp, C.POINTER(vp)]),
    "styx_batch_submit_async": (i32, [vp, vp, u64]),
    "styx_batch_wait_idle": (i32, [vp]),
    "styx_batch_submit_wait_sem": (i32, [vp, vp, u64]),
    "styx_timeline_new": (i32, [vp, C.POINTER(vp)]),
    "styx_timeline_free": (None, [vp]),
    "styx_timeline_value": (i32, [vp, C.POINTER(u64)]),
    "styx_op_to_split": (i32, [vp, i32, vp, vp, i64, i64]),
    "styx_op_from_split": (i32, [vp, i32, vp, vp, i64, i64]),
    "styx_op_dequant_rows": (i32, [vp, i32, vp, i64, i32, i64, i64, vp]),
    "styx_op_matvec": (i32, [vp, i32, vp, i32, i32, vp, vp, C.c_float, vp, i32]),
    "styx_op_router_topk": (i32, [vp, vp, vp, C.c_float, vp, vp, i32, i32, i32, i32, vp, vp,
                                  i32, i32, vp, vp, vp, vp]),
    "styx_op_topk_softmax": (i32, [vp, vp, i32, i32, i32, vp, vp, i32, i32, vp, vp]),
    "styx_op_moe_gate_up": (i32, [vp, i32, i32, vp, vp, vp, vp, vp, i32, i32, i32]),
    "styx_op_moe_down_reduce": (i32, [vp, i32, vp, vp, vp, vp, vp, i32, i32, i32]),
    "styx_op_attn_decode": (i32, [vp, vp, vp, vp, vp, vp, C.c_float, vp, vp, vp, vp, i32, vp,
                                  vp, vp, i32, i32, i32, i32, i32, C.c_float]),
    "styx_op_attn_decode_noalloc": (i32, [vp, vp, vp, vp, vp, vp, C.c_float, vp, vp, vp, vp, i32,
                                          vp, vp, i32, i32, i32, i32, i32, C.c_float]),
    "styx_op_attn_part_floats": (i64, [i32, i32, i32, i32]),
    "styx_rope_table": (None, [C.c_float, i32, i32, vp]),
    "styx_op_read_probe": (i32, [vp, vp, i64, vp, i32]),
    "styx_residency_plan": (i32, [C.c_char_p, i32, i32, vp, i64, vp, vp]),
    "styx_repin_select": (i32, [vp, i32, vp, i32, i32, vp, vp, C.POINTER(i32)]),
    "styx_moe_check_file": (i32, [C.c_char_p, vp]),
    "styx_zipf_bias_table": (i32, [i32, i32, C.c_float, C.c_float, u64, vp]),
    "styx_moe_fill_kv": (i32, [vp, i32, C.c_uint64, C.c_float]),
    "styx_moe_read_kv": (i32, [vp, i32, i32, i32, vp, vp]),
    "styx_op_gather_slabs": (i32, [vp, vp, vp, vp, vp, vp, i32, i32]),
    "styx_op_argmax": (i32, [vp, vp, i32, vp, vp, vp]),
    "styx_op_gen_quant": (i32, [vp, i32, u64, C.c_float, vp, i64]),
    "styx_op_gen_f32": (i32, [vp, u64, C.c_float, C.c_float, vp, i64]),
    "styx_gguf_inspect": (i32, [C.c_char_p, vp, u64]),
    "styx_moe_load": (i32, [vp, C.c_char_p, vp, C.POINTER(vp)]),
    "styx_moe_synth": (i32, [vp, vp, vp, C.POINTER(vp)]),
    "styx_moe_free": (None, [vp]),
    "styx_moe_get_hparams": (i32, [vp, vp]),
    "styx_moe_forward_token": (i32, [vp, u32, vp]),
    "styx_moe_generate": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "styx_moe_decode": (i32, [vp, i32, vp]),
    "styx_moe_set_timing": (i32, [vp, i32]),
    "styx_moe_moe_block_trace": (i32, [vp, vp, i64, C.POINTER(i32), C.POINTER(C.c_double)]),
    "styx_moe_set_wait_limit": (i32, [vp, i32]),
    "styx_moe_attn_trace": (i32, [vp, vp, i64, C.POINTER(i32), C.POINTER(C.c_double)]),
    "styx_moe_time_stage": (i32, [vp, C.c_char_p, i32, C.POINTER(C.c_double), C.POINTER(i32)]),
    "styx_moe_last_expert_ids": (i32, [vp, vp]),
    "styx_moe_last_hot_cold": (i32, [vp, vp]),
    "styx_moe_reset": (i32, [vp]),
    "styx_moe_repin_swaps": (u64, [vp]),
    "styx_moe_last_hidden": (i32, [vp, vp]),
    "styx_moe_export_tensor": (i32, [vp, C.c_char_p, vp, u64, C.POINTER(u64), C.POINTER(i32),
                                     C.POINTER(C.c_int64 * 4), C.POINTER(i32)]),
    "styx_moe_tensor_names": (i32, [vp, vp, u64]),
    "styx_moe_kernel_stats": (i32, [vp, vp, i32, C.POINTER(i32)]),
    "styx_moe_kernel_stats_reset": (i32, [vp]),
}

EXPORTED = tuple(_SIGS)

_lib = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libstyx_hip.so once.  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build it with `python -m styx_amd.build` "
            "(the HIP library is required; there is no fallback)")
    lib = C.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != STYX_OK:
        raise StyxError(status, load().styx_last_error().decode(errors="replace"))
