"""The C ABI's three mirrors cannot drift from include/styx_hip.h: the Rust
binding written out in the integration guide (the -sys crate a maintainer adds to
the reference) and the ctypes tables of styx_amd/_lib.py.  For every struct
the header declares, the field names and order, and the offsets and size of
the C layout (printed by a gcc build of the header itself), must match the
Rust #[repr(C)] struct and the ctypes Structure; for every function, the
Rust declaration and the ctypes signature must take the same parameters
(count, and for each one pointer vs value, constness of the pointee, and
the value's size and kind).  No GPU needed."""
from __future__ import annotations

import ctypes as C
import json
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HDR = ROOT / "include" / "styx_hip.h"


def _strip_c(src: str) -> str:
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.sub(r"^\s*#.*$", "", src, flags=re.M)


# ------------------------------------------------------------- the header --
def c_structs() -> dict[str, list[tuple[str, str, int]]]:
    """typedef struct { ... } name;  ->  name: [(field, base type + '*'s, array len)]"""
    out = {}
    for body, name in re.findall(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", _strip_c(HDR.read_text()),
                                 flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            m = re.match(r"((?:const\s+)?\w+)\s+(.*)", decl)
            base, rest = m.group(1), m.group(2)
            for d in rest.split(","):
                d = d.strip()
                stars = d.count("*")
                dm = re.match(r"[\s\*]*(?:const\s+)?(\w+)\s*(?:\[(\d+)\])?", d)
                fields.append((dm.group(1), base + "*" * stars, int(dm.group(2) or 1)))
        out[name] = fields
    return out


def c_functions() -> dict[str, tuple[str, list[str]]]:
    """name -> (return type, [parameter types]) with array parameters as pointers."""
    src = _strip_c(HDR.read_text())
    src = re.sub(r"typedef\s+struct\s*\{.*?\}\s*\w+\s*;", "", src, flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"([\w\s\*]+?)\b(styx_\w+)\s*\(([^)]*)\)\s*;", src):
        ps = []
        if params.strip() not in ("", "void"):
            for p in params.split(","):
                p = " ".join(p.split())
                arr = re.search(r"\[\s*\d*\s*\]$", p)
                p = re.sub(r"\[\s*\d*\s*\]$", "", p)
                p = re.sub(r"\s*\b\w+$", "", p)  # drop the parameter name
                if arr:
                    p += " *"
                ps.append(p)
        out[name] = (" ".join(ret.split()), ps)
    return out


def c_kind(t: str) -> tuple:
    """Canonical form of a C parameter type: ('ptr', pointee const, depth) or
    ('val', size, 'i' | 'u' | 'f')."""
    t = " ".join(t.replace("*", " * ").split())
    depth = t.count("*")
    if depth:
        # constness of the outermost pointer's pointee: `const T *`, or
        # `T *const *` (an array of const pointers passed as a pointer)
        toks = t.split()
        last = len(toks) - 1 - toks[::-1].index("*")
        if depth == 1:
            const = "const" in toks[:last]
        else:
            const = toks[last - 1] == "const"
        return ("ptr", const, depth)
    base = t.replace("const", "").strip()
    vals = {"int": (4, "i"), "int32_t": (4, "i"), "uint32_t": (4, "u"), "int64_t": (8, "i"),
            "uint64_t": (8, "u"), "float": (4, "f"), "double": (8, "f")}
    return ("val",) + vals[base]


# ------------------------------------------------------------- Rust text --
def rust_block() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```rust\n(.*?)```", text, flags=re.S)
    lib = [b for b in blocks if 'extern "C"' in b]
    assert len(lib) == 1, "INTEGRATION.md must hold one -sys block with the extern declarations"
    return lib[0]


def rust_structs() -> dict[str, list[tuple[str, str]]]:
    out = {}
    src = re.sub(r"//[^\n]*", "", rust_block())
    for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+)\s*\{(.*?)\}", src, flags=re.S):
        fields = re.findall(r"pub\s+(\w+)\s*:\s*([^,]+?)\s*(?:,|$)", body.strip())
        out[name] = [(f, " ".join(t.split())) for f, t in fields]
    return out


def rust_functions() -> dict[str, tuple[str, list[str]]]:
    src = re.sub(r"//[^\n]*", "", rust_block())
    ext = src[src.index('extern "C"'):]
    out = {}
    for name, params, ret in re.findall(r"pub fn (\w+)\(([^)]*)\)\s*(?:->\s*([^;]+))?;", ext):
        ps = [p.split(":", 1)[1].strip() for p in params.split(",") if p.strip()]
        out[name] = ((ret or "()").strip(), ps)
    return out


_RUST_VAL = {"c_int": (4, "i"), "i32": (4, "i"), "u32": (4, "u"), "i64": (8, "i"),
             "u64": (8, "u"), "f32": (4, "f"), "f64": (8, "f"), "c_char": (1, "i"),
             "u8": (1, "u")}


def rust_kind(t: str) -> tuple:
    t = " ".join(t.split())
    depth = 0
    const = None
    while t.startswith("*"):
        c = t.startswith("*const")
        if const is None:
            const = c
        t = t[len("*const"):].strip() if c else t[len("*mut"):].strip()
        depth += 1
    if depth:
        return ("ptr", const, depth)
    return ("val",) + _RUST_VAL[t]


def rust_layout(fields: list[tuple[str, str]], structs: dict) -> tuple[list[int], int]:
    """repr(C) offsets and size."""
    def size_align(t: str) -> tuple[int, int]:
        t = t.strip()
        if t.startswith("*"):
            return 8, 8
        m = re.match(r"\[(.+);\s*(\d+)\]$", t)
        if m:
            s, a = size_align(m.group(1))
            return s * int(m.group(2)), a
        if t in _RUST_VAL:
            s = _RUST_VAL[t][0]
            return s, s
        raise AssertionError(f"unknown Rust field type {t}")
    off, offs, align = 0, [], 1
    for _, t in fields:
        s, a = size_align(t)
        off = (off + a - 1) // a * a
        offs.append(off)
        off += s
        align = max(align, a)
    return offs, (off + align - 1) // align * align


# ------------------------------------------------------------ C layouts --
@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    """sizeof and every offsetof of each header struct, from gcc."""
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not available")
    structs = c_structs()
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HDR}"', "int main(void) {",
             'printf("{");']
    first = True
    for name, fields in structs.items():
        sep = "" if first else ","
        first = False
        parts = [f'\\"{f}\\": %zu' for f, _, _ in fields]
        args = ", ".join(f"offsetof({name}, {f})" for f, _, _ in fields)
        lines.append(f'printf("{sep}\\"{name}\\": {{\\"size\\": %zu, {", ".join(parts)}}}", '
                     f"sizeof({name}), {args});")
    lines += ['printf("}");', "return 0; }"]
    d = tmp_path_factory.mktemp("abi")
    (d / "lay.c").write_text("\n".join(lines))
    subprocess.run([gcc, "-std=c11", "-o", str(d / "lay"), str(d / "lay.c")], check=True)
    return json.loads(subprocess.run([str(d / "lay")], capture_output=True, text=True,
                                     check=True).stdout)


CTYPES_OF = {"styx_binding": "Binding", "styx_expert_src": "ExpertSrc",
             "styx_moe_opts": "MoeOpts", "styx_moe_hparams": "MoeHparams",
             "styx_moe_synth_cfg": "MoeSynthCfg", "styx_kernel_stat": "KernelStat",
             "styx_push_router_topk": "PushRouterTopk",
             "styx_push_moe_gate_up_silu": "PushGateUpSilu",
             "styx_push_moe_down_reduce": "PushDownReduce",
             "styx_push_attn_decode_paged": "PushAttnPaged"}


def test_header_parses():
    s, f = c_structs(), c_functions()
    assert {"styx_moe_opts", "styx_moe_hparams", "styx_push_router_topk"} <= set(s)
    assert "max_polls" in [x[0] for x in s["styx_moe_opts"]]
    assert "unfused_fallbacks" in [x[0] for x in s["styx_moe_hparams"]]
    assert len(f) > 60 and f["styx_batch_dispatch"][1][-1] == "int"


@pytest.mark.parametrize("name", sorted(c_structs()))
def test_rust_struct_matches_header(name, c_layout):
    rs = rust_structs()
    assert name in rs, f"INTEGRATION.md has no #[repr(C)] struct {name}"
    cf = [f for f, _, _ in c_structs()[name]]
    assert [f for f, _ in rs[name]] == cf, f"{name}: field names or order differ"
    offs, size = rust_layout(rs[name], rs)
    lay = c_layout[name]
    assert offs == [lay[f] for f in cf], f"{name}: offsets differ from the C layout"
    assert size == lay["size"], f"{name}: Rust size {size} vs C {lay['size']}"


@pytest.mark.parametrize("name", sorted(CTYPES_OF))
def test_ctypes_struct_matches_header(name, c_layout):
    from styx_amd import _lib
    cls = getattr(_lib, CTYPES_OF[name])
    cf = [f for f, _, _ in c_structs()[name]]
    assert [f[0] for f in cls._fields_] == cf, f"{name}: ctypes fields differ"
    lay = c_layout[name]
    assert C.sizeof(cls) == lay["size"]
    for f in cf:
        assert getattr(cls, f).offset == lay[f], (name, f)


def test_every_struct_has_a_ctypes_mirror():
    assert set(c_structs()) == set(CTYPES_OF)


def test_rust_functions_match_header():
    cf, rf = c_functions(), rust_functions()
    assert set(cf) == set(rf), (set(cf) - set(rf), set(rf) - set(cf))
    for name, (ret, ps) in cf.items():
        rret, rps = rf[name]
        assert len(ps) == len(rps), f"{name}: {len(ps)} parameters in C, {len(rps)} in Rust"
        for i, (a, b) in enumerate(zip(ps, rps)):
            assert c_kind(a) == rust_kind(b), f"{name} parameter {i}: C `{a}` vs Rust `{b}`"
        if ret == "void":
            assert rret == "()", name
        else:
            assert c_kind(ret) == rust_kind(rret), f"{name}: return C `{ret}` vs Rust `{rret}`"


def _ctypes_kind(t) -> tuple:
    if t is None:
        return None
    if t in (C.c_void_p, C.c_char_p) or (isinstance(t, type) and issubclass(t, C._Pointer)):
        return "ptr"
    return ("val", C.sizeof(t), "f" if t in (C.c_float, C.c_double) else "i")


def test_ctypes_signatures_match_header():
    from styx_amd import _lib
    for name, (ret, ps) in c_functions().items():
        assert name in _lib._SIGS, name
        rt, ats = _lib._SIGS[name]
        assert len(ats) == len(ps), f"{name}: ctypes takes {len(ats)} parameters, C {len(ps)}"
        for i, (a, t) in enumerate(zip(ps, ats)):
            ck = c_kind(a)
            k = _ctypes_kind(t)
            if ck[0] == "ptr":
                assert k == "ptr", f"{name} parameter {i}"
            else:
                assert k[:2] == ck[:2], f"{name} parameter {i}: {a} vs {t}"
