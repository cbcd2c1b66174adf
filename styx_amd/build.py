"""Build libstyx_hip.so (gfx950) in-tree with hipcc.

Usage: python -m styx_amd.build [-j N] [-v]

Every HIP source is compiled for gfx950 only, with packed FP32 instructions
disabled (-Xclang -target-feature -Xclang -packed-fp32-ops), then linked into
styx_amd/libstyx_hip.so next to this file.  Objects go to styx_amd/_build/.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libstyx_hip.so"
OBJ = PKG / "_build"
SOURCES = [
    "kernels_mv.hip",
    "kernels_aux.hip",
    "kernels_ref.hip",
    "attn.hip",
    "moe_block.hip",
    "capi.cpp",
    "dispatch.cpp",
    "dispatch_fused.cpp",
    "engine.cpp",
    "gguf.cpp",
]
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-result",
    "-Wno-unused-value",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # every atomic here is issued by one lane: the optimizer's wave-wide
    # rewrite would only add a wait for the result right after the atomic
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    f"-I{PKG.parent / 'include'}",
    f"-I{CSRC}",
]


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    lang = ["-x", "hip"] if src.suffix in (".hip", ".cpp") else []
    cmd = [HIPCC, *FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature: harmless
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    OBJ.mkdir(exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = []
        for name in SOURCES:
            src = CSRC / name
            obj = OBJ / (name + ".o")
            objs.append(obj)
            futs.append(ex.submit(_compile, src, obj, verbose))
        for f in futs:
            f.result()
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))


if __name__ == "__main__":
    main()
