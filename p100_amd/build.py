"""Builds p100_amd/libp1x.so for gfx950 with hipcc (in-tree, so the library travels with the source tree).

    python -m p100_amd.build          # compile every source, link the shared library
    python -m p100_amd.build --changed  # recompile only sources newer than their objects (or any header)
"""
from __future__ import annotations

import os
import pathlib
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libp1x.so"
OBJ = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# gfx950 only; packed FP32 instructions disabled (they are not used by these kernels on purpose).
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", str(PKG.parent / "include")]
SOURCES = ["act.hip", "mmvq.hip", "mmq.hip", "mmvh.hip", "fattn.hip", "glue.hip", "capi.cpp", "decode.cpp"]


def _compile(src: str) -> pathlib.Path:
    obj = OBJ / (src + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in (res.stderr or "").splitlines() if noise not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _stale(src: str) -> bool:
    obj = OBJ / (src + ".o")
    if not obj.exists():
        return True
    deps = [CSRC / src, *CSRC.glob("*.h"), PKG.parent / "include" / "p1x.h"]
    return max(d.stat().st_mtime for d in deps) > obj.stat().st_mtime


def build(verbose: bool = True, changed_only: bool = False) -> pathlib.Path:
    OBJ.mkdir(exist_ok=True)
    todo = [s for s in SOURCES if _stale(s)] if changed_only else SOURCES
    with ThreadPoolExecutor(max_workers=min(max(len(todo), 1), os.cpu_count() or 1)) as ex:
        list(ex.map(_compile, todo))
    objs = [OBJ / (s + ".o") for s in SOURCES]
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(changed_only="--changed" in sys.argv[1:])
