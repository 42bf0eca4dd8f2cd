"""The C-ABI library exists, loads without a GPU, and exports every entry point include/p1x.h declares."""
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "p1x.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(p1x_[a-z0-9_]+)\s*\(", text)))


def test_header_matches_python_export_list():
    import p100_amd

    assert declared() == sorted(p100_amd.EXPORTS)


def test_library_exports_every_declared_symbol():
    import p100_amd

    if not p100_amd.LIB_PATH.exists():
        p100_amd_build = pytest.importorskip("p100_amd.build")
        p100_amd_build.build()
    syms = p100_amd.load_symbols_only()
    assert sorted(syms) == declared()
    out = subprocess.run(["nm", "-D", "--defined-only", str(p100_amd.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert set(declared()) <= exported


def test_library_targets_gfx950_only(tmp_path):
    import p100_amd

    fatbin = tmp_path / "fatbin"
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", str(p100_amd.LIB_PATH), str(fatbin)],
                   check=True)
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o", f"--input={fatbin}"],
                         capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("offload bundle listing unavailable")
    targets = [t for t in out.stdout.split() if "amdgcn" in t]
    assert targets and all("gfx950" in t for t in targets), out.stdout


def test_version_without_gpu():
    import p100_amd

    syms = p100_amd.load_symbols_only()
    syms["p1x_version"].restype = int
    assert syms["p1x_version"]() >= 100


def test_struct_layouts_match_header(tmp_path):
    """The ctypes mirrors have the C structs' sizes and field offsets (compiled from include/p1x.h with gcc)."""
    import ctypes as C

    import p100_amd
    from p100_amd import llama

    structs = {
        "p1x_attn_params": (p100_amd.AttnParams, [f for f, _ in p100_amd.AttnParams._fields_]),
        "p1x_kv_strides": (p100_amd.KVStrides, [f for f, _ in p100_amd.KVStrides._fields_]),
        "p1x_llama_hparams": (llama.LlamaHParams, [f for f, _ in llama.LlamaHParams._fields_]),
        "p1x_llama_layer": (llama.LlamaLayer, [f for f, _ in llama.LlamaLayer._fields_]),
        "p1x_llama_model": (llama.LlamaModelC, [f for f, _ in llama.LlamaModelC._fields_]),
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "p1x.h"', "int main(void) {"]
    for name, (_, fields) in structs.items():
        lines.append(f'printf("{name} size %zu\\n", sizeof({name}));')
        for f in fields:
            lines.append(f'printf("{name} {f} %zu\\n", offsetof({name}, {f}));')
    lines.append('printf("p1x_decode_state size %zu\\n", sizeof(p1x_decode_state));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for ln in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        *key, val = ln.split()
        got[tuple(key)] = int(val)
    for name, (cls, fields) in structs.items():
        assert got[(name, "size")] == C.sizeof(cls), name
        for f in fields:
            assert got[(name, f)] == getattr(cls, f).offset, (name, f)
    assert got[("p1x_decode_state", "size")] == 16


def test_llama_workspace_without_gpu():
    """Workspace sizing is host arithmetic: 0 for invalid hyper-parameters, room for every buffer otherwise."""
    import ctypes as C

    import p100_amd
    from p100_amd import llama

    syms = p100_amd.load_symbols_only()
    ws = syms["p1x_llama_workspace"]
    ws.restype, ws.argtypes = C.c_size_t, [C.c_void_p]
    hp = llama.hparams(768)
    n = ws(C.byref(hp))
    E, F, V = 4096, 14336, 128256
    assert n >= (4 * E + (E + 2 * 1024) + 2 * F + V) * 4 + F + F // 32 * 16
    assert n < 64 << 20
    bad = [dict(n_head=3), dict(n_embd=96 * 32, n_head=32), dict(n_ff=100), dict(n_embd=32768, n_head=256),
           dict(n_layer=0)]
    for kw in bad:
        assert ws(C.byref(llama.hparams(768, **kw))) == 0, kw
    assert ws(C.byref(llama.hparams(768, embd_type=p100_amd.Q4_K))) == 0
    assert ws(C.byref(llama.hparams(768, wtype=p100_amd.Q4_K, output_type=p100_amd.Q6_K))) > 0
    am = syms["p1x_argmax_workspace"]
    am.restype, am.argtypes = C.c_size_t, [C.c_int64]
    assert am(1) == 8 and am(128256) == 256 * 8 and am(0) == 0


def _predicate_in_subprocess(env):
    """p1x_should_use_mmvh evaluated in a fresh process (the environment is read once), symbols only: no GPU."""
    import os
    import subprocess
    import sys

    code = ("import ctypes as C, p100_amd as P; f = P.load_symbols_only()['p1x_should_use_mmvh']; "
            "f.restype = C.c_int; f.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int64]; "
            "print([f(12, 1024, 14336, 4), f(12, 4096, 4096, 4), f(2, 4096, 4096, 1), f(2, 4096, 4096, 9), "
            "f(3, 64, 64, 1), f(12, 4096, 14336, 4)])")
    e = {k: v for k, v in os.environ.items() if k not in ("P1X_FORCE_MMVH", "P1X_DISABLE_MMVH")}
    e.update(env)
    out = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True, text=True, check=True,
                         cwd=str(ROOT))
    return eval(out.stdout.strip())


def test_should_use_mmvh_and_overrides():
    """The selection predicate (the counterpart of ggml_cuda_should_use_mmvh, 0005 patch :344-352): q4_K rows longer
    than 8192 at 4..8 columns prefer h16 where the int8 matrix-core form does not take them (fewer than 4096 rows);
    FORCE selects h16 for every supported shape (ncols 1..8, known type); DISABLE turns the preference off; FORCE
    wins over DISABLE, as in the reference."""
    assert _predicate_in_subprocess({}) == [1, 0, 0, 0, 0, 0]
    assert _predicate_in_subprocess({"P1X_DISABLE_MMVH": "1"}) == [0, 0, 0, 0, 0, 0]
    assert _predicate_in_subprocess({"P1X_FORCE_MMVH": "1"}) == [1, 1, 1, 0, 0, 1]
    assert _predicate_in_subprocess({"P1X_FORCE_MMVH": "1", "P1X_DISABLE_MMVH": "1"}) == [1, 1, 1, 0, 0, 1]


def test_fa_kernel_selection_and_plan_bounds_without_gpu():
    """The first-pass selection is host state: invalid values are refused; the automatic choice is the vector
    pass at every length, the forced matrix-core pass plans 4 heads per work-group and at most 256 work-groups;
    every d <= 128 plan of either kernel keeps its partials within 0.55 MiB (the no-allocation entry point's
    documented bound)."""
    import ctypes as C
    import itertools

    import p100_amd
    import oracle

    syms = p100_amd.load_symbols_only()
    sel = syms["p1x_fa_select_kernel"]
    sel.restype, sel.argtypes = C.c_int, [C.c_int]
    ws = syms["p1x_flash_attn_decode_workspace"]
    ws.restype, ws.argtypes = C.c_size_t, [C.c_void_p]

    def need(**kw):
        return ws(C.byref(p100_amd._params(oracle.AttnParams(**kw))))

    cfg = dict(n_head_q=32, n_head_kv=8, seq_q=1, d_qk=128, d_v=128, causal=True)
    try:
        assert sel(3) == p100_amd.EINVAL and sel(-1) == p100_amd.EINVAL
        assert sel(2) == p100_amd.OK
        mc = {n: need(seq_kv=n, **cfg) for n in (8192, 32768)}
        assert mc[32768] == 32 * 32 * 130 * 4  # 8 KV heads x 32 splits = 256 work-groups of 4 query heads
        assert sel(1) == p100_amd.OK
        split = {n: need(seq_kv=n, **cfg) for n in (8192, 32768)}
        assert split[32768] != mc[32768]
        assert sel(0) == p100_amd.OK
        assert need(seq_kv=8192, **cfg) == split[8192] and need(seq_kv=32768, **cfg) == split[32768]
        for kernel in (1, 2):
            assert sel(kernel) == p100_amd.OK
            for b, hkv, grp, sq, skv, d in itertools.product((1, 2, 3), (1, 4, 7, 8, 32), (1, 2, 4, 8), (1, 3),
                                                            (100, 4096, 40000), (64, 128)):
                n = need(batch=b, n_head_q=hkv * grp, n_head_kv=hkv, seq_q=sq, seq_kv=skv, d_qk=d, d_v=d)
                assert n <= 0.55 * (1 << 20), (kernel, b, hkv, grp, sq, skv, d, n)
    finally:
        sel(0)
