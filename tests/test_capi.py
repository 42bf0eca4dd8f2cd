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
