"""The C++ harness drop-in (tests/harness/p100_gpu.cpp, a drop-in behind the reference's C++ harness): the
host-array calls of p100::attention_reference (include/p100/attention.h:45-49) and the q81 result of
p100::qmv::evaluate (include/p100/qmv.h:41-42), served by libp1x on the device through the C ABI.

CPU: the drop-in is built by __graft_entry__.build() and links libp1x.so (its --version makes no device call).
GPU: a causal GQA attention with an additive mask and a q6_K row run through the compiled drop-in and are
checked against the oracle with the bars of the direct tests (tolerance.h:20-31 element-wise for O and LSE; the
mat-vec row's int32 group sums bit-exact, FP32 within 1e-5 |w| |x|), and invalid parameters come back as
std::invalid_argument carrying the reference's reason string (attention_reference.cpp:89-90).
"""
import pathlib
import subprocess

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
EXE = ROOT / "tests" / "harness" / "run_harness"


def test_harness_dropin_is_built_and_links():
    import p100_amd

    assert EXE.exists(), "built by __graft_entry__.build()"
    out = subprocess.run([str(EXE), "--version"], capture_output=True, text=True, timeout=120, check=True)
    ver = p100_amd.load_symbols_only()["p1x_version"]
    ver.restype = int
    assert int(out.stdout) == ver()


def _params_line(p, has_mask):
    return (f"{p.batch} {p.n_head_q} {p.n_head_kv} {p.seq_q} {p.seq_kv} {p.d_qk} {p.d_v} {p.scale!r} "
            f"{p.softcap!r} {int(p.causal)} {int(has_mask)}\n")


@pytest.mark.gpu
def test_harness_dropin_matches_oracle(orc, tmp_path):
    d = tmp_path
    # Attention: 8 query heads over 2 KV heads, d 128, two query rows, 700 keys, causal, an additive mask with
    # masked-out keys.
    p = orc.AttnParams(n_head_q=8, n_head_kv=2, seq_q=2, seq_kv=700, d_qk=128, d_v=128, causal=True)
    nq, nk, nv, no, nl = p.shapes()
    g = np.random.default_rng(11)
    q = g.standard_normal(nq).astype(np.float32)
    k = g.standard_normal(nk).astype(np.float32)
    v = g.standard_normal(nv).astype(np.float32)
    mask = (0.5 * g.standard_normal(2 * 700)).astype(np.float32)
    mask[g.integers(0, 2 * 700, 50)] = -np.inf
    (d / "attn.txt").write_text(_params_line(p, True))
    for name, a in (("q", q), ("k", k), ("v", v), ("mask", mask)):
        a.tofile(d / f"{name}.f32")
    # A mat-vec row through the Q8_1 path: q6_K, 4096 elements.
    t = orc.TYPES["q6_K"]
    rng = orc.Rng(12)
    w = rng.random_row(t, 4096)
    x = rng.normal(4096).astype(np.float32)
    (d / "qmv.txt").write_text(f"{t} 4096\n")
    w.tofile(d / "w.bin")
    x.tofile(d / "x.f32")
    # Invalid parameters: 3 query heads over 2 KV heads.
    bad = orc.AttnParams(n_head_q=3, n_head_kv=2, seq_q=1, seq_kv=16, d_qk=128, d_v=128)
    (d / "bad.txt").write_text(_params_line(bad, False))

    print(f"run_harness {d}", flush=True)
    out = subprocess.run([str(EXE), str(d)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr

    o = np.fromfile(d / "o.f32", np.float32).astype(np.float64)
    lse = np.fromfile(d / "lse.f32", np.float32).astype(np.float64)
    ref, ref_lse = orc.attention_reference(p, q, orc.round_to_fp16(k), orc.round_to_fp16(v), mask)
    assert (np.abs(o - ref) <= 1e-3 + 2e-3 * np.abs(ref)).all()
    fin = np.isfinite(ref_lse)
    assert (np.isfinite(lse) == fin).all()
    assert (np.abs(lse[fin] - ref_lse[fin]) <= 1e-3).all()

    y = float(np.fromfile(d / "y.f32", np.float32)[0])
    sums = np.fromfile(d / "sums.i32", np.int32)
    r, ref_sums = orc.evaluate_row(t, w, x, want_sums=True)
    assert (sums == ref_sums).all()
    assert abs(y - r.q81) <= 1e-5 * r.weight_norm * np.linalg.norm(x.astype(np.float64))

    assert (d / "bad.out").read_text() == orc.validate(bad) != ""
