"""Attention oracle (FP64 reference + tiled kernel-numerics model), pinned by the reference's own tests.

Known-answer cases: tests/test_reference.cpp:22-201, tests/test_tiled_model.cpp:13-152,
tests/test_tiled_model_split.cpp:14-41, tests/test_tiled_model_flush.cpp:14-66,
tests/test_tiled_model_sm60.cpp:41-145. Golden outputs: docs/research/error-budget-sm60-2026-10-10.txt
(tests/error_budget_sm60.cpp) and the consistency line of tests/error_budget_split.cpp:133, both as fixtures
under tests/golden/. Bit identity with the reference build (oracle/_ref) where present.
"""
import math

import numpy as np
import pytest

from conftest import GOLDEN

INF = math.inf
F32_TOL = 1e-5          # tests/check.h:23 fp32_abs_tolerance
ANALYTIC = 1e-6         # tests/check.h:24
ANALYTIC_TIGHT = 1e-7   # tests/check.h:25
OUT_ABS, OUT_REL, LSE_ABS = 1e-3, 2e-3, 1e-3  # include/p100/tolerance.h:20-22


def out_ok(got, ref):
    return np.abs(got.astype(np.float64) - ref) <= OUT_ABS + OUT_REL * np.abs(ref.astype(np.float64))


def lse_ok(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    neg = np.isneginf(ref)
    return np.where(neg, np.isneginf(got), np.abs(got - ref) <= LSE_ABS)


def small(orc, nq, nk, dq, dv):
    return orc.AttnParams(seq_q=nq, seq_kv=nk, d_qk=dq, d_v=dv, scale=1.0)


# ------------------------------------------------------------------ attention_reference KATs
def test_tiny(orc):
    p = small(orc, 2, 2, 2, 2)
    q = [1, 0, 0, 1]
    k = [math.log(np.float32(3)), 0, 0, math.log(np.float32(3))]
    k = np.array([np.log(np.float32(3)), 0, 0, np.log(np.float32(3))], np.float32)
    o, lse = orc.attention_reference(p, q, k, [2, 4, 6, 8])
    assert np.allclose(o, [3, 5, 5, 7], atol=ANALYTIC, rtol=0)
    assert np.allclose(lse, math.log(4), atol=ANALYTIC, rtol=0)
    o2, _ = orc.attention_reference(p, q, k, [2, 4, 6, 8], want_lse=False)
    assert (o == o2).all()


def test_uniform(orc):
    p = small(orc, 2, 3, 2, 3)
    p.scale = 0.0
    o, lse = orc.attention_reference(p, [0] * 4, [1, 2, 3, 4, 5, 6], [1, 2, 6, 3, 4, 0, 8, 9, -3])
    assert (o.reshape(2, 3) == [[4, 5, 1]] * 2).all()
    assert np.allclose(lse, math.log(3), atol=ANALYTIC_TIGHT, rtol=0)


def test_gqa(orc):
    p = small(orc, 2, 3, 1, 2)
    p.batch, p.n_head_q, p.n_head_kv = 2, 8, 2
    v = np.zeros((2, 2, 3, 2), np.float32)
    for b in range(2):
        for h in range(2):
            for j in range(3):
                v[b, h, j] = [100 * b + 10 * h + j, -100 * b - 10 * h - j]
    o, _ = orc.attention_reference(p, np.zeros(32), np.zeros(12), v.ravel())
    o = o.reshape(2, 8, 2, 2)
    for b in range(2):
        for h in range(8):
            e = 100 * b + 10 * (h // 4) + 1
            assert (o[b, h, :, 0] == e).all() and (o[b, h, :, 1] == -e).all()


def test_double_accumulation(orc):
    o, _ = orc.attention_reference(small(orc, 1, 2, 3, 1), [1, 1, 1], [1e8, 1, -1e8, 0, 0, 0], [0, 1])
    assert abs(o[0] - 1 / (1 + math.e)) <= ANALYTIC_TIGHT
    o, _ = orc.attention_reference(small(orc, 1, 3, 1, 1), [0], [0, 0, 0], [1e8, 1, -1e8])
    assert abs(o[0] - 1 / 3) <= ANALYTIC_TIGHT


def test_causal_bottom_right(orc):
    p = small(orc, 3, 5, 1, 1)
    p.causal = True
    o, lse = orc.attention_reference(p, [0, 0, 0], [0] * 5, [0, 2, 4, 6, 8])
    for i in range(3):
        assert o[i] == 2 + i and abs(lse[i] - math.log(3 + i)) <= ANALYTIC_TIGHT
    p.seq_q, p.seq_kv = 5, 3
    o, lse = orc.attention_reference(p, [0] * 5, [0] * 3, [0, 2, 4])
    assert (o[:2] == 0).all() and np.isneginf(lse[:2]).all()
    assert list(o[2:]) == [0, 1, 2]


def test_masked(orc):
    mask = [-INF, -INF, -INF, -INF, 0, -INF]
    o, lse = orc.attention_reference(small(orc, 2, 3, 1, 2), [1, 1], [1, 2, 3], [1, 2, 3, 4, 5, 6], mask)
    assert list(o) == [0, 0, 3, 4] and lse[0] == -INF and lse[1] == 2


def test_softcap(orc):
    p = small(orc, 1, 2, 1, 1)
    p.scale, p.softcap = 2.0, 3.0
    o, lse = orc.attention_reference(p, [10], [10, -10], [2, 9], [-4, 1])
    a = 3 * math.tanh(200 / 3) - 4
    b = 3 * math.tanh(-200 / 3) + 1
    s = math.exp(a) + math.exp(b)
    assert abs(o[0] - (2 * math.exp(a) + 9 * math.exp(b)) / s) <= ANALYTIC
    assert abs(lse[0] - math.log(s)) <= ANALYTIC_TIGHT


def test_large_logits(orc):
    p = small(orc, 1, 3, 1, 2)
    p.scale = 10000
    o, lse = orc.attention_reference(p, [1], [-1, 1, 0], [1, 2, 7, -3, 9, 10])
    assert list(o) == [7, -3] and lse[0] == 10000


def test_validation_reasons(orc):
    dims = ["batch", "n_head_q", "n_head_kv", "seq_q", "seq_kv", "d_qk", "d_v"]
    for dim in dims:
        for bad in (0, -1):
            p = orc.AttnParams()
            setattr(p, dim, bad)
            assert orc.validate(p) == "all dimensions must be positive"
            with pytest.raises(orc.OracleError, match="all dimensions must be positive"):
                orc.attention_reference(p, [0], [0], [0])
    p = orc.AttnParams(n_head_q=3, n_head_kv=2)
    assert orc.validate(p) == "n_head_q must be divisible by n_head_kv"
    for bad in (-1.0, INF, -INF, math.nan):
        assert orc.validate(orc.AttnParams(softcap=bad)) == "softcap must be finite and non-negative"
    for bad in (INF, -INF, math.nan):
        assert orc.validate(orc.AttnParams(scale=bad)) == "scale must be finite"
    assert orc.validate(orc.AttnParams(seq_q=5, seq_kv=3, causal=True, scale=-2)) == ""


# ------------------------------------------------------------------ tiled model
def _compare(orc, p, cfg, rng):
    rows = p.batch * p.n_head_q * p.seq_q
    kvr = p.batch * p.n_head_kv * p.seq_kv
    q = rng.uniform(rows * p.d_qk, -0.4, 0.4)
    k = rng.uniform(kvr * p.d_qk, -0.4, 0.4)
    v = rng.uniform(kvr * p.d_v, -0.4, 0.4)
    i = np.arange(p.seq_q)[:, None]
    j = np.arange(p.seq_kv)[None, :]
    mask = np.where((i == 1) | ((i + j) % 11 == 0), -INF, np.float32(0.03) * (j % 7)).astype(np.float32)
    ref, ref_lse = orc.attention_reference(p, q, k, v, mask)
    out, out_lse = orc.attention_tiled(p, cfg, q, k, v, mask)
    assert (np.abs(out - ref) <= F32_TOL).all()
    fin = np.isfinite(ref_lse)
    assert (np.isneginf(out_lse[~fin])).all() and (np.abs(out_lse[fin] - ref_lse[fin]) <= F32_TOL).all()
    if p.causal:
        explicit = orc.AttnParams(p.batch, p.n_head_q, p.n_head_kv, p.seq_q, p.seq_kv, p.d_qk, p.d_v, p.scale,
                                  p.softcap, False)
        m2 = np.where(j > i + (p.seq_kv - p.seq_q), -INF, mask).astype(np.float32)
        o2, l2 = orc.attention_tiled(explicit, cfg, q, k, v, m2)
        assert (o2.view(np.uint32) == out.view(np.uint32)).all()
        assert (l2.view(np.uint32) == out_lse.view(np.uint32)).all()


@pytest.mark.parametrize("dim", [64, 80, 128, 256])
def test_tiled_matrix(orc, dim):
    # test_tiled_model.cpp:49-75 with one generator shared across the dims in the reference's order.
    rng = orc.Rng(20261009)
    for d0 in [64, 80, 128, 256]:
        for nk in (1, 63, 65, 1000):
            for br in (16, 32, 64, 128):
                for bc in (16, 32, 64, 128):
                    for causal in (False, True):
                        p = orc.AttnParams(n_head_q=4, n_head_kv=2, seq_q=br + 1 if nk == 63 else 7, seq_kv=nk,
                                           d_qk=d0, d_v=13 if d0 == 80 else d0, softcap=0.7 if d0 == 80 else 0.0,
                                           causal=causal)
                        if d0 == 64 and nk == 65 and br == 16 and bc == 16:
                            p.batch, p.n_head_q = 2, 8
                        cfg = orc.TiledConfig(br, bc, False, False, False)
                        if d0 != dim:  # keep the generator in step without the cost of the check
                            rows = p.batch * p.n_head_q * p.seq_q
                            kvr = p.batch * p.n_head_kv * p.seq_kv
                            rng.uniform(rows * p.d_qk + kvr * (p.d_qk + p.d_v), -0.4, 0.4)
                            continue
                        _compare(orc, p, cfg, rng)
        if d0 == dim:
            break


def test_tiled_masked(orc):
    p = orc.AttnParams(seq_q=2, seq_kv=65, d_qk=1, d_v=2)
    q, k, v = np.ones(2), np.ones(65), np.full(130, 3.0)
    mask = np.full(130, -INF, np.float32)
    mask[65 + 64] = 0
    for rounded in (False, True):
        cfg = orc.TiledConfig(16, 64, rounded, rounded, rounded)
        o, lse = orc.attention_tiled(p, cfg, q, k, v, mask)
        assert list(o) == [0, 0, 3, 3] and lse[0] == -INF and lse[1] == 1
        o2, _ = orc.attention_tiled(p, cfg, q, k, v, mask, want_lse=False)
        assert (o == o2).all()
        pc = orc.AttnParams(seq_q=2, seq_kv=65, d_qk=1, d_v=2, causal=True)
        o3, l3 = orc.attention_tiled(pc, cfg, q, k, v, mask)
        assert (o3.view(np.uint32) == o.view(np.uint32)).all() and (l3.view(np.uint32) == lse.view(np.uint32)).all()


def test_tiled_rounding(orc):
    p = orc.AttnParams(seq_kv=2, d_qk=33, d_v=1, scale=1)
    q = np.ones(33, np.float32)
    k = np.zeros(66, np.float32)
    k[0] = 1
    k[16] = k[32] = 2.0 ** -11
    v = [0, 1]
    out, lse = orc.attention_tiled(p, orc.TiledConfig(16, 16, True, False, False), q, k, v)
    assert abs(out[0] - 1 / (1 + math.e)) <= ANALYTIC_TIGHT
    assert abs(lse[0] - (1 + math.log1p(math.exp(-1)))) <= ANALYTIC_TIGHT
    plain, _ = orc.attention_tiled(p, orc.TiledConfig(16, 16, False, False, False), q, k, v)
    assert abs(out[0] - plain[0]) > 1e-4
    k[17], k[32] = k[16], 0
    out, _ = orc.attention_tiled(p, orc.TiledConfig(16, 16, True, False, False), q, k, v)
    assert abs(out[0] - 1 / (1 + math.exp(1 + 2.0 ** -10))) <= ANALYTIC_TIGHT
    p = orc.AttnParams(seq_kv=2, d_qk=1, d_v=1, scale=1)
    k1 = np.array([0, np.log(np.float32(3))], np.float32)
    rp = float(orc.round_to_fp16(np.exp(-k1[1:2]).astype(np.float32))[0])
    expected = np.float32(rp) / (np.float32(1) + np.float32(rp))
    out, lse = orc.attention_tiled(p, orc.TiledConfig(16, 16, False, True, False), [1], k1, [1, 0])
    assert out[0] == expected
    assert lse[0] == np.float32(k1[1] + np.log(np.float32(1) + np.float32(rp)))
    out, _ = orc.attention_tiled(p, orc.TiledConfig(16, 16, False, True, True), [1], k1, [1, 0])
    assert out[0] == orc.round_to_fp16(np.float32([expected]))[0] and out[0] != expected
    wgt = orc.round_to_fp16(np.exp(np.float32([-4])))[0]
    out, lse = orc.attention_tiled(p, orc.TiledConfig(16, 1, False, True, False), [1], [4, 0], [0, 1])
    assert out[0] == wgt / (np.float32(1) + wgt)


def test_tiled_validation(orc):
    p = orc.AttnParams()
    for cfg in (orc.TiledConfig(0, 64, False, False, False), orc.TiledConfig(64, -1, False, False, False)):
        with pytest.raises(orc.OracleError):
            orc.attention_tiled(p, cfg, [0], [0], [0])
    for bits in range(8):
        cfg = orc.TiledConfig(qk_accum_fp16=bits & 1, qk_products_fp16=(bits >> 1) & 1,
                              qk_half2_chain=2 if bits & 4 else 0)
        bad = (bits & 1) + ((bits >> 1) & 1) + ((bits >> 2) & 1) > 1
        q = np.zeros(128, np.float32)
        if bad:
            with pytest.raises(orc.OracleError, match="mutually exclusive"):
                orc.attention_tiled(p, cfg, q, q, q)
        else:
            orc.attention_tiled(p, cfg, q, q, q)
    for bad in (0.0, -0.25):
        with pytest.raises(orc.OracleError):
            orc.attention_tiled(p, orc.TiledConfig(qk_q_prescale=bad), [0] * 128, [0] * 128, [0] * 128)
    for field in ("kv_parallel_blocks", "o_accum_np"):
        for bad in (0, -1):
            with pytest.raises(orc.OracleError):
                orc.attention_tiled(p, orc.TiledConfig(**{field: bad}), [0] * 128, [0] * 128, [0] * 128)


def test_split_fp32_within_tolerance(orc):
    # test_tiled_model_split.cpp:14-41: 4 parts x 4 accumulators == 1 x 1 within tolerance.h.
    p = orc.AttnParams(batch=2, n_head_q=4, n_head_kv=2, seq_q=7, seq_kv=137, d_qk=64, d_v=33)
    rng = orc.Rng(20261010)
    q = rng.uniform(2 * 4 * 7 * 64, -1, 1)
    k = rng.uniform(2 * 2 * 137 * 64, -1, 1)
    v = rng.uniform(2 * 2 * 137 * 33, -1, 1)
    mask = np.zeros((7, 137), np.float32)
    mask[0] = -INF
    mask[1, 1:] = -INF
    for causal in (False, True):
        p.causal = causal
        base, bl = orc.attention_tiled(p, orc.TiledConfig(3, 16, False, False, False), q, k, v, mask)
        out, ol = orc.attention_tiled(p, orc.TiledConfig(3, 16, False, False, False, kv_parallel_blocks=4,
                                                         o_accum_np=4), q, k, v, mask)
        assert out_ok(out, base).all() and lse_ok(ol, bl).all()


def test_half_reduction(orc):
    p = orc.AttnParams(seq_kv=3, d_qk=1, d_v=1)
    cfg = orc.TiledConfig(1, 3, False, True, False, o_accum_np=3, o_accum_fp16=True)
    out, _ = orc.attention_tiled(p, cfg, [0], [0, 0, 0], [2048, 1, 1])
    assert out[0] == np.float32(2048) / np.float32(3)
    cfg.o_accum_fp16 = 0
    out, _ = orc.attention_tiled(p, cfg, [0], [0, 0, 0], [2048, 1, 1])
    assert out[0] == np.float32(2050) / np.float32(3)


def test_flush_swamping_and_combine(orc):
    # test_tiled_model_flush.cpp:14-44
    p = orc.AttnParams(seq_kv=8192, d_qk=64, d_v=64)
    q, k, v = np.zeros(64), np.zeros(8192 * 64), np.ones(8192 * 64)
    for blocks, np_ in ((1, 1), (1, 4), (8, 1), (8, 4)):
        cfg = orc.TiledConfig(32, 64, False, True, True, o_accum_fp16=True, o_accum_fp16_tile_flush=True,
                              kv_parallel_blocks=blocks, o_accum_np=np_)
        o, _ = orc.attention_tiled(p, cfg, q, k, v)
        assert out_ok(o, np.ones_like(o)).all()
    p = orc.AttnParams(seq_kv=2, d_qk=1, d_v=1, scale=1)
    cfg = orc.TiledConfig(1, 1, False, True, False, l_from_unrounded_p=True, o_accum_fp16=True,
                          o_accum_fp16_tile_flush=True)
    o, lse = orc.attention_tiled(p, cfg, [1], [0, 1], [2, 3])
    alpha = np.exp(np.float32(-1))
    assert o[0] == (np.float32(2) * alpha + np.float32(3)) / (alpha + np.float32(1))
    assert lse_ok([lse[0]], [1 + math.log1p(math.exp(-1))]).all()
    p.seq_kv = 3
    cfg.bc = cfg.o_accum_np = 3
    o, _ = orc.attention_tiled(p, cfg, [0], [0, 0, 0], [2048, 1, 1])
    assert o[0] == np.float32(2050) / np.float32(3)


def test_flag_off_digest(orc):
    # test_tiled_model_flush.cpp:46-66: FNV-1a over every output and LSE word of the pre-flush model.
    p = orc.AttnParams(seq_q=3, seq_kv=137, d_qk=64, d_v=64)
    rng = orc.Rng(20261010)
    q = orc.round_to_fp16(rng.uniform(3 * 64, -1, 1))
    k = orc.round_to_fp16(rng.uniform(137 * 64, -1, 1))
    v = orc.round_to_fp16(rng.uniform(137 * 64, -1, 1))
    cfg = orc.TiledConfig(2, 16, False, True, False, o_accum_fp16=True, kv_parallel_blocks=3, o_accum_np=4,
                          kq_max_offset=float(np.float32(3) * np.float32(0.6931)), l_from_unrounded_p=True)
    out, lse = orc.attention_tiled(p, cfg, q, k, v)
    digest = 14695981039346656037
    for word in np.concatenate([out, lse]).view(np.uint32):
        digest = ((digest ^ int(word)) * 1099511628211) % (1 << 64)
    assert digest == 12704262495437203684


def test_sm60_scale_offset_products_chains(orc):
    # test_tiled_model_sm60.cpp:41-145
    p = orc.AttnParams(seq_q=3, seq_kv=131, d_qk=64, d_v=64)
    rng = orc.Rng(20261010)
    q = orc.round_to_fp16(rng.uniform(3 * 64, -0.5, 0.5))
    k = orc.round_to_fp16(rng.uniform(131 * 64, -0.5, 0.5))
    v = orc.round_to_fp16(rng.uniform(131 * 64, -0.5, 0.5))
    plain = dict(br=32, bc=64, qk_accum_fp16=False, p_fp16=False, o_fp16_out=False)
    base, bl = orc.attention_tiled(p, orc.TiledConfig(**plain), q, k, v)
    for mode in range(3):
        extra = [dict(qk_q_prescale=0.25), dict(qk_scale_in_q=1),
                 dict(kq_max_offset=float(np.float32(3) * np.float32(0.6931)))][mode]
        out, ol = orc.attention_tiled(p, orc.TiledConfig(**plain, **extra), q, k, v)
        if mode == 0:
            assert (np.abs(out.astype(np.float64) - base) <= 1e-6 * np.abs(base.astype(np.float64))).all()
        assert out_ok(out, base).all() and lse_ok(ol, bl).all()
    p = orc.AttnParams(d_qk=1, d_v=1, scale=0.3)
    o, l = orc.attention_tiled(p, orc.TiledConfig(**plain, qk_scale_in_q=1), [1], [1], [2])
    assert l[0] == orc.round_to_fp16(np.float32([0.3]))[0] and o[0] == 2
    p = orc.AttnParams(d_qk=7, d_v=1, scale=1)
    qv = np.array([-1.0, 1.0009765625, 1.0009765625, 0.00048828125, 0.00048828125, -0.00048828125, 0.25], np.float32)
    kv = np.array([1, 1.0009765625, 1.001953125, 1, 1, 1, 0.5], np.float32)
    prod = orc.round_to_fp16((qv * kv).astype(np.float32))
    expected = np.float32(0)
    for x in prod:
        expected = np.float32(expected + x)
    o, l = orc.attention_tiled(p, orc.TiledConfig(**plain, qk_products_fp16=1), qv, kv, [3])
    assert l[0] == expected and o[0] == 3


def test_error_budget_consistency_line(orc):
    # tests/error_budget_split.cpp:122-136, the verbatim L60 1/1 line.
    line = (GOLDEN / "error_budget_split.txt").read_text().splitlines()[0]
    assert line.startswith("consistency PASS ")
    want = line[len("consistency PASS "):]
    got = error_budget_row(orc, "L60", 0, 128, 4096, False, seq_q=16)
    assert got == want


def eb_inputs(orc, dist, dim, nk, seq_q):
    seed = 12345 + dist * 100000 + dim * 100 + nk
    rng = orc.Rng(seed)
    nq, nkv = seq_q * dim, nk * dim
    draws = rng.normal(nq + 2 * nkv)
    q, k, v = draws[:nq].copy(), draws[nq:nq + nkv].copy(), draws[nq + nkv:].copy()
    col_q, col_k = np.arange(nq) % dim, np.arange(nkv) % dim
    if dist == 1:
        q[col_q < 4] *= np.float32(20)
        k[col_k < 4] *= np.float32(20)
    if dist == 3:
        v[col_k < 8] += np.float32(2)
    return orc.round_to_fp16(q), orc.round_to_fp16(k), orc.round_to_fp16(v)


def eb_config(orc, name):
    f = float(np.float32(3) * np.float32(0.6931))
    po = dict(br=32, bc=64, qk_accum_fp16=False, p_fp16=True, o_fp16_out=True)
    l60 = dict(po, qk_scale_in_q=1, qk_q_prescale=0.25, qk_products_fp16=1, kq_max_offset=f,
               l_from_unrounded_p=1, o_accum_fp16=1)
    table = {"PO": po, "L60": l60, "L60o32": dict(l60, o_accum_fp16=0)}
    for n in (2, 4, 8):
        table[f"C{n}"] = dict(po, qk_scale_in_q=1, qk_q_prescale=0.25, qk_half2_chain=n)
    return orc.TiledConfig(**table[name])


_EB_CACHE = {}


def error_budget_row(orc, name, dist, dim, nk, causal, seq_q=16):
    key = (dist, dim, nk, causal, seq_q)
    if key not in _EB_CACHE:
        q, k, v = eb_inputs(orc, dist, dim, nk, seq_q)
        p = orc.AttnParams(seq_q=seq_q, seq_kv=nk, d_qk=dim, d_v=dim, causal=causal,
                           scale=64.0 / math.sqrt(dim) if dist == 2 else 0.0)
        if dist == 2:
            p.scale = float(np.float32(64.0) / np.sqrt(np.float32(dim)))
        ref, ref_lse = orc.attention_reference(p, q, k, v)
        _EB_CACHE.clear()
        _EB_CACHE[key] = (p, q, k, v, ref, ref_lse)
    p, q, k, v, ref, ref_lse = _EB_CACHE[key]
    out, lse = orc.attention_tiled(p, eb_config(orc, name), q, k, v)
    err = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    nonfinite = int((~np.isfinite(ref)).sum() + (~np.isfinite(out)).sum() + (~np.isfinite(ref_lse)).sum()
                    + (~np.isfinite(lse)).sum())
    max_abs, max_ref = err.max(), np.abs(ref.astype(np.float64)).max()
    mean_abs = np.cumsum(err)[-1] / err.size
    lse_abs = np.abs(lse.astype(np.float64) - ref_lse.astype(np.float64)).max()
    max_rel = 0 if max_ref == 0 else max_abs / max_ref
    return (f"{name} {['normal', 'outlier', 'peaked', 'vbias'][dist]} {dim} {nk} {int(causal)} "
            f"{max_abs:.6e} {max_rel:.6e} {mean_abs:.6e} {lse_abs:.6e} {nonfinite}")


def _golden_eb(kvs):
    rows = []
    for ln in (GOLDEN / "error_budget_sm60.txt").read_text().splitlines():
        f = ln.split()
        if int(f[3]) in kvs:
            rows.append(ln)
    return rows


DISTS = {"normal": 0, "outlier": 1, "peaked": 2, "vbias": 3}


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_error_budget_sm60_golden_short(orc, dim):
    """Every error_budget_sm60 row at 512 keys for this head size reproduces the committed output exactly."""
    rows = [r for r in _golden_eb({512}) if int(r.split()[2]) == dim]
    assert rows
    bad = []
    for row in rows:
        f = row.split()
        got = error_budget_row(orc, f[0], DISTS[f[1]], dim, int(f[3]), f[4] == "1")
        if got != row:
            bad.append((row, got))
    assert not bad, bad[:4]


@pytest.mark.slow
def test_error_budget_sm60_golden_4096(orc):
    rows = _golden_eb({4096})
    bad = []
    for row in rows:
        f = row.split()
        got = error_budget_row(orc, f[0], DISTS[f[1]], int(f[2]), int(f[3]), f[4] == "1")
        if got != row:
            bad.append((row, got))
    assert not bad, bad[:4]


def test_bit_identical_to_reference_build(orc, ref):
    rng = np.random.default_rng(3)
    for trial in range(40):
        hkv = int(rng.integers(1, 3))
        p = orc.AttnParams(batch=int(rng.integers(1, 3)), n_head_q=hkv * int(rng.integers(1, 3)), n_head_kv=hkv,
                           seq_q=int(rng.integers(1, 9)), seq_kv=int(rng.integers(1, 150)),
                           d_qk=int(rng.choice([1, 7, 32, 64])), d_v=int(rng.choice([1, 13, 64])),
                           scale=float(rng.choice([0.0, 0.3, 2.0])), softcap=float(rng.choice([0.0, 0.7])),
                           causal=bool(rng.integers(0, 2)))
        nq, nk, nv, _, _ = p.shapes()
        q = orc.round_to_fp16(rng.standard_normal(nq).astype(np.float32))
        k = orc.round_to_fp16(rng.standard_normal(nk).astype(np.float32))
        v = orc.round_to_fp16(rng.standard_normal(nv).astype(np.float32))
        mask = None
        if trial % 3 == 0:
            mask = rng.standard_normal(p.seq_q * p.seq_kv).astype(np.float32)
            mask[rng.random(mask.size) < 0.2] = -INF
        a = orc.attention_reference(p, q, k, v, mask)
        b = ref.attention_reference(p, q, k, v, mask)
        assert all((x.view(np.uint32) == y.view(np.uint32)).all() for x, y in zip(a, b))
        cfg = orc.TiledConfig(int(rng.choice([1, 2, 16])), int(rng.choice([1, 3, 16, 64])),
                              bool(trial % 5 == 1), bool(rng.integers(0, 2)), bool(rng.integers(0, 2)),
                              qk_scale_in_q=int(trial % 4 == 2), qk_q_prescale=float(rng.choice([1.0, 0.25])),
                              qk_products_fp16=int(trial % 7 == 3), qk_half2_chain=int(trial % 6 == 4) * 2,
                              kq_max_offset=float(rng.choice([0.0, 2.0793])),
                              l_from_unrounded_p=int(rng.integers(0, 2)), o_accum_fp16=int(rng.integers(0, 2)),
                              kv_parallel_blocks=int(rng.integers(1, 4)), o_accum_np=int(rng.integers(1, 4)),
                              o_accum_fp16_tile_flush=int(rng.integers(0, 2)))
        modes = cfg.qk_accum_fp16 + cfg.qk_products_fp16 + (cfg.qk_half2_chain > 0)
        if modes > 1:
            continue
        a = orc.attention_tiled(p, cfg, q, k, v, mask)
        b = ref.attention_tiled(p, cfg, q, k, v, mask)
        assert all((x.view(np.uint32) == y.view(np.uint32)).all() for x, y in zip(a, b)), trial


# ------------------------------------------------------------------ CPU decode attention (fa_decode_f32)
@pytest.mark.parametrize("nthreads", [1, 8])
def test_fa_decode_f32_matches_reference(orc, nthreads):
    """The ggml-style CPU decode attention (fp16 K/V, FP32 online softmax per KV chunk, log-sum-exp merge of the
    chunks) against the FP64 reference within tolerance.h, at the decode shape (32/8 heads, d 128, 8192 keys,
    causal). One thread keeps a single chunk; eight threads merge eight, so a wrong rescale or merge fails."""
    p = orc.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=8192, d_qk=128, d_v=128, causal=True)
    rng = np.random.default_rng(8192)
    q = rng.standard_normal(32 * 128).astype(np.float32)
    k16 = rng.standard_normal(8 * 8192 * 128).astype(np.float16)
    v16 = rng.standard_normal(8 * 8192 * 128).astype(np.float16)
    q[:128] *= 8  # one head with peaked logits: the running max moves late and far
    o, lse = orc.fa_decode_f32(p, q, k16.view(np.uint16), v16.view(np.uint16), nthreads=nthreads)
    ref, ref_lse = orc.attention_reference(p, q, k16.astype(np.float32), v16.astype(np.float32))
    assert out_ok(o, ref).all(), np.abs(o - ref).max()
    assert lse_ok(lse, ref_lse).all()
    assert np.abs(o - ref).max() / np.abs(ref).max() <= 2e-3


def test_fa_decode_f32_masked_rows_and_softcap(orc):
    """Two query rows over 600 keys with an additive mask that hides every key of row 0 (O = 0, LSE = -inf) and
    half of row 1, and a logit softcap; chunks merged over 4 threads."""
    p = orc.AttnParams(n_head_q=4, n_head_kv=2, seq_q=2, seq_kv=600, d_qk=64, d_v=64, softcap=5.0)
    rng = np.random.default_rng(600)
    q = rng.standard_normal(4 * 2 * 64).astype(np.float32) * 2
    k16 = rng.standard_normal(2 * 600 * 64).astype(np.float16)
    v16 = rng.standard_normal(2 * 600 * 64).astype(np.float16)
    mask = np.zeros((2, 600), np.float32)
    mask[0, :] = -np.inf
    mask[1, ::2] = -np.inf
    mask[1, 1::4] = -1.5
    o, lse = orc.fa_decode_f32(p, q, k16.view(np.uint16), v16.view(np.uint16), mask=mask, nthreads=4)
    ref, ref_lse = orc.attention_reference(p, q, k16.astype(np.float32), v16.astype(np.float32), mask=mask)
    assert out_ok(o, ref).all()
    assert lse_ok(lse, ref_lse).all()
    rows = o.reshape(4, 2, 64)
    assert (rows[:, 0] == 0).all() and np.isneginf(lse.reshape(4, 2)[:, 0]).all()


def test_weight_norms_match_evaluate_row(orc):
    """weight_norms is evaluate_row's weight_norm for every row, bit for bit, including a padded row stride."""
    for tname in ("q4_0", "q8_0", "q4_K", "q6_K"):
        t = orc.TYPES[tname]
        k = 512
        r = orc.Rng(77 + t)
        w = np.stack([r.random_row(t, k) for _ in range(9)])
        want = np.array([orc.evaluate_row(t, w[i], np.zeros(k, np.float32)).weight_norm for i in range(9)])
        assert np.array_equal(orc.weight_norms(t, w, 9, k), want), tname
        pad = np.zeros((9, w.shape[1] + 6), np.uint8)
        pad[:, :w.shape[1]] = w
        assert np.array_equal(orc.weight_norms(t, pad, 9, k, nb01=w.shape[1] + 6), want), tname
