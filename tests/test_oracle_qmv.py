"""Mat-vec oracle, pinned by the reference's own outputs and by closed forms.

* docs/research/qmv-numerics-2026-10-10.txt (tests/qmv_numerics.cpp output, fixture tests/golden/qmv_numerics.txt):
  every row is regenerated from the same seeds and compared digit for digit. This pins prepare() (Q8_1 and h16),
  the q81 integer path, both h16 chain lengths, h16_exact and the exact FP64 path for q4_0 / q8_0 / q4_K.
* Bit identity with the reference build (oracle/_ref) on random rows.
* Closed forms: dequantisation by independent numpy decoders, int32 group sums as textbook sum(q*q8),
  Q8_1 special cases (all-zero block, outliers, activation ranges x1e5 / x1e-5 of bench-only 0003).
* q6_K has no reference vectors: pinned by an independent numpy decoder, FP64 brute force, and agreement of the
  q81 / h16 / exact paths within their error scale.
"""
import math

import numpy as np
import pytest

from conftest import GOLDEN


# ------------------------------------------------------------------ independent numpy decoders (ggml layouts)
def f16(b):
    return np.frombuffer(np.asarray(b, np.uint8).tobytes(), np.float16).astype(np.float64)


def dequant(orc, wtype, row):
    row = np.asarray(row, np.uint8)
    nb, bb = orc.BLOCK[wtype]
    blocks = row.reshape(-1, bb)
    out = []
    for blk in blocks:
        if wtype == orc.Q4_0:
            d = f16(blk[0:2])[0]
            qs = blk[2:18].astype(np.int64)
            q = np.concatenate([qs & 15, qs >> 4]) - 8
            out.append(d * q)
        elif wtype == orc.Q8_0:
            out.append(f16(blk[0:2])[0] * blk[2:34].view(np.int8).astype(np.int64))
        elif wtype == orc.Q4_K:
            d, dmin = f16(blk[0:4])
            sc = blk[4:16].astype(np.int64)
            qs = blk[16:144].astype(np.int64)
            for j in range(8):
                if j < 4:
                    s, m = sc[j] & 63, sc[j + 4] & 63
                else:
                    s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4)
                    m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
                q = (qs[(j // 2) * 32:(j // 2) * 32 + 32] >> (4 * (j % 2))) & 15
                out.append(d * s * q - dmin * m)
        else:  # q6_K, ggml dequantize_row_q6_K
            ql, qh = blk[0:128].astype(np.int64), blk[128:192].astype(np.int64)
            sc = blk[192:208].view(np.int8).astype(np.int64)
            d = f16(blk[208:210])[0]
            y = np.zeros(256)
            for n in range(2):
                for l in range(32):
                    is_ = l // 16
                    a, b = ql[64 * n + l], ql[64 * n + l + 32]
                    h = qh[32 * n + l]
                    y[128 * n + l] = d * sc[8 * n + is_] * (((a & 15) | (((h >> 0) & 3) << 4)) - 32)
                    y[128 * n + l + 32] = d * sc[8 * n + is_ + 2] * (((b & 15) | (((h >> 2) & 3) << 4)) - 32)
                    y[128 * n + l + 64] = d * sc[8 * n + is_ + 4] * (((a >> 4) | (((h >> 4) & 3) << 4)) - 32)
                    y[128 * n + l + 96] = d * sc[8 * n + is_ + 6] * (((b >> 4) | (((h >> 6) & 3) << 4)) - 32)
            out.append(y)
    return np.concatenate(out)


def int_operands(orc, wtype, row):
    """Integer weight operand of the Q8_1 dot per element: unsigned nibble for q4_0, else the signed q."""
    row = np.asarray(row, np.uint8)
    nb, bb = orc.BLOCK[wtype]
    res = []
    for blk in row.reshape(-1, bb):
        if wtype == orc.Q4_0:
            qs = blk[2:18].astype(np.int64)
            res.append(np.concatenate([qs & 15, qs >> 4]))
        elif wtype == orc.Q8_0:
            res.append(blk[2:34].view(np.int8).astype(np.int64))
        elif wtype == orc.Q4_K:
            qs = blk[16:144].astype(np.int64)
            res.append(np.concatenate([(qs[(j // 2) * 32:(j // 2) * 32 + 32] >> (4 * (j % 2))) & 15 for j in range(8)]))
        else:
            ql, qh = blk[0:128].astype(np.int64), blk[128:192].astype(np.int64)
            y = np.zeros(256, np.int64)
            for n in range(2):
                for l in range(32):
                    a, b, h = ql[64 * n + l], ql[64 * n + l + 32], qh[32 * n + l]
                    y[128 * n + l] = ((a & 15) | ((h & 3) << 4)) - 32
                    y[128 * n + l + 32] = ((b & 15) | (((h >> 2) & 3) << 4)) - 32
                    y[128 * n + l + 64] = ((a >> 4) | (((h >> 4) & 3) << 4)) - 32
                    y[128 * n + l + 96] = ((b >> 4) | (((h >> 6) & 3) << 4)) - 32
            res.append(y)
    return np.concatenate(res)


TYPES = ["q4_0", "q8_0", "q4_K", "q6_K"]


@pytest.mark.parametrize("tname", TYPES)
def test_exact_path_matches_independent_decoder(orc, tname):
    t = orc.TYPES[tname]
    rng = orc.Rng(99 + t)
    k = 512
    x = rng.normal(k)
    for _ in range(6):
        w = rng.random_row(t, k)
        deq = dequant(orc, t, w)
        r = orc.evaluate_row(t, w, x)
        assert r.exact == pytest.approx(float(np.dot(deq, x.astype(np.float64))), rel=1e-12, abs=1e-12)
        assert r.weight_norm == pytest.approx(float(np.linalg.norm(deq)), rel=1e-12)


@pytest.mark.parametrize("tname", TYPES)
def test_group_sums_are_textbook_integer_dots(orc, tname):
    t = orc.TYPES[tname]
    g = orc.GROUP[t]
    rng = orc.Rng(7 + t)
    for k in (256, 1024):
        w = np.stack([rng.random_row(t, k) for _ in range(5)])
        x = rng.normal(2 * k).reshape(2, k)
        x[0, :32] = 0  # an all-zero activation block: d = 0, q = 0
        x[1, 40] *= 50
        _, sums = orc.mul_mat_vec(t, w, 5, k, x, want_sums=True)
        for c in range(2):
            q8, _, _ = orc.prepare_q8_1(x[c])
            for m in range(5):
                prod = int_operands(orc, t, w[m]) * q8.astype(np.int64)
                assert (sums[c, m] == prod.reshape(-1, g).sum(1)).all()


def test_q8_1_closed_form(orc):
    rng = np.random.default_rng(4)
    for scale in (1.0, 1e5, 1e-5):
        x = (rng.standard_normal(4096) * scale).astype(np.float32)
        x[64:96] = 0
        q, d, s = orc.prepare_q8_1(x)
        xb = x.reshape(-1, 32)
        amax = np.abs(xb).max(1)
        dd = (amax / np.float32(127)).astype(np.float32)
        # round half away from zero of the IEEE quotient (std::round)
        with np.errstate(invalid="ignore", divide="ignore"):
            quo = (xb / dd[:, None]).astype(np.float32)
        want = np.where(amax[:, None] == 0, 0, np.sign(quo) * np.floor(np.abs(quo) + 0.5))
        assert (q.reshape(-1, 32) == want).all()
        assert (d == orc.round_to_fp16(dd)).all()
        assert (np.abs(q.astype(np.int64)) <= 127).all()
        assert q.reshape(-1, 32)[2].tolist() == [0] * 32 and d[2] == 0 and s[2] == 0


def test_butterfly_sum_order(orc):
    """The Q8_1 / h16 sums use the xor-butterfly order: a case where it differs from left-to-right."""
    x = np.zeros(32, np.float32)
    x[0], x[16], x[1] = 1e8, -1e8, 1.0
    x[17] = 0.75
    _, _, s = orc.prepare_q8_1(x)
    # butterfly: lane0 = (x0+x16) + (x1+x17) + ... = 0 + 1.75
    assert s[0] == np.float32(1.75)


@pytest.mark.parametrize("tname", ["q4_0", "q8_0", "q4_K"])
def test_bit_identical_to_reference_build(orc, ref, tname):
    t = orc.TYPES[tname]
    for k in (256, 4096):
        mine = orc.Rng(60060 + k + t)
        rows_ref = ref.random_rows(60060 + k + t, t, k, 6)
        rng = orc.Rng(20261010 + k)
        x = rng.normal(k)
        x[:32] = 0
        x[33] *= 50
        P = ref.prepare(x)
        q, d, s = orc.prepare_q8_1(x)
        h, sc, sm = orc.prepare_h16(x)
        assert (q == P["q"]).all() and (d == P["qd"]).all() and (s == P["qsum"]).all()
        hv = np.frombuffer(h.tobytes(), np.float16).astype(np.float32)
        assert (hv == P["h"]).all() and (sc == P["scale"]).all() and (sm == P["sum"]).all()
        for i in range(6):
            w = mine.random_row(t, k)
            assert (w == rows_ref[i]).all()
            r = orc.evaluate_row(t, w, x)
            got = np.array([r.exact, r.h16_exact, r.weight_norm, r.q81, r.h8, r.h16])
            assert (got == ref.evaluate(t, w, x)).all()


def numerics_rows(orc, k_values):
    """tests/qmv_numerics.cpp:15-61, regenerated through the oracle."""
    out = []
    for k in k_values:
        for ti, tname in enumerate(["q4_0", "q8_0", "q4_K"]):
            t = orc.TYPES[tname]
            wr = orc.Rng(60060 + k + ti)
            rows = [wr.random_row(t, k) for _ in range(256)]
            for di, dist in enumerate(["normal", "outlier", "swiglu", "large"]):
                rng = orc.Rng(20261010 + k + di)
                if di == 2:
                    draws = rng.normal(2 * k)
                    x = (draws[0::2] * (draws[1::2] * np.float32(3))).astype(np.float32)
                else:
                    x = rng.normal(k)
                if di == 3:
                    x = (x * np.float32(1000)).astype(np.float32)
                if di == 1:
                    pos = rng.shuffle_positions(k)
                    x[pos[:4]] *= np.float32(50)
                xn = math.sqrt(float(np.cumsum(x.astype(np.float64) ** 2)[-1]))
                cells = [([], []) for _ in range(4)]
                nonfinite = [0] * 4
                for w in rows:
                    r = orc.evaluate_row(t, w, x)
                    for j, path in enumerate([r.q81, r.h8, r.h16, r.h16_exact]):
                        err = abs(float(path) - r.exact)
                        scale = r.weight_norm * xn
                        cells[j][0].append(err / scale)
                        cells[j][1].append(err / max(abs(r.exact), 1e-6 * scale))
                        nonfinite[j] += not math.isfinite(path)
                for j, pname in enumerate(["q81", "h16<8>", "h16<16>", "h16_exact"]):
                    nrm, rel = sorted(cells[j][0]), sorted(cells[j][1])
                    out.append(f"{tname} {pname} {dist} {k} {(nrm[127] + nrm[128]) * 0.5:.8e} {max(nrm):.8e} "
                               f"{(rel[127] + rel[128]) * 0.5:.8e} {max(rel):.8e} {nonfinite[j]}")
    return out


def test_qmv_numerics_golden_4096(orc):
    golden = [ln for ln in (GOLDEN / "qmv_numerics.txt").read_text().splitlines() if ln.split()[3] == "4096"]
    got = numerics_rows(orc, [4096])
    assert got == golden


@pytest.mark.slow
def test_qmv_numerics_golden_14336(orc):
    golden = [ln for ln in (GOLDEN / "qmv_numerics.txt").read_text().splitlines() if ln.split()[3] == "14336"]
    assert numerics_rows(orc, [14336]) == golden


def test_q6_k_paths_agree_with_brute_force(orc):
    t = orc.Q6_K
    rng = orc.Rng(314)
    k = 1024
    for dist in range(3):
        x = rng.normal(k) * np.float32([1, 1000, 1e-3][dist])
        x = x.astype(np.float32)
        xn = float(np.linalg.norm(x.astype(np.float64)))
        for _ in range(16):
            w = rng.random_row(t, k)
            r = orc.evaluate_row(t, w, x)
            brute = float(np.dot(dequant(orc, t, w), x.astype(np.float64)))
            norm = r.weight_norm * xn
            assert abs(r.exact - brute) <= 1e-12 * norm
            assert abs(r.q81 - brute) <= 1e-3 * norm  # Q8_1 rounding of x, fp32 accumulation
            assert abs(r.h16 - brute) <= 1e-4 * norm  # fp16 chains of 8
            assert abs(r.h16_exact - brute) <= 2e-5 * norm
            assert r.h8 == r.h16  # q6_K always uses two 8-step chains


def test_q6_k_q81_equals_scaled_group_sums(orc):
    """The q6_K q81 value is sum_blocks d * sum_groups(d8 * sc * int_sum); check it against the group sums in FP64."""
    t = orc.Q6_K
    rng = orc.Rng(2718)
    k = 512
    x = rng.normal(k)
    q8, d8, _ = orc.prepare_q8_1(x)
    for _ in range(8):
        w = rng.random_row(t, k)
        r, sums = orc.evaluate_row(t, w, x, want_sums=True)
        blocks = w.reshape(-1, 210)
        total = 0.0
        for b, blk in enumerate(blocks):
            d = f16(blk[208:210])[0]
            sc = blk[192:208].view(np.int8).astype(np.float64)
            g = sums[b * 16:(b + 1) * 16].astype(np.float64)
            total += d * float(np.sum(d8[b * 8 + np.arange(16) // 2] * sc * g))
        assert abs(r.q81 - total) <= 1e-5 * (r.weight_norm * np.linalg.norm(x))


@pytest.mark.parametrize("tname", TYPES)
def test_quantizers_round_trip(orc, tname):
    t = orc.TYPES[tname]
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(4096) * 0.02).astype(np.float32)
    w = orc.quantize(t, x)
    deq = dequant(orc, t, w)
    rel = np.linalg.norm(deq - x) / np.linalg.norm(x)
    assert rel < {"q4_0": 0.12, "q8_0": 0.01, "q4_K": 0.12, "q6_K": 0.04}[tname]


def test_q4_0_quantizer_known_block(orc):
    # ggml quantize_row_q4_0_ref: d = max/-8 with max the signed value of largest magnitude.
    x = np.linspace(-1, 0.5, 32).astype(np.float32)
    w = orc.quantize(orc.Q4_0, x)
    d = f16(w[0:2])[0]
    assert d == pytest.approx(0.125, rel=1e-3)
    q = int_operands(orc, orc.Q4_0, w)
    assert q[0] == 0  # -1 / 0.125 + 8.5 = 0.5 -> 0
    assert (q >= 0).all() and (q <= 15).all()


def test_mul_mat_vec_modes_and_stride(orc):
    t = orc.Q4_0
    rng = orc.Rng(5)
    k, m = 256, 9
    w = np.stack([rng.random_row(t, k) for _ in range(m)])
    padded = np.zeros((m, w.shape[1] + 14), np.uint8)
    padded[:, :w.shape[1]] = w
    x = rng.normal(3 * k).reshape(3, k)
    for mode in ("q81", "h8", "h16", "exact"):
        y = orc.mul_mat_vec(t, w, m, k, x, mode=mode)
        y2 = orc.mul_mat_vec(t, padded, m, k, x, mode=mode, nb01=padded.shape[1])
        assert (y == y2).all()
        for c in range(3):
            for r in range(m):
                ev = orc.evaluate_row(t, w[r], x[c])
                want = {"q81": ev.q81, "h8": ev.h8, "h16": ev.h16, "exact": np.float32(ev.exact)}[mode]
                assert y[c, r] == want
    with pytest.raises(orc.OracleError):
        orc.mul_mat_vec(t, w, m, k + 1, np.zeros(k + 1, np.float32))
