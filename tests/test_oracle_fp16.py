"""FP16 helpers of the oracle, pinned by the reference's own known-answer tests.

tests/test_fp16.cpp:9-57 (bit patterns, exhaustive finite values and ties),
tests/test_tiled_model_sm60.cpp:14-39 (double -> half without double rounding, independent scalar oracle),
and bit-identity with the reference build (oracle/_ref) where it is present.
"""
import math

import numpy as np
import pytest


def bits(x):
    return int(np.float32(x).view(np.uint32))


def test_known_patterns(orc):
    r = orc.round_to_fp16
    cases = {1.0: 0x3F800000, 65504.0: 0x477FE000, 65520.0: 0x7F800000, -65520.0: 0xFF800000,
             65519.0: 0x477FE000, 6.103515625e-5: 0x38800000, 6.1e-5: 0x387FC000, 5.96e-8: 0x33800000,
             1.0 + 2.0 ** -11: 0x3F800000, 1.0 + 3 * 2.0 ** -11: 0x3F804000, 2.0 ** -25: 0,
             -(2.0 ** -25): 0x80000000, -0.0: 0x80000000, float(np.finfo(np.float32).tiny) * 2 ** -23: 0,
             float(np.finfo(np.float32).max): 0x7F800000, -math.inf: 0xFF800000}
    for x, want in cases.items():
        assert bits(r(np.float32([x]))[0]) == want, x
    nan = np.array([0xFFC12345], np.uint32).view(np.float32)
    out = r(nan)
    assert np.isnan(out[0]) and out.view(np.uint32)[0] == 0xFFC12345


def half_value_exact(b):
    e, f = b >> 10, b & 1023
    return math.ldexp(f, -24) if e == 0 else math.ldexp(1024 + f, e - 25)


def test_exhaustive_finite_and_ties(orc):
    b = np.arange(0, 0x7BFF + 1)
    v = np.array([half_value_exact(int(x)) for x in b], np.float32)
    assert (orc.round_to_fp16(v).view(np.uint32) == v.view(np.uint32)).all()
    assert (orc.round_to_fp16(-v).view(np.uint32) == (-v).view(np.uint32)).all()
    nxt = np.array([half_value_exact(int(x) + 1) for x in b[:-1]], np.float32)
    cur = v[:-1]
    mid = ((cur.astype(np.float64) + nxt) * 0.5).astype(np.float32)  # exact: one more bit than half
    even = np.where(b[:-1] & 1, nxt, cur)
    assert (orc.round_to_fp16(mid).view(np.uint32) == even.view(np.uint32)).all()
    assert (orc.round_to_fp16(-mid).view(np.uint32) == (-even).view(np.uint32)).all()
    below = np.nextafter(mid, cur)
    above = np.nextafter(mid, nxt)
    assert (orc.round_to_fp16(below).view(np.uint32) == cur.view(np.uint32)).all()
    assert (orc.round_to_fp16(above).view(np.uint32) == nxt.view(np.uint32)).all()


def scalar_half(x):
    """Independent binary16 rounding from frexp (test_tiled_model_sm60.cpp:16-27 idea)."""
    if not math.isfinite(x) or x == 0:
        return x
    a = abs(x)
    if a >= 65520:
        return math.copysign(math.inf, x)
    _, e = math.frexp(a)
    unit = math.ldexp(1.0, max(-24, e - 11))
    s = a / unit
    n = math.floor(s)
    if s - n > 0.5 or (s - n == 0.5 and n % 2 != 0):
        n += 1
    return math.copysign(n * unit, x)


def test_double_rounding(orc):
    for mid in (2.0 ** -25, 1.0 + 2.0 ** -11, 65520.0):
        for x in (mid, np.nextafter(mid, 0.0), np.nextafter(mid, math.inf)):
            for s in (1, -1):
                got = orc.round_to_fp16_f64(s * float(x))
                assert np.float32(got).view(np.uint32) == np.float32(scalar_half(s * float(x))).view(np.uint32)
    assert math.copysign(1.0, orc.round_to_fp16_f64(-0.0)) < 0
    assert math.isnan(orc.round_to_fp16_f64(math.nan))


def test_random_doubles_against_scalar(orc):
    rng = np.random.default_rng(5)
    xs = rng.standard_normal(20000) * np.exp2(rng.integers(-30, 18, 20000))
    for x in xs:
        assert orc.round_to_fp16_f64(float(x)) == np.float32(scalar_half(float(x)))


def test_half_bits_roundtrip(orc):
    for h in list(range(0, 0x7C00, 97)) + [0x7C00, 0x8001, 0xFBFF]:
        v = orc.half_value(h)
        assert orc.half_bits(v) == h


def test_bit_identical_to_reference_build(orc, ref):
    rng = np.random.default_rng(11)
    xs = rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    xs = xs[~np.isnan(xs)]  # NaN payloads do not survive the Python float round-trip
    mine = orc.round_to_fp16(xs)
    theirs = np.array([ref.L.ref_round_to_fp16_f32(float(x)) for x in xs], np.float32)
    assert (mine.view(np.uint32) == theirs.view(np.uint32)).all()
    ds = rng.standard_normal(20000) * np.exp2(rng.integers(-40, 20, 20000))
    for d in ds:
        assert orc.round_to_fp16_f64(float(d)) == ref.L.ref_round_to_fp16_f64(float(d))
    for h in range(0, 1 << 16, 7):
        a, b = orc.half_value(h), ref.L.ref_half_value(h)
        assert (math.isnan(a) and math.isnan(b)) or a == b
