"""Pins of the oracle's single operations (CPU only).

Each check comes from outside the oracle: exact rational arithmetic for the
FMA lane order, math.fsum for the FP64 square sum, closed forms and
invariants for RoPE/softmax/SwiGLU, and NumPy's own IEEE FP16 rounding.
Every check is chosen so that a plausible slip (wrong lane combine, dropped
term, sign error, transposed index, wrong tie rule) fails it.
"""
import math
from fractions import Fraction

import numpy as np
import pytest


# ---- exact IEEE binary32 arithmetic on rationals ----
def round32(q):
    """Correctly rounded (nearest, ties to even) float32 of a Fraction."""
    f = np.float32(float(q))
    best = None
    for cand in (f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))):
        key = (abs(Fraction(float(cand)) - q), int(np.float32(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, np.float32(cand))
    return best[1]


def fma32(a, b, c):
    return round32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def add32(a, b):
    return round32(Fraction(float(a)) + Fraction(float(b)))


def dot_spec(x, w):
    """engine/core.cpp:119-127: chain c takes j % 8 == c in ascending j via
    FMA; result ((c0+c4)+(c1+c5)) + ((c2+c6)+(c3+c7))."""
    acc = [np.float32(0)] * 8
    for j in range(len(x)):
        acc[j % 8] = fma32(x[j], np.float32(w[j]), acc[j % 8])
    p = [add32(acc[c], acc[c + 4]) for c in range(4)]
    return add32(add32(p[0], p[1]), add32(p[2], p[3]))


def wide_inputs(rng, n):
    x = (rng.standard_normal(n) * 2.0 ** rng.integers(-14, 14, n)).astype(np.float32)
    w = (rng.standard_normal(n) * 0.5).astype(np.float16)
    return x, w


def test_dot_lane_order_is_exact(oracle_lib):
    rng = np.random.default_rng(11)
    distinct_from_sequential = 0
    for _ in range(40):
        x, w = wide_inputs(rng, 64)
        got = oracle_lib.dot(x, w)
        want = dot_spec(x, w)
        assert got.view(np.uint32) == want.view(np.uint32)
        seq = np.float32(0)
        for j in range(64):
            seq = fma32(x[j], np.float32(w[j]), seq)
        distinct_from_sequential += int(seq != want)
    # The inputs are adversarial enough that a single-accumulator order differs.
    assert distinct_from_sequential > 10


def test_dot_close_to_fp64(oracle_lib):
    rng = np.random.default_rng(12)
    for n in (1024, 2048, 3072):
        x = rng.standard_normal(n).astype(np.float32)
        w = (rng.standard_normal(n) * 0.02).astype(np.float16)
        exact = float(np.dot(x.astype(np.float64), w.astype(np.float64)))
        bound = n * 2.0 ** -23 * float(np.dot(np.abs(x), np.abs(w.astype(np.float32))))
        assert abs(float(oracle_lib.dot(x, w)) - exact) <= bound


def test_gemv_rows_equal_dot_and_threads(oracle_lib):
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((37, 1024)) * 0.02).astype(np.float16)
    x = rng.standard_normal(1024).astype(np.float32)
    one = oracle_lib.gemv(w, x, threads=1)
    many = oracle_lib.gemv(w, x, threads=7)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))
    for r in (0, 5, 36):
        assert one[r].view(np.uint32) == oracle_lib.dot(x, w[r]).view(np.uint32)


def test_norm_fp64_square_sum(oracle_lib):
    """engine/core.cpp:207-215 against math.fsum of the FP32 squares."""
    rng = np.random.default_rng(14)
    for n in (128, 1024):
        for _ in range(20):
            x = (rng.standard_normal(n) * 2.0 ** rng.integers(-8, 8, n)).astype(np.float32)
            w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            squares = (x * x).astype(np.float32)
            total = np.float32(math.fsum(float(v) for v in squares))
            inv = np.float32(1) / np.sqrt(total / np.float32(n) + np.float32(1e-6), dtype=np.float32)
            want = (x * inv).astype(np.float32) * w
            got = oracle_lib.norm(x, w)
            assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    x = rng.standard_normal(1024).astype(np.float32)
    y = oracle_lib.norm(x, np.ones(1024, np.float32))
    assert abs(float(np.sqrt(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 1e-5


def test_rope_tables_and_invariants(oracle_lib):
    cs, sn = oracle_lib.rope_tables(4096)
    p = np.arange(4096, dtype=np.float64)[:, None]
    angle = p / (1000000.0 ** (2.0 * np.arange(64) / 128))
    for got, want in ((cs, np.cos(angle).astype(np.float32)), (sn, np.sin(angle).astype(np.float32))):
        ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
        assert ulps.max() <= 1
    rng = np.random.default_rng(15)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal(128).astype(np.float32)
    # Position 0 is the identity, exactly.
    assert np.array_equal(oracle_lib.rope(q, cs[0], sn[0]), q)
    # Rotations preserve the norm of each (j, j+64) pair.
    r = oracle_lib.rope(q, cs[123], sn[123])
    np.testing.assert_allclose(r[:64] ** 2 + r[64:] ** 2, q[:64] ** 2 + q[64:] ** 2, rtol=1e-5, atol=1e-6)
    # Rotate-half sign convention: the first half rotates by +angle.
    expect0 = q[0] * cs[7, 0] - q[64] * sn[7, 0]
    assert abs(oracle_lib.rope(q, cs[7], sn[7])[0] - expect0) < 1e-6
    # Scores depend on relative position only.
    d1 = np.dot(oracle_lib.rope(q, cs[100], sn[100]), oracle_lib.rope(k, cs[40], sn[40]))
    d2 = np.dot(oracle_lib.rope(q, cs[1060], sn[1060]), oracle_lib.rope(k, cs[1000], sn[1000]))
    assert abs(d1 - d2) < 1e-3


def test_attention_closed_forms(oracle_lib):
    rng = np.random.default_rng(16)
    q = rng.standard_normal(128).astype(np.float32)
    keys = rng.standard_normal((1, 128)).astype(np.float16)
    values = rng.standard_normal((1, 128)).astype(np.float16)
    # One position: probability 1, output is the value row exactly.
    assert np.array_equal(oracle_lib.attention(q, keys, values), values[0].astype(np.float32))
    # Identical keys: uniform weights, output is the mean of the values.
    keys = np.repeat(keys, 33, axis=0)
    values = rng.standard_normal((33, 128)).astype(np.float16)
    np.testing.assert_allclose(oracle_lib.attention(q, keys, values), values.astype(np.float64).mean(0), atol=2e-6)
    # General case against float64 softmax attention.
    for n in (7, 300):
        keys = rng.standard_normal((n, 128)).astype(np.float16)
        values = rng.standard_normal((n, 128)).astype(np.float16)
        s = keys.astype(np.float64) @ q.astype(np.float64) / math.sqrt(128)
        p = np.exp(s - s.max())
        want = (p / p.sum()) @ values.astype(np.float64)
        np.testing.assert_allclose(oracle_lib.attention(q, keys, values), want, rtol=1e-5, atol=1e-6)


def test_swiglu_is_silu_gate(oracle_lib):
    """g * (0.5 + 0.5 tanh(g/2)) * u equals g * sigmoid(g) * u."""
    rng = np.random.default_rng(17)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    # 0.5 + 0.5 tanh(g/2) is computed near 0.5-scale, so the absolute error
    # scales with |g u| (cancellation for very negative g is inherent).
    err = np.abs(oracle_lib.swiglu(g, u) - want)
    assert np.all(err <= 4e-7 * np.abs(g.astype(np.float64) * u) + 1e-12)


def test_argmax_rules(oracle_lib):
    v = np.zeros(151936, np.float32)
    v[[5, 9, 151935]] = 3.0
    assert oracle_lib.argmax(v) == 5
    v[77] = np.float32(3.0000002)
    assert oracle_lib.argmax(v) == 77
    v[-1] = -0.0
    v[0] = 0.0
    w = np.zeros(8, np.float32)
    w[3] = -0.0
    assert oracle_lib.argmax(w) == 0
    for bad in (np.nan, np.inf, -np.inf):
        v2 = v.copy()
        v2[100] = bad
        assert oracle_lib.argmax(v2) == -1


def test_fp16_rounding_matches_ieee(oracle_lib):
    rng = np.random.default_rng(18)
    values = np.concatenate([
        (rng.standard_normal(20000) * 2.0 ** rng.integers(-30, 17, 20000)).astype(np.float32),
        np.array([65504, 65519.99, 65520, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, -0.0, 2049, 2051],
                 np.float32)])
    got = np.array([oracle_lib.lib.cpuref_f32_to_f16(float(v)) for v in values], np.uint16)
    assert np.array_equal(got, values.astype(np.float16).view(np.uint16))
    halves = np.arange(0, 65536, dtype=np.uint16)
    finite = halves[(halves & 0x7c00) != 0x7c00]
    back = np.array([oracle_lib.lib.cpuref_f16_to_f32(int(h)) for h in finite[::37]], np.float32)
    assert np.array_equal(back, finite[::37].view(np.float16).astype(np.float32))
