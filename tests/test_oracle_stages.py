"""Pins of the oracle's stage functions that do not retype them: exact rational arithmetic (fractions), library
routines (numpy argmax, int64 matrix products, math.erf), closed forms (log2, 2^x, the layer-norm spread) and
special cases.  A planted mistake in a copy of each stage must fail its pin (negative controls)."""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest


@pytest.fixture(scope="module")
def tabs(sm):
    return sm.tables()


@pytest.fixture(scope="module")
def st(tabs):
    import oracle
    return oracle.Stages(tabs)


def round_half_up(q: Fraction) -> int:
    return math.floor(q + Fraction(1, 2))


# ---------------------------------------------------------------- rshift (base2.py:18-22)
def test_rshift_is_rounding_to_nearest_ties_up(st):
    rng = np.random.default_rng(1)
    x = rng.integers(-2 ** 40, 2 ** 40, 3000)
    s = rng.integers(-15, 40, 3000)
    got = st.rshift(x, s)
    want = [round_half_up(Fraction(int(a), 1) / Fraction(2) ** int(b)) for a, b in zip(x, s)]
    assert [int(v) for v in got] == want


def test_rshift_ties_and_signs(st):
    # -2.5 -> -2, -1.5 -> -1, 1.5 -> 2, 2.5 -> 3 (half up, also for negatives)
    assert list(st.rshift(np.array([-5, -3, 3, 5]), 1)) == [-2, -1, 2, 3]
    assert list(st.rshift(np.array([7]), 0)) == [7]
    assert list(st.rshift(np.array([-7]), -3)) == [-56]


def test_rshift_numpy_wrap_semantics(st):
    # numpy int64: a left shift by >= 64 gives 0, a right shift by >= 64 gives 0 or -1, sums wrap
    x = np.array([5, -5, 2 ** 62, -(2 ** 62), 2 ** 63 - 1], np.int64)
    assert list(st.rshift(x, -64)) == [0, 0, 0, 0, 0]
    assert list(st.rshift(x, 70)) == [0, -1, 0, -1, 0]
    assert list(st.rshift(x, -2)) == list(np.left_shift(x, 2))          # wraps like numpy
    assert list(st.rshift(np.array([2 ** 63 - 1]), 1)) == [-(2 ** 62)]   # the +half wraps first, then the shift


# ---------------------------------------------------------------- to16 (base2.py:24-27)
def test_to16_definition(st):
    rng = np.random.default_rng(2)
    X = rng.integers(-2 ** 35, 2 ** 35, (50, 300)) >> rng.integers(0, 35, (50, 1))
    X[0] = 0
    X[1] = 0
    X[1, :3] = [65535, -3, 4]          # rounds up to +32768
    x16, ex = st.to16(X, -16)
    for r in range(len(X)):
        top = max(abs(int(v)) for v in X[r]).bit_length()        # bit length of the max = bit length of the OR
        sh = max(top - 15, 0)
        assert ex[r] == -16 + sh
        assert [int(v) for v in x16[r]] == [round_half_up(Fraction(int(v), 2 ** sh)) for v in X[r]]
    assert x16[1, 0] == 32768 and np.abs(x16).max() <= 32768


# ---------------------------------------------------------------- log2fix (base2.py:42-48)
def test_log2fix_exact_below_2_17(st, tabs):
    v = np.arange(1, 1 << 17, 7, dtype=np.int64)
    got = st.log2fix(v)
    want = [round(65536 * math.log2(int(a))) for a in v]
    diff = np.abs(np.array(want) - got)
    assert diff.max() <= 1 and np.mean(diff == 0) > 0.999      # the table is round(log2(1 + m/65536) 65536)


def test_log2fix_close_to_log2(st):
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.integers(1, 2 ** 62, 5000), 2 ** np.arange(0, 62)])
    got = st.log2fix(v)
    err = got - np.array([65536 * math.log2(int(a)) for a in v])
    assert err.max() <= 0.51 and err.min() >= -1.45 - 0.51       # mantissa truncated to 16 bits, table rounded
    assert all(int(st.log2fix(np.array([2 ** k]))[0]) == 65536 * k for k in range(62))


# ---------------------------------------------------------------- power (base2.py:50-53)
def test_power_whole_powers_are_exact(st):
    rng = np.random.default_rng(4)
    x = rng.integers(-2 ** 40, 2 ** 40, 2000)
    k = rng.integers(-30, 8, 2000)
    got = st.power(x, k * 65536)
    assert [int(g) for g in got] == [round_half_up(Fraction(int(a)) * Fraction(2) ** int(b)) for a, b in zip(x, k)]


def test_power_close_to_two_to_the_f(st):
    rng = np.random.default_rng(5)
    x = rng.integers(-2 ** 30, 2 ** 30, 5000)
    F = rng.integers(-20 * 65536, 10 * 65536, 5000)
    got = st.power(x, F).astype(np.float64)
    want = x.astype(np.float64) * np.exp2(F / 65536.0)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -16 + 1.0)


# ---------------------------------------------------------------- race (base2.py:34-40)
def test_race_is_first_argmax(st):
    rng = np.random.default_rng(6)
    for n in (1, 2, 17, 1000, 50257):
        v = rng.integers(-50, 50, n)
        assert st.race(v) == int(np.argmax(v))
    v = np.array([-(2 ** 63), 2 ** 63 - 1, 2 ** 63 - 1, 0], np.int64)
    assert st.race(v) == 1


# ---------------------------------------------------------------- edge (base2.py:78-83)
def test_edge_is_gelu(st):
    h = np.arange(-(2 ** 19), 2 ** 19, 37, dtype=np.int64)
    got = st.edge(h) / 65536.0
    x = h / 65536.0
    gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x])
    assert np.abs(got - gelu).max() < 2e-3 * 8          # the share is read at 2^-12 steps of x
    big = np.array([2 ** 19 + 16, 2 ** 25, -(2 ** 19) - 17, -(2 ** 30)], np.int64)
    assert list(st.edge(big)) == [2 ** 19 + 16, 2 ** 25, 0, 0]   # past the table: the share is 1 or 0


# ---------------------------------------------------------------- gauge_log (base2.py:55-60)
def test_gauge_is_log2_of_the_spread(st):
    rng = np.random.default_rng(7)
    R = (rng.standard_normal((40, 768)) * rng.choice([50.0, 2000.0, 2.0 ** 18], (40, 1)) + rng.integers(-500, 500, (40, 1))).astype(np.int64)
    x16, ex, LS = st.gauge_log(R)
    for r in range(len(R)):
        x = R[r] / 65536.0
        sigma = math.sqrt(np.var(x) + 1e-5)
        # LS is log2(sigma) in units of 2^-16 octave (the variance is taken at the light's 16-bit resolution)
        assert abs(LS[r] / 65536.0 - math.log2(sigma)) < 3e-3 + 2.0 ** (-14 + ex[r] + 16) / sigma


# ---------------------------------------------------------------- product (base2.py:29-32)
def test_product_is_int64_matmul(st):
    rng = np.random.default_rng(8)
    x = rng.integers(-32768, 32769, (3, 3072))
    w = rng.integers(-32768, 32768, (3072, 700)).astype(np.int16)
    assert np.array_equal(st.product(x, w), x @ w.astype(np.int64))


# ---------------------------------------------------------------- tables (base2_convert.py:48-61)
def test_tables_constants(tabs):
    assert len(tabs["arrival"]) == 17745
    assert int(tabs["log2_768"]) == 628160
    assert int(tabs["eps40"]) == 6485183463414
    assert tabs["arrival"][0] == 2 ** 24 and tabs["arrival"][-1] >= 1
    assert np.all(np.diff(tabs["arrival"]) <= 0)
    assert abs(tabs["arrival"][1024] - 2 ** 24 / math.e) <= 0.5
    phi = tabs["phi"]
    assert phi[32768] == 32768 and phi[0] == 0 and phi[-1] == 65536 and np.all(np.diff(phi) >= 0)
    assert tabs["log2"][0] == 0 and tabs["exp2"][0] == 65536 and tabs["exp2"][-1] == 131071
    f = np.arange(0, 65536, 97)
    assert np.abs(tabs["exp2"][f] - np.exp2(f / 65536.0) * 65536).max() <= 0.5


# ---------------------------------------------------------------- negative controls: planted mistakes fail the pins
def test_planted_mistakes_are_caught(st, tabs):
    rng = np.random.default_rng(9)
    x = rng.integers(-2 ** 20, 2 ** 20, 500)
    truncating = np.right_shift(x, 3)                               # rshift without the half
    exact = [round_half_up(Fraction(int(a), 8)) for a in x]
    assert [int(v) for v in truncating] != exact
    v = np.array([3, 9, 9, 1])
    assert len(v) - 1 - int(np.argmax(v[::-1])) != st.race(v)         # ties to the last index
    h = np.arange(-(2 ** 18), 2 ** 18, 101, dtype=np.int64)
    share = tabs["phi"][np.clip(st.rshift(h, 3) + 32768, 0, 65535)]          # the share read at the wrong scale
    wrong = st.rshift(h * share, 16) / 65536.0
    x = h / 65536.0
    gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x])
    assert np.abs(wrong - gelu).max() > 2e-3 * 8
