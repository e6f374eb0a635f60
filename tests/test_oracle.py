"""The oracle pinned: each restated function against what fixes it independently.

Known answers from the reference's own tests, closed forms, brute force on
small inputs, and mathematical invariants, chosen so a plausible slip (a
roundf where the quantizer floors, a dropped clamp, a transposed operand, a
sum in the wrong order) fails one of them.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import reference as R
from tests.conftest import bits


# -- rounding ------------------------------------------------------------------


ROUND_VALUES = np.array([0.5, -0.5, 1.5, 2.5, -2.5, 0.49999997, -0.49999997, 1e-30, -0.0, 0.0,
                         2.0**23 + 1, -(2.0**24), 3.7, -3.7, 126.5, -126.5], dtype=np.float32)


def test_round_is_half_away_from_zero_on_the_reference_known_values():
    """The 16 values of the reference's test_int8.py:82-88, with its expected formula."""
    expected = np.array([math.copysign(math.floor(abs(v) + 0.5), v) if abs(v) < 2**23 else v
                         for v in ROUND_VALUES.astype(np.float64)], dtype=np.float32)
    assert np.array_equal(bits(R.round_half_away(ROUND_VALUES)), bits(expected))
    # and it is not NumPy's half-to-even
    assert R.round_half_away(np.float32(2.5)) == 3.0 and np.round(np.float32(2.5)) == 2.0


# -- the weight quantizer ------------------------------------------------------


def special_rows():
    """The reference's special rows (test_int8.py:69-73), seeded the same way."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((37, 70)) * 0.04).astype(np.float32)
    w[3] = 0.0
    w[5, :4] = [0.5, -0.5, 1.5, -2.5]
    w[5, 4] = 127.0 / 64
    return w


def test_quantize_int8_special_rows():
    w = special_rows()
    values, scales = R.quantize_int8(w)
    assert values.dtype == np.int8 and scales.dtype == np.float32
    assert scales[3] == 1.0 and not values[3].any()               # all-zero row: scale 1
    # row 5's magnitude is |-2.5|: that element is exactly -127 steps of 2.5/127
    assert scales[5] == np.float32(np.float32(2.5) / np.float32(127))
    assert list(values[5, :5]) == [25, -25, 76, -127, 101]        # 25.4, 76.2, 100.8 to nearest
    assert np.abs(values).max() <= 127


def test_quantize_int8_closed_form():
    """Each value is the nearest integer of w / scale, halves away from zero, in float32."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 96)) * 0.02).astype(np.float32)
    values, scales = R.quantize_int8(w)
    assert np.array_equal(scales, (np.abs(w).max(axis=1) / np.float32(127)).astype(np.float32))
    s = (w / scales[:, None]).astype(np.float32)
    assert np.all(np.abs(values.astype(np.float64) - s.astype(np.float64)) <= 0.5 + 1e-6)
    assert np.all(np.abs(values).max(axis=1) == 127)              # every row reaches its scale


def test_quantize_int8_floors_in_float32_not_roundf():
    """|s| = 0.49999997: float32 |s| + 0.5 rounds to 1.0, so the quantizer gives 1 (quantize.py:68)."""
    w = np.array([[0.49999997, 127.0, -0.49999997, 0.0]], dtype=np.float32)
    values, scales = R.quantize_int8(w)
    assert scales[0] == 1.0
    assert list(values[0]) == [1, 127, -1, 0]
    assert R.round_half_away(np.float32(0.49999997)) == 0.0       # where roundf says 0


# -- the activation quantizers ---------------------------------------------------


def test_quantize_token_is_the_block_quantizer_with_one_block():
    rng = np.random.default_rng(2)
    for k in (32, 64, 128):
        x = (rng.standard_normal((5, k)) * 3).astype(np.float32)
        x[1] = 0.0
        xq, xs = R.quantize_token(x)
        bq, bs, _ = R.quantize_blocks(x, block=k)
        assert np.array_equal(xq, bq) and np.array_equal(bits(xs), bits(bs[:, 0]))


def test_quantize_token_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((9, 896)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    x[4] = 0.0
    x[6, :3] = [127.0 * 0.5, -127.0, 63.5]                        # scale 1, exact halves
    xq, xs = R.quantize_token(x)
    assert xs[4] == 1.0 and not xq[4].any()
    assert xs[6] == 1.0 and list(xq[6, :3]) == [64, -127, 64]     # 63.5 -> 64, away from zero
    nonzero = [i for i in range(9) if i != 4]
    assert np.all(np.abs(xq[nonzero]).max(axis=1) == 127)
    # the nearest integer to x / scale, in float32
    s = (x / xs[:, None]).astype(np.float32).astype(np.float64)
    assert np.all(np.abs(xq - s) <= 0.5)


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
def test_quantizers_propagate_nan_as_the_reference_does():
    """A NaN in a row (or block) makes its scale NaN: the reference takes maxima with
    ``acc < v || v != v`` (fusion.py:603-609) and numpy's max. Its clamp is two selects
    (quantize.py:116-118), so every x / NaN becomes 127; an infinite maximum makes the
    finite values 0 and the infinite ones inf / inf = NaN -> 127. A max that skips NaN
    (fmaxf) gives a finite scale instead and fails here. The weight quantizer clips with
    numpy, whose cast of NaN to int8 is 0 on this platform."""
    x = np.ones((3, 64), np.float32)
    x[0, 5] = np.nan
    x[1, 7] = np.inf
    xq, xs = R.quantize_token(x)
    assert np.isnan(xs[0]) and np.all(xq[0] == 127)
    assert xs[1] == np.inf and xq[1, 7] == 127 and not np.delete(xq[1], 7).any()
    assert xs[2] == np.float32(1 / 127) and np.all(xq[2] == 127)
    bq, bs, off = R.quantize_blocks(x, 32)
    assert np.isnan(bs[0, 0]) and bs[0, 1] == np.float32(1 / 127) and np.isnan(off[0, 0])
    assert np.all(bq[0, :32] == 127)
    w = np.ones((2, 8), np.float32)
    w[0, 3] = np.nan
    q, s = R.quantize_int8(w)
    assert np.isnan(s[0]) and not q[0].any() and s[1] == np.float32(1 / 127)


def test_quantize_blocks_offset_is_128_times_the_scaled_block_sums():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((3, 96)) * 2).astype(np.float32)
    xq, xs, offset = R.quantize_blocks(x, 32)
    exact = 128 * np.array([sum(float(np.float32(xq[m, 32 * b:32 * b + 32].astype(np.int64).sum()) * xs[m, b])
                                for b in range(3)) for m in range(3)])
    assert np.allclose(offset[:, 0], exact, rtol=1e-6)


# -- the per-token projection ------------------------------------------------------


def test_accumulators_are_the_integer_dot_products():
    rng = np.random.default_rng(5)
    xq = rng.integers(-127, 128, (3, 37)).astype(np.int8)
    q = rng.integers(-127, 128, (5, 37)).astype(np.int8)
    acc = R.matmul_i8_token_acc(xq, q)
    for m in range(3):
        for n in range(5):
            assert acc[m, n] == sum(int(a) * int(b) for a, b in zip(xq[m], q[n]))
    assert acc.dtype == np.int32


def test_accumulator_extremes_fit_int32():
    k = 4864
    ones = np.full((1, k), 127, np.int8)
    assert R.matmul_i8_token_acc(ones, -ones)[0, 0] == -127 * 127 * k == -78_451_456


def test_epilogue_rounds_once_per_operation():
    """Each multiply and add is one correctly rounded float32 operation, in the stated order."""
    rng = np.random.default_rng(6)
    xq = rng.integers(-127, 128, (4, 300)).astype(np.int8)
    q = rng.integers(-127, 128, (6, 300)).astype(np.int8)
    xs = rng.random(4).astype(np.float32)
    ws = (rng.random(6) * 1e-3).astype(np.float32)
    bias, res = rng.standard_normal(6).astype(np.float32), rng.standard_normal((4, 6)).astype(np.float32)
    y = R.matmul_i8_token(xq, xs, q, ws, bias, res)
    acc = xq.astype(np.int64) @ q.astype(np.int64).T

    def f32(v: Fraction) -> float:            # round an exact rational to float32, ties to even
        return float(np.float32(float(v))) if v == Fraction(float(v)) else _round_f32(v)

    for m in range(4):
        for n in range(6):
            a = Fraction(float(np.float32(acc[m, n])))
            v = f32(a * Fraction(float(xs[m])))
            v = f32(Fraction(v) * Fraction(float(ws[n])))
            v = f32(Fraction(v) + Fraction(float(bias[n])))
            v = f32(Fraction(float(res[m, n])) + Fraction(v))
            assert np.float32(v) == y[m, n]


def _round_f32(v: Fraction) -> float:
    lo = np.float32(float(v))
    cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - v), int(np.array(c).view(np.uint32)) & 1))
    return float(best)


# -- rms_norm -----------------------------------------------------------------------


def test_gpu_row_sum_is_exact_when_the_arithmetic_is():
    """Powers of two that sum without rounding: every order gives the same bits."""
    rng = np.random.default_rng(7)
    v = np.ldexp(1.0, rng.integers(-10, 10, (3, 896))).astype(np.float32)
    exact = v.astype(np.float64).sum(axis=1)
    assert np.array_equal(R.gpu_row_sum(v), exact.astype(np.float32))


def test_gpu_row_sum_order_is_the_stated_tree():
    """One lane's value is reached only through its own thread and butterfly:
    a huge value in thread 0 swallows the small ones of threads 0 and 32
    before anything else is added, as the tree says."""
    v = np.zeros((1, 512), np.float32)
    v[0, 0] = 2.0**30
    v[0, 256] = 1.0        # thread 0, second element: absorbed (2^30 + 1 rounds to 2^30)
    v[0, 1] = 64.0         # thread 1: kept
    got = R.gpu_row_sum(v)[0]
    assert got == np.float32(2.0**30 + 64.0)


def test_rms_norm_orders_agree_to_rounding():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((16, 896)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    g = (1 + 0.1 * rng.standard_normal(896)).astype(np.float32)
    a, b = R.rms_norm_reference(x, g, 1e-6), R.rms_norm_gpu_order(x, g, 1e-6)
    np.testing.assert_allclose(a, b, rtol=2e-6, atol=1e-6)
    exact = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * g
    np.testing.assert_allclose(a, exact, rtol=2e-6, atol=1e-6)


# -- the host C path against the NumPy restatement -----------------------------------


@pytest.mark.parametrize("isa", [0, 1, 2, 3])
def test_host_c_is_bitwise_the_numpy_oracle_on_every_isa(host, isa):
    used = host.limit_isa(isa)
    try:
        rng = np.random.default_rng(isa)
        for m, n, k in [(1, 257, 896), (3, 40, 77), (7, 16, 4864), (2, 33, 100), (1, 1, 1)]:
            xq = rng.integers(-127, 128, (m, k)).astype(np.int8)
            q = rng.integers(-127, 128, (n, k)).astype(np.int8)
            assert np.array_equal(host.matmul_i8_token_acc(xq, q), R.matmul_i8_token_acc(xq, q)), (used, m, n, k)
            xs, ws = rng.random(m).astype(np.float32), rng.random(n).astype(np.float32)
            b, r = rng.random(n).astype(np.float32), rng.random((m, n)).astype(np.float32)
            assert np.array_equal(bits(host.matmul_i8_token(xq, xs, q, ws, b, r)),
                                  bits(R.matmul_i8_token(xq, xs, q, ws, b, r)))
    finally:
        host.limit_isa(3)


def test_host_rows_on_the_pool_are_the_serial_rows(host):
    """Config 2's host baseline with its rows spread over threads computes the serial bits, and
    the GPU-order oracle's (rows independent; 1, 8 and 13 rows cover partial and whole tasks)."""
    rng = np.random.default_rng(12)
    g = (1 + 0.1 * rng.standard_normal(896)).astype(np.float32)
    before = host.load().nc_host_threads()
    host.set_threads(4)
    try:
        for m in (1, 8, 13, 512):
            x = rng.standard_normal((m, 896)).astype(np.float32)
            x[rng.random(x.shape) < 0.01] *= 20
            serial, pooled = host.rms_norm_quant(x, g, 1e-6), host.rms_norm_quant_pool(x, g, 1e-6)
            for a, b in zip(serial, pooled):
                assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8)), m
            _, xq, xs = R.rms_norm_quant_gpu_order(x, g, 1e-6)
            assert np.array_equal(pooled[1], xq) and np.array_equal(bits(pooled[2]), bits(xs))
    finally:
        host.set_threads(before)
