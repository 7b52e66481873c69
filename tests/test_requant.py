"""The requantization epilogue (no reference counterpart): hand-computed known answers
and float64 bounds.  The arithmetic is defined in include/miq_qconv.h."""
import numpy as np
import pytest

import oracle


def rq(acc, bias=0, w_scale=1.0, in_scale=1.0, out_scale=1.0, relu=False):
    a = np.array([[acc]], np.int32)
    return int(oracle.requant_i8(a, np.array([bias], np.int32), np.array([w_scale], np.float32), in_scale,
                                 out_scale, relu)[0, 0])


@pytest.mark.parametrize("acc,want", [(0, 0), (1, 0), (3, 2), (5, 2), (7, 4), (-1, 0), (-3, -2), (-5, -2), (2, 1)])
def test_ties_to_even(acc, want):
    assert rq(acc, in_scale=0.5) == want  # acc * 0.5 exactly on .5 steps


@pytest.mark.parametrize("acc,relu,want", [(1000, False, 127), (-1000, False, -128), (-1000, True, 0), (254, False, 127),
                                           (-257, False, -128), (127, False, 127), (-128, False, -128), (-1, True, 0)])
def test_saturation_and_relu(acc, relu, want):
    assert rq(acc, relu=relu) == want


def test_bias_is_added_before_scaling():
    assert rq(10, bias=-20) == -10
    assert rq(10, bias=-20, relu=True) == 0
    assert rq(-300, bias=310, in_scale=0.25) == 2   # (10) * 0.25 = 2.5 -> 2
    assert rq(0, bias=-7, in_scale=0.5) == -4       # -3.5 -> -4


def test_scale_factors():
    assert rq(100, w_scale=0.5, in_scale=0.5) == 25
    assert rq(100, in_scale=1.0, out_scale=4.0) == 25
    assert rq(100, w_scale=2.0, in_scale=0.25, out_scale=0.5) == 100


def test_large_accumulator_rounds_through_float():
    # t = 129 * 2^17 + 1 is odd and above 2^24: float(t) rounds to the even neighbour
    # 129 * 2^17, so t * 2^-18 becomes exactly 64.5 and rounds to even 64 (exact: 64.5000038 -> 65)
    t = 129 * 2 ** 17 + 1
    assert rq(t, in_scale=2.0 ** -18) == 64
    assert rq(t - 1, in_scale=2.0 ** -18) == 64
    assert rq(t + 1, in_scale=2.0 ** -18) == 65     # 129*2^17 + 2 is representable: 64.5000076 -> 65
    assert rq(-t, in_scale=2.0 ** -18) == -64


def test_int32_wraparound_of_bias_add():
    assert rq(2 ** 31 - 1, bias=1, in_scale=2.0 ** -31) == -1   # wraps to -2^31 -> -1.0


def test_non_finite_scales():
    nan, inf = float("nan"), float("inf")
    assert rq(5, w_scale=nan) == -128
    assert rq(5, w_scale=nan, relu=True) == 0
    assert rq(5, w_scale=inf) == 127
    assert rq(-5, w_scale=inf) == -128
    assert rq(0, w_scale=inf) == -128   # 0 * inf is NaN


def test_dequant_known_values():
    acc = np.array([[3, -5, 0, 7]], np.int32)
    ws = np.array([0.5, 0.5, 0.5, 0.25], np.float32)
    bias = np.array([1, 0, -2, 1], np.int32)
    y = oracle.dequant_f32(acc, bias, ws, 1.0, 1.0, False)
    np.testing.assert_array_equal(y[0], np.array([2.0, -2.5, -1.0, 2.0], np.float32))
    y = oracle.dequant_f32(acc, bias, ws, 1.0, 1.0, True)
    np.testing.assert_array_equal(y[0], np.array([2.0, 0.0, 0.0, 2.0], np.float32))
    assert not np.signbit(y[0, 1])


def test_requant_against_float64_bounds():
    rng = np.random.default_rng(11)
    k = 37
    acc = rng.integers(-3 * 10 ** 6, 3 * 10 ** 6, size=(4000, k)).astype(np.int32)
    bias = rng.integers(-1024, 1025, size=k).astype(np.int32)
    ws = rng.uniform(1e-3, 1e-2, size=k).astype(np.float32)
    in_scale, out_scale = np.float32(0.02), np.float32(1.0)
    for relu in (False, True):
        q = oracle.requant_i8(acc, bias, ws, in_scale, out_scale, relu).astype(np.int64)
        m64 = (np.float64(in_scale) / np.float64(out_scale)) * ws.astype(np.float64)
        v64 = (acc.astype(np.float64) + bias) * m64
        lo = 0 if relu else -128
        exact = np.clip(np.round(v64), lo, 127)
        assert np.abs(q - exact).max() <= 1
        # away from rounding boundaries the result is the correctly rounded exact value
        frac = np.abs(v64 - np.floor(v64) - 0.5)
        safe = frac > 1e-4
        np.testing.assert_array_equal(q[safe], exact[safe])
        deq = oracle.dequant_f32(acc, bias, ws, in_scale, out_scale, relu).astype(np.float64)
        want = np.maximum(v64, 0) if relu else v64
        assert np.all(np.abs(deq - want) <= 4 * np.finfo(np.float32).eps * np.abs(want) + 1e-30)
