"""Pins the numpy oracle against the reference's own known answers and
against brute force / closed forms, so that the GPU parity tests that use it
check something real."""
import numpy as np
import pytest

from oracle import ops


def test_argmax_reference_kat():
    # reference: src/backend/mlx_metal/api_test.cc:1016-1055 and the JAX tie
    # fixture src/plugin/jax/jax_op_suite.py:125 (argmax_values).
    values = np.array([[1.0, 7.0, 7.0, 3.0], [-2.0, 5.0, 4.0, 5.0]], dtype=np.float32)
    v, i = ops.argmax_rows(values)
    np.testing.assert_array_equal(v, [7.0, 5.0])
    np.testing.assert_array_equal(i, [1, 1])
    bv, bi = ops.argmax_rows_bruteforce(values)
    np.testing.assert_array_equal(bi, [1, 1])


def test_argmax_nan_and_ties_match_bruteforce_and_numpy():
    rng = np.random.default_rng(3)
    for trial in range(40):
        x = rng.integers(-3, 4, size=(5, 17)).astype(np.float32)  # many ties
        if trial % 3 == 0:
            x[rng.integers(0, 5), rng.integers(0, 17)] = np.nan
        if trial % 5 == 0:
            x[1, :] = np.nan
        if trial % 7 == 0:
            x[2, :] = -np.inf
        v, i = ops.argmax_rows(x)
        bv, bi = ops.argmax_rows_bruteforce(x)
        np.testing.assert_array_equal(i, bi)
        np.testing.assert_array_equal(np.isnan(v), np.isnan(bv))
        np.testing.assert_array_equal(v[~np.isnan(v)], bv[~np.isnan(bv)])
        # numpy.argmax implements the same first-max / first-NaN rule.
        np.testing.assert_array_equal(i, np.argmax(x, axis=1))
        vi, ii = ops.argmax_rows(x, "min")
        np.testing.assert_array_equal(ii, np.argmin(x, axis=1))


def test_argmax_signed_zero_tie_goes_to_lower_index():
    x = np.array([[0.0, -0.0, 0.0], [-0.0, 0.0, -1.0]], dtype=np.float32)
    _, i = ops.argmax_rows(x)
    np.testing.assert_array_equal(i, [0, 0])


def test_f16_reduce_reference_kat():
    # reference: api_test.cc:930-1014: f16 {1,2,3,4} as [2,2]
    x = np.array([[1, 2], [3, 4]], dtype=np.float16)
    s, mx, mn = ops.f16_row_reduce(x)
    np.testing.assert_array_equal(s, [3, 7])
    np.testing.assert_array_equal(mx, [2, 4])
    np.testing.assert_array_equal(mn, [1, 3])
    # bf16 {1,2,3,4} (bits 0x3f80, 0x4000, 0x4040, 0x4080) sums to {3, 7}
    b = np.array([[0x3F80, 0x4000], [0x4040, 0x4080]], dtype=np.uint16)
    np.testing.assert_array_equal(ops.bf16_bits_to_f32(b).sum(axis=1), [3, 7])


def test_f16_sum_closed_form():
    # A row of n copies of c sums to n*c exactly when representable.
    x = np.full((3, 1000), 0.5, dtype=np.float16)
    s, mx, mn = ops.f16_row_reduce(x)
    np.testing.assert_array_equal(s, np.float16(500.0))
    np.testing.assert_array_equal(mx, np.float16(0.5))


def test_bf16_round_trip_and_rounding():
    x = np.array([1.0, -2.0, 3.14159, 1e-30, np.inf, -np.inf], dtype=np.float32)
    b = ops.f32_to_bf16_bits(x)
    np.testing.assert_array_equal(b[:2], [0x3F80, 0xC000])
    assert ops.bf16_bits_to_f32(b)[2] == np.float32(3.140625)
    # round-to-nearest-even on the exact halfway case 1 + 2^-8
    h = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8], dtype=np.float32)
    np.testing.assert_array_equal(ops.f32_to_bf16_bits(h), [0x3F80, 0x3F82])
    assert np.isnan(ops.bf16_bits_to_f32(ops.f32_to_bf16_bits(np.array([np.nan], np.float32))))[0]


def test_c1_closed_forms():
    # y <= 0 everywhere and x = 0: every term is 0 -> sums are 0.
    x = np.zeros((2, 8), np.float32)
    y = -np.ones((2, 8), np.float32)
    np.testing.assert_array_equal(ops.c1_rowsum(x, y), [0.0, 0.0])
    # x = 1, y = 0: term = tanh(0.5) for each element.
    x = np.ones((1, 10), np.float32)
    y = np.zeros((1, 10), np.float32)
    np.testing.assert_allclose(ops.c1_rowsum(x, y), [10 * np.tanh(0.5)], rtol=1e-15)
    # x = 1, y = 2: tanh(2.5) - 2 per element.
    y = np.full((1, 10), 2.0, np.float32)
    np.testing.assert_allclose(ops.c1_rowsum(x, y), [10 * (np.tanh(2.5) - 2.0)], rtol=1e-15)


def test_c1_matches_bruteforce_loop():
    x, y = ops.c1_inputs(3, 50, seed=5)
    import math
    want = [sum(math.tanh(float(a) * float(b) + 0.5) * float(a) - max(float(b), 0.0) for a, b in zip(xr, yr))
            for xr, yr in zip(x, y)]
    np.testing.assert_allclose(ops.c1_rowsum(x, y), want, rtol=1e-12)
