"""Pins of oracle/frontend.py (reduce_precision, reduce_window) against
independent answers: numpy's own conversions, closed forms and the
reference's import case; plus the frontend's parsing of the widened ops
(no GPU: plan structure only)."""
import json

import numpy as np
import pytest

from oracle import frontend as F
from oracle import ops
from pjrtx_amd.hlo import Builder


def test_reduce_precision_e8m7_is_bf16_rounding():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(4096) * np.exp(rng.uniform(-30, 30, 4096))).astype(np.float32)
    got = F.reduce_precision(x, "f32", 8, 7)
    want = ops.bf16_bits_to_f32(ops.f32_to_bf16_bits(x))
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_reduce_precision_e5m10_is_f16_conversion_in_the_normal_range():
    rng = np.random.default_rng(1)
    x = (rng.uniform(-1, 1, 4096) * np.exp2(rng.uniform(-13.5, 15.5, 4096))).astype(np.float32)
    x = x[np.abs(x) >= np.float32(2.0 ** -14)]
    got = F.reduce_precision(x, "f32", 5, 10)
    want = x.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got, want)


def test_reduce_precision_special_cases():
    x = np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 1e6, -1e6, 2.0 ** -14, 2.0 ** -15, -2.0 ** -20, np.inf,
                  -np.inf, np.nan], np.float32)
    got = F.reduce_precision(x, "f32", 5, 10)
    want = np.array([0.0, -0.0, 1.0, 65504.0, np.inf, np.inf, -np.inf, 2.0 ** -14, 0.0, -0.0, np.inf, -np.inf,
                     np.nan], np.float32)
    np.testing.assert_array_equal(got, want)
    assert np.signbit(got[9]) and np.signbit(got[1])
    # the type's own format is the identity (the reference's e8m23 case)
    y = np.random.default_rng(2).standard_normal(100).astype(np.float32)
    np.testing.assert_array_equal(F.reduce_precision(y, "f32", 8, 23), y)
    h = np.array([6.1e-5, 5.96e-8, 1.0, -3.0, 65504.0], np.float16)  # f16 subnormals stay at e5m10
    np.testing.assert_array_equal(F.reduce_precision(h, "f16", 5, 10), h)
    # zero mantissa bits: powers of two; a tie goes to the even biased
    # exponent (3 = 1.5 * 2^1, exponent 128: down to 2; 6 = 1.5 * 2^2,
    # exponent 129: up to 8)
    z = F.reduce_precision(np.array([1.4, 1.5, 1.6, 3.0, 5.0, 6.0], np.float32), "f32", 8, 0)
    np.testing.assert_array_equal(z, np.array([1.0, 2.0, 2.0, 2.0, 4.0, 8.0], np.float32))


def test_reduce_window_reference_import_case():
    # stablehlo_import_tests.zig:173-207: window 2, stride 1, padding [1, 0] over [3]
    x = np.array([1.5, 2.0, -4.0], np.float32)
    got = F.reduce_window(x, 0.0, "add", [2], padding=[(1, 0)])
    np.testing.assert_array_equal(got, np.array([1.5, 3.5, -2.0], np.float32))


def test_reduce_window_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.integers(-50, 50, 40).astype(np.int64)
    got = F.reduce_window(x, 0, "add", [5])
    c = np.concatenate([[0], np.cumsum(x)])
    np.testing.assert_array_equal(got, c[5:] - c[:-5])
    y = rng.standard_normal((9, 11)).astype(np.float32)
    got = F.reduce_window(y, -np.inf, "maximum", [3, 4], strides=[2, 3])
    want = np.lib.stride_tricks.sliding_window_view(y, (3, 4)).max(axis=(2, 3))[::2, ::3]
    np.testing.assert_array_equal(got, want)
    # dilation: every other element
    got = F.reduce_window(x, 0, "add", [3], window_dilations=[2])
    want = x[:-4] + x[2:-2] + x[4:]
    np.testing.assert_array_equal(got, want)


def _plan(plugin, text):
    return json.loads(plugin.plan_json(text))["steps"]


def test_frontend_ops_plan(plugin):
    b = Builder(mesh='["x"=1]')
    x = b.param((4, 6), "f32")
    y = b.reduce_precision(x, 5, 10)
    z = b.reduce_precision(y, 8, 7, generic=True)
    u, v = b.optimization_barrier([z, x])
    w = b.sharding_constraint(u)
    rw = b.reduce_window(w, b.constant(0.0, "f32"), "add", [2, 3], strides=[1, 2], padding=[(1, 0), (0, 1)])
    steps = _plan(plugin, b.build([rw, v]))
    assert [s["kind"] for s in steps] == ["loop", "library"]
    assert steps[0]["ops"] == ["reduce_precision", "reduce_precision"]
    assert steps[1]["library"] == "reduce_window"


def test_reference_import_cases_parse(plugin):
    # stablehlo_import_tests.zig:364-380 (sdy mesh prefix), 386-408 (barrier
    # with two results), 173-207 (reduce_window metadata), 278 (e8m23)
    text = """sdy.mesh @mesh = <["x"=2]>
func.func @main(%arg0: tensor<4xf32> {sdy.sharding = #sdy.sharding<@mesh, [{"x"}]>}) -> tensor<4xf32> {
  %0 = stablehlo.add %arg0, %arg0 : tensor<4xf32>
  return %0 : tensor<4xf32>
}"""
    assert [s["kind"] for s in _plan(plugin, text)] == ["loop"]
    text = """sdy.mesh @mesh = <["x"=2]>
func.func @main(%arg0: tensor<4xf32>, %arg1: tensor<4xf32>) -> (tensor<4xf32>, tensor<4xf32>) {
  %0, %1 = "stablehlo.optimization_barrier"(%arg0, %arg1) : (tensor<4xf32>, tensor<4xf32>) -> (tensor<4xf32>, tensor<4xf32>)
  return %0, %1 : tensor<4xf32>, tensor<4xf32>
}"""
    assert all(s["kind"] in ("alias", "library") for s in _plan(plugin, text))
    text = """module {
  func.func @main(%arg0: tensor<3xf32>) -> tensor<3xf32> {
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = "stablehlo.reduce_window"(%arg0, %cst) ({
    ^bb0(%lhs: tensor<f32>, %rhs: tensor<f32>):
      %sum = stablehlo.add %lhs, %rhs : tensor<f32>
      stablehlo.return %sum : tensor<f32>
    }) {
      base_dilations = array<i64: 1>,
      padding = dense<[[1, 0]]> : tensor<1x2xi64>,
      window_dimensions = array<i64: 2>,
      window_dilations = array<i64: 1>,
      window_strides = array<i64: 1>
    } : (tensor<3xf32>, tensor<f32>) -> tensor<3xf32>
    return %0 : tensor<3xf32>
  }
}"""
    steps = _plan(plugin, text)
    assert [s.get("library") for s in steps] == ["reduce_window"]
    text = """module {
  func.func @main(%arg0: tensor<2x2xf32>) -> tensor<2x2xf32> {
    %0 = "stablehlo.reduce_precision"(%arg0) <{exponent_bits = 8 : i32, mantissa_bits = 23 : i32}> : (tensor<2x2xf32>) -> tensor<2x2xf32>
    return %0 : tensor<2x2xf32>
  }
}"""
    assert [s["ops"] for s in _plan(plugin, text)] == [["reduce_precision"]]


def test_unsupported_reduce_window_fails_closed(plugin):
    b = Builder()
    x = b.param((8,), "f32")
    y = b.reduce_window(x, b.constant(0.0, "f32"), "add", [2], window_dilations=[0])
    with pytest.raises(Exception, match="positive"):
        _plan(plugin, b.build([y]))
    b = Builder()
    x = b.param((8,), "s32")
    i = b.param((8,), "s32")
    v, k = b.reduce_window_arg(x, i, b.constant(0, "s32"), b.constant(0, "s32"), [2])
    with pytest.raises(Exception, match="argmax|value type"):
        _plan(plugin, b.build([v, k]))


def test_reduce_window_base_dilation_closed_forms():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(7).astype(np.float32)
    # window 1: the input placed every b-th position of a zero array
    for bd in (2, 3):
        got = F.reduce_window(x, 0.0, "add", [1], base_dilations=[bd])
        want = np.zeros((len(x) - 1) * bd + 1, np.float32)
        want[::bd] = x
        np.testing.assert_array_equal(got, want)
    # window 2, base dilation 2: [x0, x1, x1, x2, x2, ...]
    got = F.reduce_window(x, 0.0, "add", [2], base_dilations=[2])
    np.testing.assert_array_equal(got, x[(np.arange(2 * len(x) - 2) + 1) // 2])
    # 2-D, with padding: every window of the dilated, padded array
    y = rng.integers(-9, 9, (4, 5)).astype(np.int32)
    dil = np.zeros((7, 13), np.int32)
    dil[::2, ::3] = y
    padded = np.pad(dil, ((1, 2), (0, 1)))
    want = np.lib.stride_tricks.sliding_window_view(padded, (3, 2)).sum(axis=(2, 3))[::1, ::2]
    got = F.reduce_window(y, 0, "add", [3, 2], strides=[1, 2], padding=[(1, 2), (0, 1)], base_dilations=[2, 3])
    np.testing.assert_array_equal(got, want)


def test_reduce_window_negative_padding_crops():
    x = np.arange(10, dtype=np.float32)
    got = F.reduce_window(x, 0.0, "add", [1], padding=[(-2, -3)])
    np.testing.assert_array_equal(got, x[2:-3])
    got = F.reduce_window(x, -np.inf, "maximum", [3], padding=[(-1, 2)])
    want = np.lib.stride_tricks.sliding_window_view(np.pad(x[1:], (0, 2), constant_values=-np.inf), 3).max(-1)
    np.testing.assert_array_equal(got, want)


def test_reduce_window_arg_matches_numpy_argmax():
    rng = np.random.default_rng(6)
    x = rng.integers(-3, 4, (5, 12)).astype(np.float32)   # many ties
    x[1, 4] = np.nan
    x[3, 7] = np.nan
    x[3, 9] = np.nan
    idx = np.broadcast_to(np.arange(12, dtype=np.int32), x.shape).copy()
    for kind in ("max", "min"):
        v, i = F.reduce_window_arg(x, idx, -np.inf if kind == "max" else np.inf, 0, kind, [1, 4], strides=[1, 2])
        win = np.lib.stride_tricks.sliding_window_view(x, (1, 4))[:, ::2, 0, :]
        # numpy: first extreme (NaN counts as the extreme); the index is the
        # window start plus the position in the window
        pos = np.argmax(win, -1) if kind == "max" else np.argmin(win, -1)
        start = np.arange(win.shape[1]) * 2
        np.testing.assert_array_equal(i, start[None, :] + pos)
        np.testing.assert_array_equal(v, np.take_along_axis(win, pos[..., None], -1)[..., 0])
    # padding contributes (-inf, 0): an all-padding window returns it
    v, i = F.reduce_window_arg(x[:1, :3], idx[:1, :3], -np.inf, 0, "max", [1, 2], padding=[(0, 0), (2, 0)])
    np.testing.assert_array_equal(i[0, 0], 0)
    assert v[0, 0] == -np.inf


def test_reduce_window_arg_reference_op_suite_case():
    # jax_op_suite.py:122 (f32_a) and 294-310: window (1, 2), stride 1, VALID,
    # indices = arange(4) per row; f32_a has no ties, so every rule agrees
    x = (np.arange(12, dtype=np.float32).reshape(3, 4) - np.float32(3.0)) / np.float32(7.0)
    idx = np.broadcast_to(np.arange(4, dtype=np.int32), x.shape).copy()
    v, i = F.reduce_window_arg(x, idx, -np.inf, 0, "max", [1, 2])
    np.testing.assert_array_equal(v, x[:, 1:])
    np.testing.assert_array_equal(i, np.broadcast_to(np.arange(1, 4, dtype=np.int32), (3, 3)))


def test_reduce_window_new_forms_plan(plugin):
    b = Builder()
    x = b.param((6, 8), "f32")
    i = b.param((6, 8), "s32")
    v, k = b.reduce_window_arg(x, i, b.constant(float("-inf"), "f32"), b.constant(0, "s32"), [2, 2],
                               strides=[2, 2], padding=[(1, -1), (0, 0)], base_dilations=[1, 2])
    y = b.reduce_window(x, b.constant(0.0, "f32"), "add", [3, 1], base_dilations=[2, 1], padding=[(-1, 0), (0, 0)])
    steps = _plan(plugin, b.build([v, k, y]))
    assert [s.get("library") for s in steps] == ["reduce_window", "reduce_window"]
