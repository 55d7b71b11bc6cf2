"""stablehlo.while on the GPU: loops whose count constants fix (run back to
back), loops whose predicate is read every iteration (an argument bound, a
data-dependent condition with a reduction), loop-carried buffers updated in
place, nested loops and a GEMV inside the body, each against the same loop
run in numpy. The caller's arguments must come back unchanged."""
import json

import numpy as np
import pytest

from oracle import ops
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


def _doubling(bound_param: bool, bound: int = 5):
    b = Builder()
    x = b.param((4,), "f32")
    n = b.param((), "s32") if bound_param else b.constant(bound, "s32")
    two = b.constant(2.0, "f32")
    i, v = b.while_loop([b.constant(0, "s32"), x], lambda i, v: b.compare("LT", i, n),
                        lambda i, v: [b.add(i, b.constant(1, "s32")), b.multiply(v, b.broadcast_in_dim(two, (4,), []))])
    return b.build([v, i])


def test_fixed_count_loop(client):
    text = _doubling(False, 5)
    exe = client.compile(text)
    assert json.loads(exe.optimized_program())["steps"][0]["while_trips"] == 5
    x = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    v, i = exe(x)
    np.testing.assert_array_equal(v, x * 32)
    assert int(i) == 5


@pytest.mark.parametrize("n", [0, 1, 7])
def test_argument_bound_loop(client, n):
    exe = client.compile(_doubling(True))
    x = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    v, i = exe(x, np.array(n, np.int32))
    np.testing.assert_array_equal(v, x * np.float32(2.0 ** n))
    assert int(i) == n


def test_data_dependent_condition_with_reduction(client):
    b = Builder()
    x = b.param((64,), "f32")
    limit = b.constant(1000.0, "f32")
    (v,) = b.while_loop([x], lambda v: b.compare("LT", b.sum(v, [0]), limit),
                        lambda v: b.add(b.multiply(v, b.scalar_like(2.0, v)), b.scalar_like(1.0, v)))
    x0 = np.linspace(0.0, 1.0, 64, dtype=np.float32)
    (got,) = client.compile(b.build([v]))(x0)
    want = x0.copy()
    while want.sum(dtype=np.float32) < 1000.0:
        want = want * np.float32(2.0) + np.float32(1.0)
    np.testing.assert_allclose(got, want, rtol=1e-6)


def test_rows_written_in_place_and_argument_untouched(client):
    b = Builder()
    buf = b.param((8, 4), "f32")
    row = b.param((1, 4), "f32")
    n8 = b.constant(8, "s32")

    def body(i, bb):
        f = b.broadcast_in_dim(b.convert(i, "f32"), (1, 4), [])
        return [b.add(i, b.constant(1, "s32")),
                b.dynamic_update_slice(bb, b.multiply(row, f), [i, b.constant(0, "s32")])]

    i, out = b.while_loop([b.constant(0, "s32"), buf], lambda i, bb: b.compare("LT", i, n8), body)
    exe = client.compile(b.build([out]))
    base = np.full((8, 4), 7.0, np.float32)
    r = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    bufd = client.buffer(base)
    rowd = client.buffer(r)
    (o1,) = exe.execute_buffers([bufd, rowd])
    (o2,) = exe.execute_buffers([bufd, rowd])
    want = np.arange(8, dtype=np.float32)[:, None] * r
    np.testing.assert_array_equal(o1.to_numpy(), want)
    np.testing.assert_array_equal(o2.to_numpy(), want)
    np.testing.assert_array_equal(bufd.to_numpy(), base)   # the argument is not written


def test_nested_loops(client):
    b = Builder()
    acc0 = b.param((), "f32")
    n3 = b.constant(3, "s32")
    one_f = b.constant(1.0, "f32")

    def outer_body(i, acc):
        lim = b.add(i, b.constant(1, "s32"))
        j, a = b.while_loop([b.constant(0, "s32"), acc], lambda j, a: b.compare("LT", j, lim),
                            lambda j, a: [b.add(j, b.constant(1, "s32")), b.add(a, one_f)])
        return [b.add(i, b.constant(1, "s32")), a]

    i, acc = b.while_loop([b.constant(0, "s32"), acc0], lambda i, a: b.compare("LT", i, n3), outer_body)
    (got,) = client.compile(b.build([acc]))(np.array(0.5, np.float32))
    assert float(got) == 6.5


def test_gemv_in_the_body(client):
    rng = np.random.default_rng(3)
    K = 256
    b = Builder()
    h0 = b.param((1, K), "bf16")
    w = b.param((K, K), "bf16")
    n4 = b.constant(4, "s32")
    i, h = b.while_loop([b.constant(0, "s32"), h0], lambda i, h: b.compare("LT", i, n4),
                        lambda i, h: [b.add(i, b.constant(1, "s32")),
                                      b.tanh(b.dot_general(h, w, contract=((1,), (0,))))])
    hb = ops.f32_to_bf16_bits(rng.standard_normal((1, K)).astype(np.float32))
    wb = ops.f32_to_bf16_bits((rng.standard_normal((K, K)) / np.sqrt(K)).astype(np.float32))
    (got,) = client.compile(b.build([h]))(hb, wb, dtypes=["bf16", "bf16"])
    want = ops.bf16_bits_to_f32(hb).astype(np.float64)
    wf = ops.bf16_bits_to_f32(wb).astype(np.float64)
    for _ in range(4):
        want = np.tanh(ops.bf16_bits_to_f32(ops.f32_to_bf16_bits((want @ wf).astype(np.float32))).astype(np.float64))
        want = ops.bf16_bits_to_f32(ops.f32_to_bf16_bits(want.astype(np.float32))).astype(np.float64)
    got64 = ops.bf16_bits_to_f32(got).astype(np.float64)
    assert np.abs(got64 - want).max() <= 2e-2 * np.abs(want).max()


def test_zero_iterations_return_the_initial_state(client):
    exe = client.compile(_doubling(True))
    x = np.array([1.5, 2.5, 3.5, 4.5], np.float32)
    v, i = exe(x, np.array(-4, np.int32))
    np.testing.assert_array_equal(v, x)
    assert int(i) == 0
