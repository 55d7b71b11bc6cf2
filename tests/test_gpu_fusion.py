"""GPU parity of the fused elementwise / reduction path through the PJRT C API
(Compile -> BufferFromHostBuffer -> Execute -> ToHostBuffer), against the
numpy oracle. Each case runs twice, as the reference's CPU-vs-plugin suite
does (reference: src/plugin/jax/jax_op_suite.py:98-109).

Tolerances (stated by the task): integer / index / argmax values bit-exact;
f32 1e-5 relative; f16 / bf16 2e-2 relative (plus one f16 ulp near zero).
"""
import numpy as np
import pytest

from oracle import ops
from pjrtx_amd import programs
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


def run_twice(exe, *args, dtypes=None):
    first = exe(*args, dtypes=dtypes)
    second = exe(*args, dtypes=dtypes)
    for a, b in zip(first, second):
        np.testing.assert_array_equal(a, b)  # deterministic across runs
    return first


def check_f16(got, want):
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    tol = np.maximum(2e-2 * np.abs(want), 2 * np.spacing(np.abs(want).astype(np.float16)).astype(np.float64))
    assert np.all(np.abs(got - want) <= tol), (got, want)


@pytest.mark.parametrize("rows,cols", [(8, 256), (64, 1000), (4096, 4096)])
def test_c1_rowsum(client, rows, cols):
    x, y = ops.c1_inputs(rows, cols, seed=rows + cols)
    exe = client.compile(programs.c1_elementwise_rowsum(rows, cols))
    (out,) = run_twice(exe, x, y)
    assert out.dtype == np.float32 and out.shape == (rows,)
    np.testing.assert_allclose(out, ops.c1_rowsum(x, y), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rows,vocab", [(2, 100), (4, 4096), (3, 131072 + 7), (64, 128256)])
def test_c2_argmax_and_f16_reductions(client, rows, vocab):
    logits = ops.c2_inputs(rows, vocab, seed=vocab)
    exe = client.compile(programs.c2_argmax_f16_reductions(rows, vocab))
    vals, idx, s, mx, mn = run_twice(exe, logits, dtypes=["bf16"])
    rv, ri, rs, rmx, rmn = ops.c2_reference(logits)
    np.testing.assert_array_equal(idx, ri)
    np.testing.assert_array_equal(vals, rv)
    np.testing.assert_array_equal(mx, rmx)
    np.testing.assert_array_equal(mn, rmn)
    check_f16(s, rs)


def test_argmax_ties_and_nans(client):
    rows, vocab = 6, 50000
    rng = np.random.default_rng(11)
    v = rng.integers(-4, 5, size=(rows, vocab)).astype(np.float32)  # heavy ties
    v[1, 30000] = np.nan
    v[1, 45000] = np.nan
    v[2, :] = -np.inf
    v[3, 49999] = 100.0
    v[4, 0] = 100.0
    v[4, 49999] = 100.0
    bits = ops.f32_to_bf16_bits(v)
    exe = client.compile(programs.c2_argmax_only(rows, vocab, "bf16"))
    vals, idx = run_twice(exe, bits, dtypes=["bf16"])
    rv, ri = ops.argmax_rows(ops.bf16_bits_to_f32(bits))
    np.testing.assert_array_equal(idx, ri)
    got = ops.bf16_bits_to_f32(vals)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(rv))
    np.testing.assert_array_equal(got[~np.isnan(got)], rv[~np.isnan(rv)])


def test_argmax_f32_reference_kat(client):
    # reference: api_test.cc:1016-1055 / jax_op_suite.py reduce_argmax_axis1
    x = np.array([[1.0, 7.0, 7.0, 3.0], [-2.0, 5.0, 4.0, 5.0]], dtype=np.float32)
    exe = client.compile(programs.c2_argmax_only(2, 4, "f32"))
    vals, idx = run_twice(exe, x)
    np.testing.assert_array_equal(vals, [7.0, 5.0])
    np.testing.assert_array_equal(idx, [1, 1])


def test_f16_reduce_reference_kat(client):
    # reference: api_test.cc:930-1014
    b = Builder()
    x = b.param((2, 2), "f16")
    p = b.build([b.sum(x, [1]), b.max(x, [1]), b.min(x, [1])])
    s, mx, mn = run_twice(client.compile(p), np.array([[1, 2], [3, 4]], dtype=np.float16))
    np.testing.assert_array_equal(s, [3, 7])
    np.testing.assert_array_equal(mx, [2, 4])
    np.testing.assert_array_equal(mn, [1, 3])


def test_elementwise_chain_reference_suite(client):
    # jax_op_suite.py "elementwise_float_chain":
    # tanh((x + y) * rsqrt(max(y, floor))) - exp(x * tiny)
    a = (np.arange(12, dtype=np.float32).reshape(3, 4) - np.float32(3.0)) / np.float32(7.0)
    bb = np.linspace(0.5, 1.7, 12, dtype=np.float32).reshape(3, 4)
    fl = np.full((3, 4), 0.25, np.float32)
    tiny = np.full((3, 4), 0.01, np.float32)
    b = Builder()
    x, y, f, t = (b.param((3, 4), "f32") for _ in range(4))
    out = b.subtract(b.tanh(b.multiply(b.add(x, y), b.rsqrt(b.maximum(y, f)))), b.exp(b.multiply(x, t)))
    (got,) = run_twice(client.compile(b.build([out])), a, bb, fl, tiny)
    want = np.tanh((a.astype(np.float64) + bb) / np.sqrt(np.maximum(bb, fl))) - np.exp(a.astype(np.float64) * tiny)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_views_transpose_broadcast_reshape(client):
    # jax_op_suite.py "reshape_transpose_broadcast"
    a = (np.arange(12, dtype=np.float32).reshape(3, 4) - 3) / 7
    b = Builder()
    x = b.param((3, 4), "f32")
    r = b.reshape(x, (2, 6))
    bc = b.broadcast_in_dim(r, (2, 2, 6), [1, 2])
    out = b.transpose(bc, [1, 2, 0])
    (got,) = run_twice(client.compile(b.build([out])), a)
    want = np.broadcast_to(a.reshape(2, 6), (2, 2, 6)).transpose(1, 2, 0)
    np.testing.assert_array_equal(got, want)


def test_reduce_middle_axis_and_all(client):
    cube = (np.arange(24, dtype=np.float32).reshape(2, 3, 4) - 8) / 5
    b = Builder()
    x = b.param((2, 3, 4), "f32")
    outs = [b.max(x, [1]), b.min(x, [1]), b.sum(x, [0, 1, 2]), b.sum(x, [0, 2])]
    got = run_twice(client.compile(b.build(outs)), cube)
    np.testing.assert_array_equal(got[0], cube.max(axis=1))
    np.testing.assert_array_equal(got[1], cube.min(axis=1))
    np.testing.assert_allclose(got[2], cube.astype(np.float64).sum(), rtol=1e-6)
    np.testing.assert_allclose(got[3], cube.astype(np.float64).sum(axis=(0, 2)), rtol=1e-6)


def test_integer_and_predicate_ops(client):
    # jax_op_suite.py "bitwise_int", "zml_shift_right_arithmetic", "zml_predicate_logic"
    a = np.arange(8, dtype=np.int32)
    bb = np.arange(10, 18, dtype=np.int32)
    sh = np.full((8,), 1, np.int32)
    neg = np.array([-8, -4, -1, 0, 1, 4, 8, 16], dtype=np.int32)
    b = Builder()
    x, y, s, n = (b.param((8,), "s32") for _ in range(4))
    o1 = b.xor(b.and_(x, y), b.shift_left(x, s))
    o2 = b.shift_right_arithmetic(n, s)
    o3 = b.shift_right_logical(n, s)
    got = run_twice(client.compile(b.build([o1, o2, o3])), a, bb, sh, neg)
    np.testing.assert_array_equal(got[0], (a & bb) ^ (a << sh))
    np.testing.assert_array_equal(got[1], neg >> sh)
    np.testing.assert_array_equal(got[2], (neg.view(np.uint32) >> 1).view(np.int32))


def test_outputs_that_alias_inputs_are_copies(client):
    b = Builder()
    x = b.param((4,), "f32")
    text = b.build([x, x])
    a = np.arange(4, dtype=np.float32)
    got = client.compile(text)(a)
    np.testing.assert_array_equal(got[0], a)
    np.testing.assert_array_equal(got[1], a)


def test_execute_rejects_wrong_argument(client):
    from pjrtx_amd.pjrt import PjrtError
    exe = client.compile(programs.c1_elementwise_rowsum(8, 256))
    with pytest.raises(PjrtError) as e:
        exe(np.zeros((8, 256), np.float32))
    assert e.value.code == 3
    with pytest.raises(PjrtError):
        exe(np.zeros((8, 255), np.float32), np.zeros((8, 255), np.float32))


def test_execute_loops_through_plugin_and_pjrt_c_api(client):
    """The plugin's own execute loop and the loop through the PJRT C API table
    (one PJRT_LoadedExecutable_Execute per step, its event and outputs
    destroyed) both run, leave the arguments usable and time a positive
    interval; an execute afterwards still gives the oracle's rows."""
    x, y = ops.c1_inputs(64, 1000, seed=5)
    exe = client.compile(programs.c1_elementwise_rowsum(64, 1000))
    bufs = [client.buffer(x), client.buffer(y)]
    assert exe.run_loop(bufs, 4) > 0
    assert exe.run_loop_pjrt(bufs, 4) > 0
    (out,) = exe.execute_buffers(bufs)
    np.testing.assert_allclose(out.to_numpy(), ops.c1_rowsum(x, y), rtol=1e-5, atol=1e-6)
