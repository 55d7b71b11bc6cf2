"""The widened frontend on the GPU: reduce_precision (fused elementwise),
reduce_window (library kernel), optimization_barrier and sdy.sharding_constraint
(identities) under an sdy.mesh prefix. Checked bit for bit against
oracle/frontend.py: reduce_precision is integer bit arithmetic, and
reduce_window folds each window sequentially in row-major order in the
accumulation type, as the oracle does (16-bit floats accumulate in f32 and
round once)."""
import numpy as np
import pytest

from oracle import frontend as F
from oracle import ops
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


def _special_f32():
    return np.array([0.0, -0.0, 1.0, -1.5, 65504.0, 65520.0, 1e6, -1e30, 2.0 ** -14, 2.0 ** -15, -2.0 ** -20,
                     1e-40, np.inf, -np.inf, np.nan, 3.0, 6.0, 1.4, 1.5], np.float32)


@pytest.mark.parametrize("e,m", [(8, 7), (5, 10), (8, 23), (4, 3), (5, 2), (8, 0), (1, 1), (7, 22)])
def test_reduce_precision_f32(client, e, m):
    rng = np.random.default_rng(e * 100 + m)
    x = (rng.standard_normal(5000) * np.exp(rng.uniform(-40, 40, 5000))).astype(np.float32)
    x = np.concatenate([x, _special_f32()])
    b = Builder()
    p = b.param(x.shape, "f32")
    (got,) = client.compile(b.build([b.reduce_precision(p, e, m)]))(x)
    want = F.reduce_precision(x, "f32", e, m)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dt,e,m", [("f16", 5, 10), ("f16", 4, 3), ("f16", 5, 2), ("bf16", 8, 7), ("bf16", 5, 2),
                                    ("bf16", 4, 3), ("f64", 11, 52), ("f64", 8, 23), ("f64", 5, 10)])
def test_reduce_precision_other_types(client, dt, e, m):
    rng = np.random.default_rng(7)
    v = (rng.standard_normal(3000) * np.exp(rng.uniform(-12, 12, 3000))).astype(np.float32)
    v = np.concatenate([v, np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 6.1e-5, 5.96e-8], np.float32)])
    if dt == "bf16":
        x = ops.f32_to_bf16_bits(v)
    elif dt == "f16":
        x = v.astype(np.float16)
    else:
        x = v.astype(np.float64) * 1e-200
    b = Builder()
    p = b.param(x.shape, dt)
    text = b.build([b.reduce_precision(p, e, m)])
    (got,) = client.compile(text)(x, dtypes=[dt] if dt == "bf16" else None)
    want = F.reduce_precision(x, dt, e, m)
    if dt == "bf16":
        np.testing.assert_array_equal(np.asarray(got, np.uint16), want)
    else:
        ut = {"f16": np.uint16, "f64": np.uint64}[dt]
        np.testing.assert_array_equal(np.asarray(got).view(ut), np.asarray(want).view(ut))


RW_CASES = [
    # dtype, shape, op, init, window, strides, dilations, padding
    ("f32", (3,), "add", 0.0, [2], [1], [1], [(1, 0)]),                        # the reference's case
    ("f32", (33, 47), "add", 0.0, [3, 5], [2, 3], [1, 2], [(1, 2), (0, 4)]),
    ("f32", (16, 20, 6), "maximum", -np.inf, [2, 3, 2], [2, 1, 2], [1, 1, 1], [(0, 1), (1, 1), (0, 0)]),
    ("f32", (50,), "minimum", np.inf, [4], [3], [2], [(2, 2)]),
    ("f32", (12, 9), "multiply", 1.0, [2, 2], [1, 1], [1, 1], [(0, 0), (0, 0)]),
    ("f32", (10, 10), "add", 1.25, [3, 3], [1, 1], [1, 1], [(1, 1), (1, 1)]),   # init not the identity
    ("bf16", (40, 30), "add", 0.0, [4, 3], [2, 2], [1, 1], [(1, 0), (0, 2)]),
    ("f16", (64,), "maximum", -np.inf, [7], [2], [1], [(3, 3)]),
    ("s32", (25, 25), "add", 0, [5, 5], [1, 1], [1, 1], [(2, 2), (2, 2)]),
    ("s32", (30,), "maximum", -2 ** 31, [4], [2], [1], [(0, 0)]),
    ("f64", (20, 8), "add", 0.0, [3, 2], [1, 2], [2, 1], [(0, 0), (1, 0)]),
]


@pytest.mark.parametrize("case", range(len(RW_CASES)))
def test_reduce_window_bit_exact(client, case):
    dt, shape, op, init, window, strides, dil, pad = RW_CASES[case]
    rng = np.random.default_rng(case)
    if dt == "s32":
        x = rng.integers(-2 ** 31, 2 ** 31, shape, dtype=np.int64).astype(np.int32) if op == "add" else \
            rng.integers(-1000, 1000, shape).astype(np.int32)
        xin, xval, acc = x, x, np.int32
    elif dt == "bf16":
        v = rng.standard_normal(shape).astype(np.float32)
        xin = ops.f32_to_bf16_bits(v)
        xval, acc = ops.bf16_bits_to_f32(xin), np.float32
    elif dt == "f16":
        xin = rng.standard_normal(shape).astype(np.float16)
        xin.reshape(-1)[::17] = np.nan
        xval, acc = xin.astype(np.float32), np.float32
    else:
        npt = np.float64 if dt == "f64" else np.float32
        xin = (rng.standard_normal(shape) * (0.5 if op == "multiply" else 1.0) + (1.0 if op == "multiply" else 0.0)).astype(npt)
        if op == "maximum":
            xin.reshape(-1)[::23] = np.nan
        xval, acc = xin, npt
    b = Builder()
    p = b.param(shape, dt)
    y = b.reduce_window(p, b.constant(init, dt), op, window, strides=strides, window_dilations=dil, padding=pad)
    (got,) = client.compile(b.build([y]))(xin, dtypes=[dt] if dt == "bf16" else None)
    want = F.reduce_window(xval, init, op, window, strides=strides, window_dilations=dil, padding=pad, acc_dtype=acc)
    if dt == "bf16":
        np.testing.assert_array_equal(np.asarray(got, np.uint16), ops.f32_to_bf16_bits(want))
    elif dt == "f16":
        np.testing.assert_array_equal(np.asarray(got).view(np.uint16), want.astype(np.float16).view(np.uint16))
    elif dt == "s32":
        np.testing.assert_array_equal(got, want)
    else:
        ut = np.uint64 if dt == "f64" else np.uint32
        np.testing.assert_array_equal(np.asarray(got).view(ut), want.view(ut))


RW_DILATED = [
    # dtype, shape, op, init, window, strides, window dilations, padding, base dilations
    ("f32", (9,), "add", 0.0, [2], [1], [1], [(0, 0)], [2]),
    ("f32", (7, 6), "add", 0.0, [3, 2], [1, 2], [1, 1], [(1, 2), (0, 1)], [2, 3]),
    ("f32", (12, 10), "maximum", -np.inf, [2, 3], [2, 1], [2, 1], [(-1, 1), (2, -2)], [1, 2]),
    ("bf16", (16, 9), "add", 0.0, [4, 2], [3, 1], [1, 2], [(0, 0), (1, 1)], [3, 2]),
    ("s32", (11,), "add", 0, [3], [2], [1], [(-2, -1)], [1]),
    ("f64", (5, 5), "minimum", np.inf, [2, 2], [1, 1], [1, 1], [(1, 1), (1, 1)], [2, 2]),
]


@pytest.mark.parametrize("case", range(len(RW_DILATED)))
def test_reduce_window_base_dilation_and_negative_padding(client, case):
    """Base dilation (holes contribute the init value) and negative padding
    (cropping), bit-exact against the oracle's StableHLO restatement."""
    dt, shape, op, init, window, strides, dil, pad, bd = RW_DILATED[case]
    rng = np.random.default_rng(100 + case)
    if dt == "s32":
        xin = rng.integers(-1000, 1000, shape).astype(np.int32)
        xval, acc = xin, np.int32
    elif dt == "bf16":
        xin = ops.f32_to_bf16_bits(rng.standard_normal(shape).astype(np.float32))
        xval, acc = ops.bf16_bits_to_f32(xin), np.float32
    else:
        npt = np.float64 if dt == "f64" else np.float32
        xin = rng.standard_normal(shape).astype(npt)
        xval, acc = xin, npt
    b = Builder()
    p = b.param(shape, dt)
    y = b.reduce_window(p, b.constant(init, dt), op, window, strides=strides, window_dilations=dil, padding=pad,
                        base_dilations=bd)
    (got,) = client.compile(b.build([y]))(xin, dtypes=[dt] if dt == "bf16" else None)
    want = F.reduce_window(xval, init, op, window, strides=strides, window_dilations=dil, padding=pad, acc_dtype=acc,
                           base_dilations=bd)
    if dt == "bf16":
        np.testing.assert_array_equal(np.asarray(got, np.uint16), ops.f32_to_bf16_bits(want))
    elif dt == "s32":
        np.testing.assert_array_equal(got, want)
    else:
        ut = np.uint64 if dt == "f64" else np.uint32
        np.testing.assert_array_equal(np.asarray(got).view(ut), want.view(ut))


RW_ARG = [
    # value dtype, index dtype, shape, kind, window, strides, window dilations, padding, base dilations
    ("f32", "s32", (3, 4), "max", [1, 2], [1, 1], [1, 1], [(0, 0), (0, 0)], [1, 1]),   # the op suite's case
    ("f32", "s32", (8, 40), "max", [2, 5], [2, 3], [1, 1], [(0, 1), (2, 2)], [1, 1]),
    ("f32", "s32", (8, 40), "min", [3, 4], [1, 2], [1, 2], [(1, 1), (0, 3)], [1, 1]),
    ("bf16", "s32", (6, 30), "max", [2, 3], [1, 2], [1, 1], [(0, 0), (1, -1)], [2, 1]),
    ("f16", "u32", (50,), "max", [6], [3], [1], [(2, 2)], [1]),
    ("f32", "s64", (10, 12), "max", [2, 2], [2, 2], [1, 1], [(0, 0), (0, 0)], [1, 2]),
    ("f64", "s32", (9, 9), "min", [3, 3], [2, 2], [1, 1], [(1, 1), (1, 1)], [1, 1]),
]


@pytest.mark.parametrize("case", range(len(RW_ARG)))
def test_reduce_window_argmax_pairs(client, case):
    """Two-operand (values, indices) windows with the argmax / argmin pair
    region (the reference's max-pool-with-indices form): ties (values drawn
    from a few integers), NaNs, padding and holes contributing (init value,
    init index); values and indices bit-exact against the oracle."""
    vt, it, shape, kind, window, strides, dil, pad, bd = RW_ARG[case]
    rng = np.random.default_rng(200 + case)
    vals = rng.integers(-3, 4, shape).astype(np.float32)
    if case == 0:
        vals = (np.arange(12, dtype=np.float32).reshape(3, 4) - np.float32(3.0)) / np.float32(7.0)
    else:
        vals.reshape(-1)[::13] = np.nan
    npi = {"s32": np.int32, "u32": np.uint32, "s64": np.int64}[it]
    idx = np.broadcast_to(np.arange(shape[-1]), shape).astype(npi) if case == 0 else \
        rng.permutation(int(np.prod(shape))).reshape(shape).astype(npi)
    if vt == "bf16":
        vin = ops.f32_to_bf16_bits(vals)
        vval = ops.bf16_bits_to_f32(vin)
    else:
        npv = {"f32": np.float32, "f16": np.float16, "f64": np.float64}[vt]
        vin = vals.astype(npv)
        vval = vin
    init_v = -np.inf if kind == "max" else np.inf
    b = Builder()
    pv, pi = b.param(shape, vt), b.param(shape, it)
    v, k = b.reduce_window_arg(pv, pi, b.constant(init_v, vt), b.constant(0, it), window, strides=strides,
                               window_dilations=dil, padding=pad, base_dilations=bd, kind=kind)
    got_v, got_i = client.compile(b.build([v, k]))(vin, idx, dtypes=[vt if vt == "bf16" else None, None])
    want_v, want_i = F.reduce_window_arg(vval, idx, init_v, 0, kind, window, strides=strides, window_dilations=dil,
                                         padding=pad, base_dilations=bd)
    np.testing.assert_array_equal(got_i, want_i)
    if vt == "bf16":
        np.testing.assert_array_equal(np.asarray(got_v, np.uint16), ops.f32_to_bf16_bits(want_v))
    else:
        ut = {"f32": np.uint32, "f16": np.uint16, "f64": np.uint64}[vt]
        np.testing.assert_array_equal(np.asarray(got_v).view(ut), np.asarray(want_v).view(ut))


def test_barrier_and_sharding_constraint_under_a_mesh(client):
    """jax.jit's Shardy prefix on one device: the mesh and shardings are
    ignored, the barrier and the constraint pass their operands through."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8, 16)).astype(np.float32)
    w = rng.standard_normal((8, 16)).astype(np.float32)
    b = Builder(mesh='["x"=1]')
    px, pw = b.param(x.shape, "f32"), b.param(w.shape, "f32")
    s, t = b.optimization_barrier([b.add(px, pw), b.multiply(px, pw)])
    r = b.sharding_constraint(b.subtract(s, t))
    got = client.compile(b.build([r, t]))(x, w)
    np.testing.assert_array_equal(got[0], (x + w) - x * w)
    np.testing.assert_array_equal(got[1], x * w)
