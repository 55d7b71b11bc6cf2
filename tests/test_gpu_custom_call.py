"""Registered custom-call targets on the GPU: each runs as the elementwise op
it names, bit for bit the same as the program written with that stablehlo op
(whose parity the elementwise suite pins), and exact against numpy where the
op is exact (reference: src/backend/mlx_metal/custom_call.zig:155-238,
execution_integration_custom_call_tests.zig)."""
import numpy as np
import pytest

from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu

SHAPE = (64, 96)


def _inputs(dtype, n, seed):
    rng = np.random.default_rng(seed)
    if dtype == "f32":
        xs = [rng.standard_normal(SHAPE).astype(np.float32) * 3 for _ in range(n)]
        xs[0][0, :4] = [np.inf, -np.inf, np.nan, 0.0]
        return xs
    if dtype == "s32":
        return [rng.integers(-2**31, 2**31, SHAPE, dtype=np.int64).astype(np.int32) for _ in range(n)]
    return [rng.integers(0, 2, SHAPE).astype(np.bool_) for _ in range(n)]


def _run(client, text, xs, dtype):
    return client.compile(text)(*xs, dtypes=[None] * len(xs))[0]


def _call_prog(target, n, dtype, out_dtype=None, then_negate=False):
    b = Builder()
    ps = [b.param(SHAPE, dtype) for _ in range(n)]
    y = b.custom_call(target, ps, SHAPE, out_dtype or dtype)
    if then_negate:  # the lowered op fuses with its consumer
        y = b.not_(y) if dtype == "pred" else b.negate(y)
    return b.build([y])


def _op_prog(method, n, dtype, then_negate=False):
    b = Builder()
    ps = [b.param(SHAPE, dtype) for _ in range(n)]
    y = getattr(b, method)(*ps)
    if then_negate:
        y = b.not_(y) if dtype == "pred" else b.negate(y)
    return b.build([y])


CASES = [
    # (kind, op name, Builder method, dtype, numpy reference or None)
    ("binary", "add", "add", "f32", lambda a, b: a + b),
    ("binary", "multiply", "multiply", "f32", lambda a, b: a * b),
    ("binary", "maximum", "maximum", "f32", None),
    ("binary", "atan2", "atan2", "f32", None),
    ("binary", "subtract", "subtract", "s32", lambda a, b: a - b),
    ("binary", "xor", "xor", "s32", lambda a, b: a ^ b),
    ("binary", "and", "and_", "pred", lambda a, b: a & b),
    ("unary", "exp", "exp", "f32", None),
    ("unary", "sqrt", "sqrt", "f32", None),
    ("unary", "floor", "floor", "f32", np.floor),
    ("unary", "popcnt", "popcnt", "s32", lambda a: np.array([bin(int(v) & 0xffffffff).count("1") for v in a.ravel()],
                                                             np.int32).reshape(a.shape)),
    ("unary", "not", "not_", "pred", lambda a: ~a),
    ("unary", "count_leading_zeros", "clz", "s32",
     lambda a: np.array([32 - (int(v) & 0xffffffff).bit_length() for v in a.ravel()], np.int32).reshape(a.shape)),
]


@pytest.mark.parametrize("kind,op,method,dtype,ref", CASES, ids=[f"{c[1]}_{c[3]}" for c in CASES])
def test_registered_target_runs_as_its_op(client, plugin, kind, op, method, dtype, ref):
    t = f"pjrtx.test.gpu.{op}.{dtype}"
    n = 2 if kind == "binary" else 1
    (plugin.register_custom_call_binary if kind == "binary" else plugin.register_custom_call_unary)(t, op)
    try:
        xs = _inputs(dtype, n, seed=len(op))
        for fused in (False, True):
            got = _run(client, _call_prog(t, n, dtype, then_negate=fused), xs, dtype)
            want = _run(client, _op_prog(method, n, dtype, then_negate=fused), xs, dtype)
            np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))
        if ref is not None:
            with np.errstate(all="ignore"):
                np.testing.assert_array_equal(_run(client, _call_prog(t, n, dtype), xs, dtype), ref(*xs))
    finally:
        plugin.unregister_custom_call(t)


def test_is_finite_target(client, plugin):
    t = "pjrtx.test.gpu.is_finite"
    plugin.register_custom_call_unary(t, "is_finite")
    try:
        (x,) = _inputs("f32", 1, seed=3)
        got = _run(client, _call_prog(t, 1, "f32", out_dtype="pred"), [x], "f32")
        np.testing.assert_array_equal(got, np.isfinite(x))
    finally:
        plugin.unregister_custom_call(t)


def test_extension_markers_and_identity_targets(client, plugin):
    """Targets registered through the PJRT GPU custom-call extension (sqrt,
    add and identity markers) and the built-in identity and f32 add targets."""
    ts = {"pjrtx.test.gpu.ext_sqrt": "PjRTx_CustomCall_UnarySqrt", "pjrtx.test.gpu.ext_add": "PjRTx_CustomCall_BinaryAdd",
          "pjrtx.test.gpu.ext_id": "PjRTx_CustomCall_Identity"}
    for t, m in ts.items():
        plugin.register_custom_call_handler(t, plugin.marker(m))
    try:
        a, b = _inputs("f32", 2, seed=9)
        np.testing.assert_array_equal(_run(client, _call_prog("pjrtx.test.gpu.ext_add", 2, "f32"), [a, b], "f32"), a + b)
        got = _run(client, _call_prog("pjrtx.test.gpu.ext_sqrt", 1, "f32"), [np.abs(a)], "f32")
        want = _run(client, _op_prog("sqrt", 1, "f32"), [np.abs(a)], "f32")
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(_run(client, _call_prog("pjrtx.test.gpu.ext_id", 1, "f32"), [a], "f32"), a)
        np.testing.assert_array_equal(_run(client, _call_prog("annotate_device_placement", 1, "f32"), [a], "f32"), a)
        np.testing.assert_array_equal(
            _run(client, _call_prog("pjrtx.mlx_metal.custom_binary_add_f32", 2, "f32"), [a, b], "f32"), a + b)
    finally:
        for t in ts:
            plugin.unregister_custom_call(t)
