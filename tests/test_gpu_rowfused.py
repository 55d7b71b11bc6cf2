"""Row-fused kernels (planner fuse_row_chains + codegen row_fused): softmax,
RMSNorm and layer norm as one workgroup per row, against numpy, including
rows that are not a multiple of the 256-thread span and rows with -inf /
masked entries. f32 within 1e-5 relative (plus an absolute floor for
sums), bf16 outputs within 2e-2."""
import json

import numpy as np
import pytest

from oracle import ops
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


def _softmax(b, x):
    mx = b.max(x, [x.rank - 1])
    kept = list(range(x.rank - 1))
    e = b.exp(b.subtract(x, b.broadcast_in_dim(mx, x.shape, kept)))
    s = b.reduce(e, b.constant(0.0, "f32"), [x.rank - 1], "add")
    return b.divide(e, b.broadcast_in_dim(s, x.shape, kept))


def _np_softmax(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


# (1100, 40) and (2, 1024, 1000) take the wave-per-row form (many short rows,
# a row count that is not a multiple of the 4 rows per workgroup).
@pytest.mark.parametrize("shape", [(3, 40), (5, 1000), (2, 3, 2048), (1, 16384), (1100, 40), (2, 1025, 1000)])
def test_softmax_row_kernel(client, shape):
    rng = np.random.default_rng(sum(shape))
    x = (3 * rng.standard_normal(shape)).astype(np.float32)
    x[..., 1] = -np.inf  # masked entries
    b = Builder()
    xp = b.param(shape, "f32")
    exe = client.compile(b.build([_softmax(b, xp)]))
    kinds = [s["kind"] for s in json.loads(exe.optimized_program())["steps"]]
    steps = json.loads(exe.optimized_program())["steps"]
    assert kinds == ["rowfused"]
    assert steps[0]["wave_per_row"] == (steps[0]["rows"] >= 1024)
    (out,) = exe(x)
    np.testing.assert_allclose(out, _np_softmax(x), rtol=1e-5, atol=1e-7)


def test_rmsnorm_row_kernel_bf16(client):
    rows, d, eps = 7, 2048, 1e-5
    rng = np.random.default_rng(1)
    xb = ops.f32_to_bf16_bits(rng.standard_normal((rows, d)).astype(np.float32))
    wb = ops.f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(d)).astype(np.float32))
    b = Builder()
    x = b.param((rows, d), "bf16")
    w = b.param((d,), "bf16")
    xf = b.convert(x, "f32")
    ss = b.reduce(b.multiply(xf, xf), b.constant(0.0, "f32"), [1], "add")
    r = b.rsqrt(b.add(b.divide(ss, b.scalar_like(float(d), ss)), b.scalar_like(eps, ss)))
    y = b.multiply(b.convert(b.multiply(xf, b.broadcast_in_dim(r, xf.shape, [0])), "bf16"),
                   b.broadcast_in_dim(w, (rows, d), [1]))
    exe = client.compile(b.build([y]))
    assert [s["kind"] for s in json.loads(exe.optimized_program())["steps"]] == ["rowfused"]
    (out,) = exe(xb, wb, dtypes=["bf16", "bf16"])
    xd = ops.bf16_bits_to_f32(xb).astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + eps) * ops.bf16_bits_to_f32(wb)
    got = ops.bf16_bits_to_f32(out).astype(np.float64)
    assert np.abs(got - want).max() <= 2e-2 * np.abs(want).max()


def test_layernorm_mean_var_row_kernel(client):
    rows, d = 9, 3000
    rng = np.random.default_rng(2)
    x = (5 + rng.standard_normal((rows, d))).astype(np.float32)
    b = Builder()
    xp = b.param((rows, d), "f32")
    mean = b.divide(b.reduce(xp, b.constant(0.0, "f32"), [1], "add"),
                    b.broadcast_in_dim(b.constant(float(d), "f32"), (rows,), []))
    xc = b.subtract(xp, b.broadcast_in_dim(mean, (rows, d), [0]))
    var = b.divide(b.reduce(b.multiply(xc, xc), b.constant(0.0, "f32"), [1], "add"),
                   b.broadcast_in_dim(b.constant(float(d), "f32"), (rows,), []))
    y = b.multiply(xc, b.broadcast_in_dim(b.rsqrt(b.add(var, b.broadcast_in_dim(b.constant(1e-6, "f32"), (rows,), []))),
                                          (rows, d), [0]))
    exe = client.compile(b.build([y, mean]))
    steps = json.loads(exe.optimized_program())["steps"]
    assert [s["kind"] for s in steps] == ["rowfused"] and steps[0]["phases"] == 3
    out, m = exe(x)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    want = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(m, mu[:, 0], rtol=1e-6)
