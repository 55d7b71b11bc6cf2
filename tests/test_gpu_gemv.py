"""Generated decode GEMVs (kGemv steps): split-K products folded in-launch by
the last workgroup of each column segment, with an RMSNorm prologue and
elementwise epilogues (SwiGLU; RoPE with the KV-row writes is covered by the
llama tests). Each result must equal float64 within the bf16/f16 bar, be
the same bits on every run (fixed fold order), and be the same bits when
the partials are published by device-scope fences instead of the XCD-local
path (PJRTX_XCD_LOCAL=0, in a subprocess: the device probe runs once)."""
import json

import numpy as np
import pytest

from oracle import llama as OL
from oracle import ops
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


def _bits(rng, shape, dt, scale=1.0):
    v = (scale * rng.standard_normal(shape)).astype(np.float32)
    return ops.f32_to_bf16_bits(v) if dt == "bf16" else v.astype(np.float16)


def _f64(a, dt):
    return (ops.bf16_bits_to_f32(a) if dt == "bf16" else np.asarray(a, np.float32)).astype(np.float64)


def _group(M, K, Ns, dt):
    b = Builder()
    x = b.param((M, K), dt)
    ws = [b.param((K, n), dt) for n in Ns]
    return b.build([b.dot_general(x, w, contract=((1,), (0,))) for w in ws])


def _steps(exe):
    return json.loads(exe.optimized_program())["steps"]


@pytest.mark.parametrize("M,K,Ns,dt", [
    (1, 2048, (2048, 2048, 2048), "bf16"),   # q/k/v
    (1, 2048, (2048, 512, 512), "bf16"),     # grouped-query k/v widths
    (1, 2048, (5632, 5632), "bf16"),         # gate / up
    (1, 5632, (2048,), "bf16"),              # down projection (K split 22 ways)
    (1, 2048, (32000,), "bf16"),             # lm_head
    (2, 1024, (1024, 2048, 64, 4096), "f16"),
    (4, 4096, (1000,), "bf16"),              # ragged last tile
    (3, 8192, (520, 8), "f16"),              # X chunks staged per split; an 8-column member
])
def test_gemv_matches_float64_and_is_deterministic(client, M, K, Ns, dt):
    rng = np.random.default_rng(K + sum(Ns) + M)
    x = _bits(rng, (M, K), dt)
    ws = [_bits(rng, (K, n), dt, 1 / np.sqrt(K)) for n in Ns]
    exe = client.compile(_group(M, K, Ns, dt))
    steps = _steps(exe)
    assert [s["kind"] for s in steps] == ["gemv"] and steps[0]["members"] == len(Ns)
    outs = exe(x, *ws, dtypes=[dt] * (1 + len(Ns)))
    for got, w in zip(outs, ws):
        want = _f64(x, dt) @ _f64(w, dt)
        assert np.abs(_f64(got, dt) - want).max() <= 2e-2 * np.abs(want).max()
    again = exe(x, *ws, dtypes=[dt] * (1 + len(Ns)))
    for a, b in zip(outs, again):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("M,K,N,dt", [(1, 2048, 2048, "bf16"), (2, 5632, 2048, "f16"), (1, 2048, 32000, "bf16")])
def test_gemv_residual_add(client, M, K, N, dt):
    """x + dot(h, w): the fold rounds the product, adds x and rounds again,
    as the separate add would."""
    rng = np.random.default_rng(K + N)
    b = Builder()
    h, w, x = b.param((M, K), dt), b.param((K, N), dt), b.param((M, N), dt)
    text = b.build([b.add(x, b.dot_general(h, w, contract=((1,), (0,))))])
    args = [_bits(rng, (M, K), dt), _bits(rng, (K, N), dt, 1 / np.sqrt(K)), _bits(rng, (M, N), dt)]
    exe = client.compile(text)
    steps = _steps(exe)
    assert [s["kind"] for s in steps] == ["gemv"] and "residual_add" in steps[0]
    (got,) = exe(*args, dtypes=[dt] * 3)
    ref = _f64(args[2], dt) + _f64(args[0], dt) @ _f64(args[1], dt)
    assert np.abs(_f64(got, dt) - ref).max() <= 2e-2 * np.abs(ref).max()


def _rmsnorm(b, x, g, d, eps=1e-5):
    xf = b.convert(x, "f32")
    ss = b.reduce(b.multiply(xf, xf), b.constant(0.0, "f32"), [1], "add")
    ms = b.divide(ss, b.scalar_like(float(d), ss))
    r = b.rsqrt(b.add(ms, b.scalar_like(eps, ms)))
    y = b.convert(b.multiply(xf, b.broadcast_in_dim(r, xf.shape, [0])), "bf16")
    return b.multiply(y, b.broadcast_in_dim(g, y.shape, [1]))


def _norm_swiglu_program(d, f):
    b = Builder()
    x, g, w1, w3 = b.param((1, d), "bf16"), b.param((d,), "bf16"), b.param((d, f), "bf16"), b.param((d, f), "bf16")
    h = _rmsnorm(b, x, g, d)
    mm = lambda a, w: b.dot_general(a, w, contract=((1,), (0,)))  # noqa: E731
    gate = b.convert(mm(h, w1), "f32")
    act = b.multiply(b.convert(b.multiply(gate, b.logistic(gate)), "bf16"), mm(h, w3))
    return b.build([act])


@pytest.mark.parametrize("d,f", [(2048, 5632), (128, 320), (512, 1024)])
def test_rmsnorm_prologue_swiglu_epilogue(client, monkeypatch, d, f):
    """RMSNorm -> gate/up -> SwiGLU as one launch: equals the unfused plan
    (row-fused norm, grouped GEMV, elementwise loop) and the numpy oracle
    within the bf16 bar."""
    rng = np.random.default_rng(d + f)
    x = _bits(rng, (1, d), "bf16")
    g = _bits(rng, (d,), "bf16")
    w1 = _bits(rng, (d, f), "bf16", 0.02)
    w3 = _bits(rng, (d, f), "bf16", 0.02)
    text = _norm_swiglu_program(d, f)
    exe = client.compile(text)
    steps = _steps(exe)
    assert [s["kind"] for s in steps] == ["gemv"]
    assert steps[0]["prologue"] == "rowfused" and "logistic" in steps[0]["epilogue_loop"]
    (got,) = exe(x, g, w1, w3, dtypes=["bf16"] * 4)
    monkeypatch.setenv("PJRTX_GEMV_FUSION", "0")
    plain = client.compile(text)
    assert len(_steps(plain)) == 3
    (want,) = plain(x, g, w1, w3, dtypes=["bf16"] * 4)
    gf, wf = _f64(got, "bf16"), _f64(want, "bf16")
    assert np.abs(gf - wf).max() <= 2e-2 * np.abs(wf).max()
    # numpy oracle: the same roundings, f32 products
    h = OL.rmsnorm(OL.bf16_bits_to_f32(x), OL.bf16_bits_to_f32(g), 1e-5)
    gate = OL.mm(h, OL.bf16_bits_to_f32(w1))
    up = OL.mm(h, OL.bf16_bits_to_f32(w3))
    act = OL.bf16_round(OL.bf16_round(gate / (np.float32(1) + np.exp(-gate))) * up).astype(np.float64)
    assert np.abs(gf - act).max() <= 2e-2 * np.abs(act).max()


def test_fence_path_gives_the_same_bits(client, run_fresh):
    """With the XCD placement unavailable (PJRTX_XCD_LOCAL=0) the partials
    are published with agent-scope fences; the fold order is the same, so
    are the bits."""
    rng = np.random.default_rng(7)
    d, f = 2048, 5632
    args = [_bits(rng, (1, d), "bf16"), _bits(rng, (d,), "bf16"), _bits(rng, (d, f), "bf16", 0.02),
            _bits(rng, (d, f), "bf16", 0.02)]
    text = _norm_swiglu_program(d, f)
    (got,) = client.compile(text)(*args, dtypes=["bf16"] * 4)
    (other,) = run_fresh(text, args, ["bf16"] * 4, {"PJRTX_XCD_LOCAL": "0"})
    np.testing.assert_array_equal(got, other)
