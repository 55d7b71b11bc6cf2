"""Dot groups (planner: decode-shaped dots sharing one LHS, the reference's
dot group of executable_metal_graph_lowering_fusion.zig:394-424) on the
library path (PJRTX_GEMV_FUSION=0; the generated GEMVs are tested in
test_gpu_gemv.py) run as one gemv_wide launch. Each member must equal float64 within the bf16/f16 bar and
be bit-identical to the same dot planned alone (same kernel, same summation
order)."""
import json

import numpy as np
import pytest

from oracle import ops
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


def _program(M, K, Ns, dt):
    b = Builder()
    x = b.param((M, K), dt)
    ws = [b.param((K, n), dt) for n in Ns]
    return b.build([b.dot_general(x, w, contract=((1,), (0,))) for w in ws])


def _bits(rng, shape, dt, scale=1.0):
    v = (scale * rng.standard_normal(shape)).astype(np.float32)
    return ops.f32_to_bf16_bits(v) if dt == "bf16" else v.astype(np.float16)


def _f64(a, dt):
    return (ops.bf16_bits_to_f32(a) if dt == "bf16" else np.asarray(a, np.float32)).astype(np.float64)


@pytest.mark.parametrize("M,K,Ns,dt", [
    (1, 2048, (2048, 512, 512), "bf16"),     # q/k/v with grouped-query k/v widths
    (1, 2048, (5632, 5632), "bf16"),         # gate / up
    (2, 1024, (1024, 2048, 64, 4096), "f16"),
    (4, 4096, (2048, 2048), "bf16"),
    (4, 8192, (2048, 2048), "bf16"),         # M*K past the LDS stage: members run one by one
])
def test_dot_group_matches_oracle_and_single_dots(client, monkeypatch, M, K, Ns, dt):
    monkeypatch.setenv("PJRTX_GEMV_FUSION", "0")
    rng = np.random.default_rng(K + sum(Ns) + M)
    x = _bits(rng, (M, K), dt)
    ws = [_bits(rng, (K, n), dt, 1 / np.sqrt(K)) for n in Ns]
    text = _program(M, K, Ns, dt)
    exe = client.compile(text)
    steps = json.loads(exe.optimized_program())["steps"]
    assert [s.get("library") for s in steps] == ["dot_group"]
    assert steps[0]["group_size"] == len(Ns)
    auto = exe(x, *ws, dtypes=[dt] * (1 + len(Ns)))   # the column width the launcher picks
    for got, w in zip(auto, ws):
        want = _f64(x, dt) @ _f64(w, dt)
        assert np.abs(_f64(got, dt) - want).max() <= 2e-2 * np.abs(want).max()
    # At one forced width the group and each dot alone share the summation order.
    monkeypatch.setenv("PJRTX_GEMV_COLS", "64")
    outs = exe(x, *ws, dtypes=[dt] * (1 + len(Ns)))
    monkeypatch.setenv("PJRTX_DOT_GROUPS", "0")
    single = client.compile(text)
    assert [s.get("library") for s in json.loads(single.optimized_program())["steps"]] == ["dot_general"] * len(Ns)
    alone = single(x, *ws, dtypes=[dt] * (1 + len(Ns)))
    for got, ref, w, n in zip(outs, alone, ws, Ns):
        want = _f64(x, dt) @ _f64(w, dt)
        g = _f64(got, dt)
        assert np.abs(g - want).max() <= 2e-2 * np.abs(want).max()
        # Bit-identical where the dot alone takes the same one-pass kernel
        # (at least 32 tiles of 64 columns) or the group falls back to single
        # dots.
        if (n // 64 >= 32 and M * K <= 16384) or M * K > 16384:
            np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("M,K,N,dt", [(1, 2048, 2048, "bf16"), (2, 5632, 2048, "f16"), (1, 2048, 32000, "bf16")])
def test_residual_add_merged_into_dot(client, monkeypatch, M, K, N, dt):
    """x + dot(h, w) with the dot read only by the add: one launch writing
    the sum, bit-identical to the dot followed by the elementwise add."""
    monkeypatch.setenv("PJRTX_GEMV_FUSION", "0")
    rng = np.random.default_rng(K + N)
    b = Builder()
    h, w, x = b.param((M, K), dt), b.param((K, N), dt), b.param((M, N), dt)
    text = b.build([b.add(x, b.dot_general(h, w, contract=((1,), (0,))))])
    args = [_bits(rng, (M, K), dt), _bits(rng, (K, N), dt, 1 / np.sqrt(K)), _bits(rng, (M, N), dt)]
    exe = client.compile(text)
    steps = json.loads(exe.optimized_program())["steps"]
    assert len(steps) == 1 and "residual_add" in steps[0]
    (got,) = exe(*args, dtypes=[dt] * 3)
    monkeypatch.setenv("PJRTX_DOT_RESIDUAL", "0")
    plain = client.compile(text)
    assert len(json.loads(plain.optimized_program())["steps"]) == 2
    (want,) = plain(*args, dtypes=[dt] * 3)
    np.testing.assert_array_equal(got, want)
    ref = _f64(args[2], dt) + _f64(args[0], dt) @ _f64(args[1], dt)
    assert np.abs(_f64(got, dt) - ref).max() <= 2e-2 * np.abs(ref).max()
