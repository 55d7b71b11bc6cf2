"""Fused attention on the GPU (kernels/attention.hip through attention.cc):
the reference's scaled-dot-product-attention custom call and the rewritten
softmax-attention pattern, against the float64 oracle (oracle/attention.py)
and against the unfused path.

Tolerances: f32 within 1e-5 relative (the row kernel accumulates in f32);
bf16 / f16 outputs within 2e-2 of the row's scale (the fused kernel rounds
the probabilities to the input type before the division by the row sum; the
unfused graph after it). The first query of a causal mask reads only key 0,
so its output equals value row 0 bit for bit on every path."""
import json
import pathlib

import numpy as np
import pytest

from oracle import attention as A
from oracle import ops
from pjrtx_amd import programs
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu

SDPA = "pjrtx.mlx_metal.scaled_dot_product_attention"
KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def to_bits(x, dt):
    x = np.asarray(x, np.float32)
    return ops.f32_to_bf16_bits(x) if dt == "bf16" else x.astype(np.float16)


def from_bits(b, dt):
    if dt == "bf16":
        return ops.bf16_bits_to_f32(b).astype(np.float64)
    return np.asarray(b, np.float64)


def assert_close16(got, want, rtol=2e-2):
    want = np.asarray(want, np.float64)
    scale = np.sqrt(np.mean(want ** 2, axis=-1, keepdims=True)) + 1e-30
    err = np.abs(got - want) / np.maximum(np.abs(want), scale)
    assert err.max() <= rtol, f"max scaled error {err.max():.3g}"


def sdpa_exe(client, dt, qs, kvs, tok_dtype="s32"):
    b = Builder()
    q, k, v = b.param(qs, dt), b.param(kvs, dt), b.param(kvs, dt)
    t = b.param((), tok_dtype)
    return client.compile(b.build([b.custom_call(SDPA, [q, k, v, t], qs, dt)]))


@pytest.mark.parametrize("name", ["sdpa_one_head", "sdpa_grouped_heads"])
def test_sdpa_reference_kats(client, name):
    k = KATS[name]
    exe = sdpa_exe(client, "f32", tuple(k["q_shape"]), tuple(k["kv_shape"]), "u32")
    arr = lambda key, shp: np.array(k[key], np.float32).reshape(shp)  # noqa: E731
    (out,) = exe(arr("q", k["q_shape"]), arr("k", k["kv_shape"]), arr("v", k["kv_shape"]),
                 np.array(k["token_index"], np.uint32))
    np.testing.assert_allclose(out.reshape(-1), k["expected"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("qs,kvs,tok", [
    ((3, 4, 16), (9, 2, 16), 2),
    ((1, 7, 2, 48), (1, 33, 1, 48), 20),
    ((2, 5, 8, 130), (2, 70, 4, 130), 60),
    ((4, 2, 64), (4, 2, 64), -1),          # query 0 has no allowed key: NaN
])
def test_sdpa_f32_rows(client, qs, kvs, tok):
    rng = np.random.default_rng(sum(qs) + tok)
    q = rng.standard_normal(qs).astype(np.float32)
    k = rng.standard_normal(kvs).astype(np.float32)
    v = rng.standard_normal(kvs).astype(np.float32)
    (out,) = sdpa_exe(client, "f32", qs, kvs)(q, k, v, np.array(tok, np.int32))
    want = A.sdpa_f64(q, k, v, np.int32(tok))
    np.testing.assert_array_equal(np.isnan(out), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_allclose(out[ok], want[ok], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("qs,kvs,tok", [
    ((1, 1, 16, 128), (1, 640, 16, 128), 517),   # decode-shaped: one query over a cache
    ((5, 8, 64), (40, 2, 64), 30),               # grouped heads, row kernel
    ((1, 200, 8, 128), (1, 333, 2, 128), 100),   # tile kernel, ragged lengths, grouped heads
    ((2, 130, 4, 64), (2, 130, 4, 64), 0),       # tile kernel, head dim 64, causal from 0
    ((1, 2, 4, 64), (1, 2000, 2, 64), 100),      # decode, 8 key splits of which 7 are empty
    ((1, 1, 8, 128), (1, 5000, 8, 128), 4321),   # decode, 20 key splits
])
def test_sdpa_16bit(client, dt, qs, kvs, tok):
    rng = np.random.default_rng(qs[-2] * 7 + kvs[-3] + tok)
    q = to_bits(rng.standard_normal(qs), dt)
    k = to_bits(rng.standard_normal(kvs), dt)
    v = to_bits(rng.standard_normal(kvs), dt)
    (out,) = sdpa_exe(client, dt, qs, kvs)(q, k, v, np.array(tok, np.int32), dtypes=[dt, dt, dt, None])
    want = A.sdpa_f64(from_bits(q, dt), from_bits(k, dt), from_bits(v, dt), np.int32(tok))
    assert_close16(from_bits(out, dt), want)
    if tok == 0:  # first query: value row 0 exactly
        np.testing.assert_array_equal(np.asarray(out)[..., 0, :, :] if len(qs) == 4 else out[0],
                                      np.asarray(v)[..., 0, :, :] if len(qs) == 4 else v[0])


@pytest.mark.parametrize("b_,h,s,d,dt,causal", [
    (1, 4, 200, 128, "bf16", True),
    (2, 2, 256, 64, "bf16", False),
    (1, 2, 96, 128, "f16", True),
    (1, 1, 8, 64, "bf16", True),   # few queries: row kernel
])
def test_fused_pattern_matches_unfused(client, monkeypatch, b_, h, s, d, dt, causal):
    rng = np.random.default_rng(s + d)
    shp = (b_, h, s, d)
    q = to_bits(rng.standard_normal(shp) / np.sqrt(d), dt)
    k = to_bits(rng.standard_normal(shp), dt)
    v = to_bits(rng.standard_normal(shp), dt)
    text = programs.c3_attention(b_, h, s, d, causal=causal, dtype=dt)
    fused = client.compile(text)
    assert [st.get("library") for st in json.loads(fused.optimized_program())["steps"]] == ["attention"]
    (got,) = fused(q, k, v, dtypes=[dt] * 3)
    monkeypatch.setenv("PJRTX_FUSED_ATTENTION", "0")
    (plain,) = client.compile(text)(q, k, v, dtypes=[dt] * 3)
    want = A.attention_graph_ref(from_bits(q, dt), from_bits(k, dt), from_bits(v, dt), dt, causal=causal)
    assert_close16(from_bits(got, dt), want)
    assert_close16(from_bits(got, dt), from_bits(plain, dt))
    if causal:
        np.testing.assert_array_equal(np.asarray(got)[:, :, 0], np.asarray(v)[:, :, 0])


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_decode_split_merge_paths_agree(client, run_fresh, dt):
    """Decode attention splits the keys over workgroups. Merged in the same
    launch by the row's last split (XCD-local counters) or by the separate
    merge kernel (PJRTX_XCD_LOCAL=0, a fresh process): same merge order,
    same bits; both match the float64 oracle."""
    qs, kvs, tok = (1, 1, 16, 128), (1, 640, 16, 128), 517
    rng = np.random.default_rng(11)
    conv = (lambda x: to_bits(x, dt)) if dt != "f32" else (lambda x: np.asarray(x, np.float32))
    q, k, v = conv(rng.standard_normal(qs)), conv(rng.standard_normal(kvs)), conv(rng.standard_normal(kvs))
    b = Builder()
    pq, pk, pv, t = b.param(qs, dt), b.param(kvs, dt), b.param(kvs, dt), b.param((), "s32")
    text = b.build([b.custom_call(SDPA, [pq, pk, pv, t], qs, dt)])
    dts = [dt, dt, dt, None] if dt != "f32" else [None] * 4
    args = [q, k, v, np.array(tok, np.int32)]
    (got,) = client.compile(text)(*args, dtypes=dts)
    (other,) = run_fresh(text, args, dts, {"PJRTX_XCD_LOCAL": "0"})
    np.testing.assert_array_equal(got, other)
    want = A.sdpa_f64(from_bits(q, dt) if dt != "f32" else q, from_bits(k, dt) if dt != "f32" else k,
                      from_bits(v, dt) if dt != "f32" else v, np.int32(tok))
    if dt == "f32":
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    else:
        assert_close16(from_bits(got, dt), want)
