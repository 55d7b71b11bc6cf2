"""Pins the attention oracle (oracle/attention.py) against the reference's
known answers for its scaled-dot-product-attention custom call
(tests/golden/reference_kats.json, transcribed from
src/backend/mlx_metal/api_test.cc:271-352) and against closed forms that a
dropped scale, a transposed operand, a wrong head mapping or an off-by-one
mask would break."""
import json
import pathlib

import numpy as np
import pytest

from oracle import attention as A

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


@pytest.mark.parametrize("name", ["sdpa_one_head", "sdpa_grouped_heads"])
def test_sdpa_reference_kats(name):
    k = KATS[name]
    q = np.array(k["q"], np.float32).reshape(k["q_shape"])
    kk = np.array(k["k"], np.float32).reshape(k["kv_shape"])
    v = np.array(k["v"], np.float32).reshape(k["kv_shape"])
    out = A.sdpa_f64(q, kk, v, np.uint32(k["token_index"]))
    np.testing.assert_allclose(out.reshape(-1), k["expected"], atol=1e-12)


def test_equal_scores_give_running_means():
    """k = 0: every allowed key scores the same, so query i returns the mean
    of value rows 0..i (causal, offset 0), and of all rows without a mask."""
    rng = np.random.default_rng(0)
    q = rng.standard_normal((2, 3, 7, 8))
    k = np.zeros((2, 3, 7, 8))
    v = rng.standard_normal((2, 3, 7, 8))
    out = A.attention_f64(q, k, v, scale=0.7, causal=True)
    want = np.cumsum(v, axis=2) / np.arange(1, 8)[:, None]
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-12)
    out = A.attention_f64(q, k, v, scale=0.7, causal=False)
    np.testing.assert_allclose(out, np.broadcast_to(v.mean(2, keepdims=True), v.shape), rtol=1e-12, atol=1e-12)


def test_offset_and_slope_of_the_mask():
    """k = 0 again: query i sees keys 0..min(i*q_coef + offset, Skv-1)."""
    rng = np.random.default_rng(1)
    v = rng.standard_normal((1, 2, 9, 4))
    q = rng.standard_normal((1, 2, 5, 4))
    k = np.zeros((1, 2, 9, 4))
    for q_coef, offset in [(1, 3), (0, 4), (1, -0)]:
        out = A.attention_f64(q, k, v, causal=True, q_coef=q_coef, offset=offset)
        for i in range(5):
            n = min(q_coef * i + offset, 8) + 1
            np.testing.assert_allclose(out[:, :, i], v[:, :, :n].mean(2), rtol=1e-12, atol=1e-12)


def test_dominant_score_selects_its_row_and_first_query_is_exact():
    rng = np.random.default_rng(2)
    D, S = 16, 12
    k = rng.standard_normal((1, 1, S, D))
    v = rng.standard_normal((1, 1, S, D))
    j = 5
    q = 200.0 * k[:, :, j:j + 1, :] / np.linalg.norm(k[0, 0, j])  # q.k_j dominates every other key by far
    out = A.attention_f64(q, k, v, causal=False)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0, j], rtol=1e-9, atol=1e-9)
    # Causal, offset 0: query 0 may only read key 0, whatever the scores.
    qq = rng.standard_normal((1, 1, 3, D))
    out = A.attention_f64(qq, k, v, causal=True)
    np.testing.assert_array_equal(out[0, 0, 0], v[0, 0, 0])


def test_grouped_heads_equal_repeated_heads_and_empty_rows_are_nan():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 6, 4, 8))
    k = rng.standard_normal((1, 2, 5, 8))
    v = rng.standard_normal((1, 2, 5, 8))
    grouped = A.attention_f64(q, k, v, causal=True, offset=1)
    for h in range(6):
        one = A.attention_f64(q[:, h:h + 1], k[:, h // 3:h // 3 + 1], v[:, h // 3:h // 3 + 1], causal=True, offset=1)
        np.testing.assert_allclose(grouped[:, h:h + 1], one, rtol=1e-14)
    empty = A.attention_f64(q, k, v, causal=True, offset=-1)  # query 0 has no allowed key
    assert np.isnan(empty[:, :, 0]).all() and not np.isnan(empty[:, :, 1:]).any()


def test_custom_call_layouts_and_scale():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((6, 4, 16)).astype(np.float32)   # [q, h, hd]
    k = rng.standard_normal((9, 2, 16)).astype(np.float32)
    v = rng.standard_normal((9, 2, 16)).astype(np.float32)
    r3 = A.sdpa_f64(q, k, v, np.int32(2))
    r4 = A.sdpa_f64(q[None], k[None], v[None], np.int32(2))
    np.testing.assert_allclose(r3, r4[0], rtol=1e-14)
    # scale 1/sqrt(16) = 0.25: the same as unscaled attention on q / 4.
    t = lambda x: np.transpose(x[None], (0, 2, 1, 3))  # noqa: E731
    plain = A.attention_f64(t(q) * 0.25, t(k), t(v), causal=True, offset=2)
    np.testing.assert_allclose(r3, np.transpose(plain, (0, 2, 1, 3))[0], rtol=1e-12)
    # token index cast to int32: 2**32 + 2 behaves as 2.
    np.testing.assert_allclose(A.sdpa_f64(q, k, v, np.int64(2**32 + 2)), r3, rtol=1e-14)


def test_graph_ref_close_to_f64():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 2, 33, 64)).astype(np.float32) / 8
    k = rng.standard_normal((1, 2, 33, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 33, 64)).astype(np.float32)
    for dt in ["bf16", "f16"]:
        r = lambda x: A._round16(x, dt)  # noqa: E731
        g = A.attention_graph_ref(r(q), r(k), r(v), dt, causal=True)
        f = A.attention_f64(r(q), r(k), r(v), causal=True)
        assert np.abs(g - f).max() <= 2e-2 * np.abs(f).max()
