"""Pins the llama-like decoder oracle (oracle/llama.py) with closed forms, an
independent float64 restatement and the KV-cache consistency property."""
import dataclasses

import numpy as np

from oracle import llama as O
from pjrtx_amd import llama_like as L

CFG = L.TINY


def _weights(cfg=CFG, seed=0):
    return O.weights_f32(cfg, L.init_weights(cfg, seed))


def test_weight_layout_matches_config():
    assert L.num_params(L.FULL) == 542_148_608  # 8 layers, d 2048, ffn 5632, vocab 32000, untied lm_head
    shapes = dict(L.weight_shapes(L.FULL))
    assert shapes["l7.w2"] == (5632, 2048) and shapes["lm_head"] == (2048, 32000)


def test_bf16_round_ties_to_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -2.5], np.float32)
    np.testing.assert_array_equal(O.bf16_round(x), [1.0, 1.0, 1.0 + 2 ** -6, 1.0, -2.5])


def test_rope_is_a_rotation():
    rng = np.random.default_rng(0)
    x = O.bf16_round(rng.standard_normal((CFG.heads, 5, CFG.head_dim)).astype(np.float32))
    cos, sin = O.rope_tables(CFG, np.arange(5, dtype=np.int32))
    y = (x * cos[None] + np.concatenate([-x[..., 16:], x[..., :16]], -1) * sin[None])
    half = CFG.head_dim // 2
    n_in = x[..., :half] ** 2 + x[..., half:] ** 2
    n_out = y[..., :half] ** 2 + y[..., half:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)
    # position 0 is the identity (after bf16 rounding of an already-bf16 input)
    np.testing.assert_array_equal(O.rope(x[:, :1], cos[:1], sin[:1]), x[:, :1])


def test_rope_scores_depend_on_position_difference():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 1, CFG.head_dim)).astype(np.float32)
    k = rng.standard_normal((1, 1, CFG.head_dim)).astype(np.float32)

    def rot(a, p):
        c, s = O.rope_tables(CFG, np.array([p], np.int32))
        half = CFG.head_dim // 2
        return a * c[None] + np.concatenate([-a[..., half:], a[..., :half]], -1) * s[None]

    d1 = float(np.sum(rot(q, 7) * rot(k, 3)))
    d2 = float(np.sum(rot(q, 14) * rot(k, 10)))
    assert abs(d1 - d2) < 1e-4 * max(1.0, abs(d1))


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(2)
    x = O.bf16_round(rng.standard_normal((3, CFG.d_model)).astype(np.float32))
    w = O.bf16_round(rng.standard_normal(CFG.d_model).astype(np.float32))
    got = O.rmsnorm(x, w, 1e-5)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-5) * w
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2)


def test_uniform_attention_gives_running_mean_of_values():
    cfg = dataclasses.replace(CFG, layers=1)
    W = _weights(cfg)
    W["l0.wq"][:] = 0.0  # q = 0 -> all unmasked scores 0 -> uniform weights
    kc, vc = O.empty_caches(cfg)
    toks = np.array([5, 9, 2, 7], np.int32)
    O.forward(cfg, W, toks, 0, kc, vc)
    # Recompute what the context of the last position must be: mean of V rows.
    x = W["embed"][toks]
    h = O.rmsnorm(x, W["l0.attn_norm"], cfg.eps)
    v = O.mm(h, W["l0.wv"]).reshape(4, cfg.heads, cfg.head_dim).transpose(1, 0, 2)
    np.testing.assert_array_equal(vc[0][:, :4], v)
    # with q == 0 the weights over the 4 visible keys are exactly 1/4
    p = np.full((cfg.heads, 1, cfg.max_len), 0.0, np.float32)
    p[..., :4] = 0.25
    want = O.bf16_round(np.matmul(p, vc[0]))[:, 0]
    np.testing.assert_allclose(want, v.mean(axis=1), rtol=1e-2, atol=1e-3)


def test_forward_matches_float64_restatement():
    W = _weights()
    prompt = L.prompt_tokens(CFG, seed=3)
    kc, vc = O.empty_caches(CFG)
    _, logits = O.forward(CFG, W, prompt, 0, kc, vc)
    want = O.forward_f64(CFG, W, prompt)
    scale = np.abs(want).max()
    assert np.abs(logits - want).max() < 3e-2 * scale
    assert np.corrcoef(logits, want)[0, 1] > 0.999


def test_kv_cache_decode_equals_longer_prefill():
    W = _weights()
    prompt = L.prompt_tokens(CFG, seed=4)
    kc, vc = O.empty_caches(CFG)
    t0, _ = O.forward(CFG, W, prompt, 0, kc, vc)
    _, step_logits = O.forward(CFG, W, np.array([t0], np.int32), len(prompt), kc, vc)
    kc2, vc2 = O.empty_caches(CFG)
    _, full_logits = O.forward(CFG, W, np.append(prompt, t0).astype(np.int32), 0, kc2, vc2)
    np.testing.assert_allclose(step_logits, full_logits, rtol=0, atol=2e-2 * np.abs(full_logits).max())
    for a, b in zip(kc, kc2):
        np.testing.assert_allclose(a[:, :len(prompt) + 1], b[:, :len(prompt) + 1], atol=2e-2)


def test_greedy_generate_follows_argmax_and_teacher_forcing():
    W = _weights()
    prompt = L.prompt_tokens(CFG, seed=5)
    toks, logits = O.generate(CFG, W, prompt, 4)
    assert [int(np.argmax(lg)) for lg in logits] == toks.tolist()
    toks2, logits2 = O.generate(CFG, W, prompt, 4, forced=toks[:-1])
    np.testing.assert_array_equal(toks2, toks)
    for a, b in zip(logits, logits2):
        np.testing.assert_array_equal(a, b)


def test_incremental_float64_decoder_equals_full_recompute():
    """The incremental float64 decoder (caches in float64) gives, after the
    prefill and after each decode step, the logits of `forward_f64` over the
    whole prefix: an independent full recompute (float64 rounding only)."""
    W = _weights()
    prompt = L.prompt_tokens(CFG, seed=6)
    dec = O.DecoderF64(CFG, W)
    seen = list(prompt)
    got = dec.step(prompt)
    np.testing.assert_allclose(got, O.forward_f64(CFG, W, np.array(seen)), rtol=0, atol=1e-10)
    rng = np.random.default_rng(8)
    for _ in range(CFG.max_len - len(prompt)):
        t = int(rng.integers(0, CFG.vocab))
        got = dec.step([t])
        seen.append(t)
        want = O.forward_f64(CFG, W, np.array(seen))
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-10 * max(1.0, np.abs(want).max()))
    assert dec.n == CFG.max_len
