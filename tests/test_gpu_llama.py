"""C5 llama-like decode through the plugin, checked against the numpy oracle
(oracle/llama.py): teacher-forced logits within bf16 tolerance, greedy
tokens, cache donation, and at full size the KV-cache property (one decode
step equals a one-token-longer prefill)."""
import numpy as np
import pytest

from oracle import llama as O
from pjrtx_amd import llama_like as L

pytestmark = pytest.mark.gpu

# bf16 logits: the program rounds every stored activation to bf16, and
# the GPU accumulates dots and sums in a different order from numpy. The
# bar is 2e-2 of the logit range.
TOL = 2e-2


def _check_step(gpu_logits, ora_logits, gpu_tok):
    scale = float(np.abs(ora_logits).max())
    err = float(np.abs(gpu_logits - ora_logits).max())
    assert err <= TOL * scale, f"logits differ by {err} (scale {scale})"
    assert gpu_tok == int(np.argmax(gpu_logits))  # the program's argmax of its own logits
    top = np.sort(ora_logits)[::-1]
    if top[0] - top[1] > 2 * TOL * scale:  # a clear winner must agree
        assert gpu_tok == int(np.argmax(ora_logits))


def _gpu_logits(buf):
    return O.bf16_bits_to_f32(buf.to_numpy())[0]


@pytest.fixture(scope="module")
def tiny(client):
    w = L.init_weights(L.TINY, seed=0)
    return L.LlamaRunner(client, L.TINY, w), O.weights_f32(L.TINY, w)


def _first_flip_is_exempt(gpu_toks, ora_toks, ora_logits):
    """Free-running greedy sequences must be equal; they may part only at a
    step where the oracle's top-2 margin is within the logit bar (2 x TOL of
    the logit range), and the comparison ends there (the histories differ
    afterwards). Returns the step of the parting, or None."""
    for i, (a, b) in enumerate(zip(gpu_toks, ora_toks)):
        if int(a) != int(b):
            ref = np.asarray(ora_logits[i], np.float64)
            top = np.sort(ref)[::-1]
            assert top[0] - top[1] <= 2 * TOL * np.abs(ref).max(), (i, a, b, top[:2])
            return i
    return None


def test_tiny_greedy_decode_matches_oracle(tiny):
    runner, W = tiny
    cfg = L.TINY
    for seed in (1, 2, 3):
        prompt = L.prompt_tokens(cfg, seed=seed)
        toks, _, logits = runner.generate(prompt, cfg.new_tokens, keep_logits=True)
        # teacher-forced logits, step by step
        _, forced_logits = O.generate(cfg, W, prompt, cfg.new_tokens, forced=toks[:-1])
        for i in range(cfg.new_tokens):
            _check_step(O.bf16_bits_to_f32(logits[i])[0], forced_logits[i], int(toks[i]))
        # free-running greedy tokens: equal, up to a margin-exempt parting
        ora_toks, ora_logits = O.generate(cfg, W, prompt, cfg.new_tokens)
        _first_flip_is_exempt(toks, ora_toks, ora_logits)


def test_tiny_cache_donation(tiny, client):
    runner, _ = tiny
    cfg = L.TINY
    prompt = L.prompt_tokens(cfg, seed=2)
    tok, _, caches = runner.start(prompt)
    # Not donated: the caller's caches stay valid and unchanged.
    before = [c.to_numpy() for c in caches]
    pos = client.buffer(np.array(len(prompt), np.int32))
    nd = list(range(len(runner.weights) + 2, len(runner.weights) + 2 + len(caches)))
    outs_keep = runner.decode.execute_buffers(runner.weights + [tok, pos] + caches, non_donatable=nd)
    assert not any(c.is_deleted() for c in caches)
    for c, b in zip(caches, before):
        np.testing.assert_array_equal(c.to_numpy(), b)
    # Donated: same results, the inputs read as deleted afterwards.
    outs = runner.decode.execute_buffers(runner.weights + [tok, pos] + caches)
    assert all(c.is_deleted() for c in caches)
    for a, b in zip(outs, outs_keep):
        np.testing.assert_array_equal(a.to_numpy(), b.to_numpy())
    # The new token's row was written at the position; earlier rows kept.
    k0 = outs[2].to_numpy()
    assert np.array_equal(k0[:, :, :len(prompt)], before[0][:, :, :len(prompt)])
    assert np.any(k0[:, :, len(prompt)] != 0)


def test_tiny_plan_updates_caches_in_place(client):
    import json
    exe = client.compile(L.decode_program(L.TINY))
    plan = json.loads(exe.optimized_program())
    dus = [s for s in plan["steps"] if s.get("library") == "dynamic_update_slice"]
    windows = [w for s in plan["steps"] for w in s.get("window_outputs", [])]
    # Every cache update is in place: its own step, or a window written by
    # the elementwise kernel that computes the row (RoPE of k, the v copy).
    assert len(dus) + len(windows) == 2 * L.TINY.layers and all(s["in_place"] for s in dus)
    assert len(plan["written_params"]) == 2 * L.TINY.layers


@pytest.fixture(scope="module")
def full(client):
    w = L.init_weights(L.FULL, seed=0)
    return L.LlamaRunner(client, L.FULL, w), w


def test_full_prefill_and_decode_match_oracle(full):
    """At full size the bf16 restatement's own rounding noise (8 layers, 512
    positions) is as large as the bar: its logits sit 0.072-0.074 (max) and
    1.9% (relative L2) from the float64 model, where 2e-2 x max|logit| is
    0.074-0.086. So the GPU is held to being as accurate as that faithful
    bf16 evaluation: its distance to the float64 restatement (no bf16
    rounding) may exceed the bf16 restatement's by at most 20%, in max and in
    relative L2, and it stays within twice the bar of the bf16 restatement
    (two evaluations each about the bar from the exact value)."""
    runner, wbits = full
    cfg = L.FULL
    W = O.weights_f32(cfg, wbits)
    prompt = L.prompt_tokens(cfg, seed=1)
    steps = 3
    toks, timing, logits = runner.generate(prompt, steps, keep_logits=True)
    kc, vc = O.empty_caches(cfg)
    seen = list(prompt)
    for i in range(steps):
        if i == 0:
            t, lg = O.forward(cfg, W, prompt, 0, kc, vc)
        else:
            t, lg = O.forward(cfg, W, np.array([toks[i - 1]], np.int32), len(prompt) + i - 1, kc, vc)
            seen.append(int(toks[i - 1]))
        exact = O.forward_f64(cfg, W, np.array(seen, np.int32))
        g = O.bf16_bits_to_f32(logits[i])[0].astype(np.float64)
        scale = float(np.abs(exact).max())
        norm = float(np.linalg.norm(exact))
        gpu_max, ora_max = np.abs(g - exact).max(), np.abs(lg - exact).max()
        gpu_l2, ora_l2 = np.linalg.norm(g - exact) / norm, np.linalg.norm(lg - exact) / norm
        assert gpu_max <= max(TOL * scale, 1.2 * ora_max), (i, gpu_max, ora_max, scale)
        assert gpu_l2 <= max(TOL, 1.2 * ora_l2), (i, gpu_l2, ora_l2)
        assert np.abs(g - lg).max() <= 2 * TOL * scale, (i, np.abs(g - lg).max(), scale)
        assert int(toks[i]) == int(np.argmax(g))
        top = np.sort(exact)[::-1]
        if top[0] - top[1] > 2 * TOL * scale:
            assert int(toks[i]) == int(np.argmax(exact))


def test_full_decode_128_steps_teacher_forced(full):
    """All 128 decode steps of C5 at full size, teacher-forced with the GPU's
    tokens, each held to the bar against the exact model: the incremental
    float64 decoder (float64 caches, no bf16 rounding; oracle.DecoderF64).

    A faithful bf16 evaluation of this model cannot meet 2e-2 of the largest
    logit at every step: the bf16 restatement (oracle.forward, numpy order)
    is off the exact logits by 1.9% of the logit range at the median step and
    exceeds 2e-2 at about a third of the steps (up to 2.5%), and by 1.9%
    relative L2 (up to 2.2%). So the GPU is held to that evaluation's own
    accuracy, step by step and on average:

    * per step, relative L2 distance from the exact logits at most
      max(2e-2, 1.2 x the restatement's), and max distance at most
      max(2e-2 x max|logit|, 1.5 x the restatement's) (the max over 32,000
      logits is an extreme value: the per-step ratio of two equally accurate
      evaluations spreads to about 1.2 over 128 steps, the L2 ratio to 1.1);
    * over the 128 steps, the mean relative L2 distance is within 2e-2, and
      the mean ratios of the GPU's distances (max and L2) to the
      restatement's are at most 1.05: the GPU is not systematically less
      accurate than the bf16 evaluation;
    * per step, within twice the bar of the restatement; the token is the
      argmax of the GPU's own logits, and it equals the exact argmax wherever
      the exact top-2 margin is wider than twice the bar.

    Measured (MI355X): GPU max distance 1.85% of the range at the median step
    (restatement 1.92%), relative L2 1.88% (1.91%); ratios median 0.99 (max)
    and 0.98 (L2). The steps where the GPU's token is not the exact argmax
    are printed (all inside the margin)."""
    runner, wbits = full
    cfg = L.FULL
    W = O.weights_f32(cfg, wbits)
    prompt = L.prompt_tokens(cfg, seed=1)
    steps = cfg.new_tokens
    toks, _, logits = runner.generate(prompt, steps, keep_logits=True)
    _, ora_logits = O.generate(cfg, W, prompt, steps, forced=toks[:-1])
    dec = O.DecoderF64(cfg, W)
    flips, stats = [], []
    for i in range(steps):
        exact = dec.step(prompt if i == 0 else [int(toks[i - 1])])
        g = O.bf16_bits_to_f32(logits[i])[0].astype(np.float64)
        lg = np.asarray(ora_logits[i], np.float64)
        scale = float(np.abs(exact).max())
        norm = float(np.linalg.norm(exact))
        gpu_max, ora_max = np.abs(g - exact).max(), np.abs(lg - exact).max()
        gpu_l2, ora_l2 = np.linalg.norm(g - exact) / norm, np.linalg.norm(lg - exact) / norm
        assert gpu_l2 <= max(TOL, 1.2 * ora_l2), (i, gpu_l2, ora_l2)
        assert gpu_max <= max(TOL * scale, 1.5 * ora_max), (i, gpu_max, ora_max, scale)
        assert np.abs(g - lg).max() <= 2 * TOL * scale, (i, np.abs(g - lg).max(), scale)
        assert int(toks[i]) == int(np.argmax(g))
        stats.append((gpu_max / scale, gpu_l2, gpu_max / ora_max, gpu_l2 / ora_l2))
        if int(toks[i]) != int(np.argmax(exact)):
            top = np.sort(exact)[::-1]
            assert top[0] - top[1] <= 2 * TOL * scale, (i, top[:2])
            flips.append(i)
    st = np.array(stats)
    print(f"C5 128 steps vs float64: max distance / range median {np.median(st[:, 0]):.4f} max {st[:, 0].max():.4f}; "
          f"relative L2 mean {st[:, 1].mean():.4f} max {st[:, 1].max():.4f}; GPU / restatement distance ratio mean "
          f"{st[:, 2].mean():.3f} (max), {st[:, 3].mean():.3f} (L2); steps where the GPU's token is not the exact "
          f"argmax (margin-exempt): {flips}")
    assert st[:, 1].mean() <= TOL, st[:, 1].mean()
    assert st[:, 2].mean() <= 1.05 and st[:, 3].mean() <= 1.05, (st[:, 2].mean(), st[:, 3].mean())


def test_full_decode_step_equals_longer_prefill(full, client):
    runner, _ = full
    cfg = L.FULL
    prompt = L.prompt_tokens(cfg, seed=7)
    tok, _, caches = runner.start(prompt)
    _, step_logits, _ = runner.step(tok, len(prompt), caches)
    import dataclasses
    longer = dataclasses.replace(cfg, prompt=cfg.prompt + 1)
    exe = client.compile(L.prefill_program(longer))
    ext = np.append(prompt, tok.to_numpy()[0]).astype(np.int32)
    z = np.zeros(L.cache_shape(cfg), np.uint16)
    outs = exe.execute_buffers(runner.weights + [client.buffer(ext)] +
                               [client.buffer(z, "bf16") for _ in range(2 * cfg.layers)])
    a, b = _gpu_logits(step_logits), _gpu_logits(outs[1])
    assert np.abs(a - b).max() <= TOL * np.abs(b).max()


def test_tiny_decode_loop_in_one_execute_matches_per_step(tiny):
    """All decode steps in one execute (stablehlo.while over a constant
    count) give the same greedy tokens as one execute per step."""
    runner, _ = tiny
    cfg = L.TINY
    prompt = L.prompt_tokens(cfg, seed=3)
    per_step, _, _ = runner.generate(prompt, cfg.new_tokens)
    looped, timing = runner.generate_in_one_execute(prompt, cfg.new_tokens)
    np.testing.assert_array_equal(looped, per_step)
    assert timing["decode_steps"] == cfg.new_tokens - 1


def test_full_decode_loop_in_one_execute_matches_per_step(full):
    runner, _ = full
    cfg = L.FULL
    prompt = L.prompt_tokens(cfg, seed=1)
    per_step, _, _ = runner.generate(prompt, 16)
    looped, _ = runner.generate_in_one_execute(prompt, 16)
    np.testing.assert_array_equal(looped, per_step)


# Caches of 200 slots: the decode attention splits each head's keys over 4
# workgroups of 64 keys, so the o-projection GEMV merges the attention's
# split partials (positions 60..69 go from one active split to two).
SPLIT = L.LlamaConfig(layers=2, d_model=128, heads=4, head_dim=32, ffn=320, vocab=512, max_len=200, prompt=60,
                      new_tokens=10)


def test_split_decode_attention_merged_in_gemv_matches_oracle(client):
    import json
    plan = json.loads(client.compile(L.decode_program(SPLIT)).optimized_program())
    assert sum(bool(s.get("partials_out")) for s in plan["steps"]) == SPLIT.layers
    assert sum(s.get("attention_splits_merged") == 4 for s in plan["steps"]) == SPLIT.layers
    w = L.init_weights(SPLIT, seed=0)
    runner = L.LlamaRunner(client, SPLIT, w)
    W = O.weights_f32(SPLIT, w)
    for seed in (1, 2):
        prompt = L.prompt_tokens(SPLIT, seed=seed)
        toks, _, logits = runner.generate(prompt, SPLIT.new_tokens, keep_logits=True)
        _, forced_logits = O.generate(SPLIT, W, prompt, SPLIT.new_tokens, forced=toks[:-1])
        for i in range(SPLIT.new_tokens):
            _check_step(O.bf16_bits_to_f32(logits[i])[0], forced_logits[i], int(toks[i]))


@pytest.mark.parametrize("env", [{}, {"PJRTX_GEMV_PERSIST": "1", "PJRTX_GEMV_PWGS": "256"}],
                         ids=["chunk_x", "whole_x"])
def test_full_decode_attention_merge_in_gemv_is_bit_exact(full, client, monkeypatch, env):
    """The o-projection GEMV's merge of the attention's split partials gives
    the same bits as the attention launch's own merge: every output of a
    decode step (token, logits, caches) at positions with one split active
    (0, 5, 63), with two (64, 65), with several (300) and with all ten (639),
    over random caches. `whole_x` stages all of X per workgroup (persistent
    GEMV items) instead of the workgroup's K chunk."""
    import json
    runner, _ = full
    cfg = L.FULL
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    merged = client.compile(L.decode_program(cfg))
    plan = json.loads(merged.optimized_program())
    oproj = [s for s in plan["steps"] if s.get("attention_splits_merged")]
    assert len(oproj) == cfg.layers and all(s["attention_splits_merged"] == 10 for s in oproj)
    assert all(s["stage_all_x"] == bool(env) for s in oproj)
    monkeypatch.setenv("PJRTX_ATTN_MERGE_GEMV", "0")
    own = client.compile(L.decode_program(cfg))
    assert not any(s.get("partials_out") for s in json.loads(own.optimized_program())["steps"])
    rng = np.random.default_rng(11)
    caches = [client.buffer(L.f32_to_bf16_bits(rng.standard_normal(L.cache_shape(cfg)).astype(np.float32)), "bf16")
              for _ in range(2 * cfg.layers)]
    tok = client.buffer(np.array([17], np.int32))
    for pos in (0, 5, 63, 64, 65, 300, 639):
        args = runner.weights + [tok, client.buffer(np.array(pos, np.int32))] + caches
        keep = list(range(len(args)))
        a = merged.execute_buffers(args, non_donatable=keep)
        b = own.execute_buffers(args, non_donatable=keep)
        for i, (x, y) in enumerate(zip(a, b)):
            np.testing.assert_array_equal(x.to_numpy(), y.to_numpy(), err_msg=f"position {pos}, output {i}")
