"""hipGraph replay of repeated executions (runtime.cc, Executable::
capture_graph / replay_graph): the llama-like decode step is captured on its
second execution with the same weights and (donated, in-place) caches, then
replayed with the token and position staged in. Every replayed step must be
bit-identical to eager execution, including with eager work and host
synchronization between replays."""
import numpy as np
import pytest

from oracle import ops
from pjrtx_amd import llama_like as L
from pjrtx_amd import programs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def runner(client):
    return L.LlamaRunner(client, L.TINY, L.init_weights(L.TINY, seed=3))


def _decode(runner, client, prompt, steps, between=None):
    tok, logits, caches = runner.start(prompt)
    toks, lgs = [int(tok.to_numpy()[0])], [logits.to_numpy()]
    for i in range(steps):
        pos = client.buffer(np.array(len(prompt) + i, np.int32))
        tok, logits, caches = runner.step_with(tok, pos, caches)
        toks.append(int(tok.to_numpy()[0]))
        lgs.append(logits.to_numpy())
        if between is not None:
            between(i)
    return toks, lgs


def test_graph_replay_matches_eager(runner, client, monkeypatch):
    prompt = L.prompt_tokens(L.TINY, seed=11)
    steps = L.TINY.max_len - L.TINY.prompt - 1
    monkeypatch.setenv("PJRTX_GRAPHS", "0")
    eager_toks, eager_logits = _decode(runner, client, prompt, steps)
    before = runner.decode.graph_stats()
    monkeypatch.setenv("PJRTX_GRAPHS", "1")
    other = client.compile(programs.c2_argmax_only(4, 1000))
    x = ops.f32_to_bf16_bits(np.random.default_rng(0).standard_normal((4, 1000)).astype(np.float32))
    want_idx = ops.argmax_rows(ops.bf16_bits_to_f32(x))[1]

    def eager_work(i):  # unrelated eager executions and host reads between replays
        _, idx = other(x, dtypes=["bf16"])
        np.testing.assert_array_equal(idx, want_idx)

    graph_toks, graph_logits = _decode(runner, client, prompt, steps, between=eager_work)
    after = runner.decode.graph_stats()
    assert graph_toks == eager_toks
    for a, b in zip(graph_logits, eager_logits):
        np.testing.assert_array_equal(a, b)
    assert after["captures"] - before["captures"] >= 1
    assert after["replays"] - before["replays"] >= steps - 2


def test_graph_entries_follow_new_caches(runner, client):
    """A new generation brings new cache buffers: the executable captures
    again (or finds its entry) and stays bit-identical to eager."""
    prompt = L.prompt_tokens(L.TINY, seed=12)
    t1, l1 = _decode(runner, client, prompt, 6)
    t2, l2 = _decode(runner, client, prompt, 6)
    assert t1 == t2
    for a, b in zip(l1, l2):
        np.testing.assert_array_equal(a, b)
