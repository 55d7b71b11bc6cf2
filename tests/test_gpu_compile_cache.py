"""Compile cache: compiling a program text again reuses its parsed and
planned form (a hit), yet gives an executable of its own (own statistics)
with the same results; a different PJRTX_* environment is a different
entry, because those switches change plans."""
import os
import time

import numpy as np
import pytest

from pjrtx_amd import llama_like as L
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


def _prog(tag):
    b = Builder(f"jit_cache_{tag}")
    x = b.param((64, 1000), "f32")
    return b.build([b.sum(b.multiply(x, x), [1])])


def test_second_compile_hits_and_runs_alone(client, plugin):
    text = _prog(os.getpid())
    before = plugin.compile_cache_stats()
    e1 = client.compile(text)
    mid = plugin.compile_cache_stats()
    e2 = client.compile(text)
    after = plugin.compile_cache_stats()
    assert mid["misses"] == before["misses"] + 1 and after["hits"] == mid["hits"] + 1
    x = np.random.default_rng(0).standard_normal((64, 1000)).astype(np.float32)
    np.testing.assert_array_equal(e1(x), e2(x))
    assert e1.stats()["executions"] == 1 and e2.stats()["executions"] == 1


def test_environment_switch_is_a_separate_entry(client, plugin, monkeypatch):
    text = _prog(f"env{os.getpid()}")
    client.compile(text)
    before = plugin.compile_cache_stats()
    monkeypatch.setenv("PJRTX_REDUCE_TARGET_BLOCKS", "64")
    client.compile(text)
    assert plugin.compile_cache_stats()["misses"] == before["misses"] + 1


def test_cached_decode_compile(client, plugin):
    text = L.decode_program(L.FULL)
    t0 = time.perf_counter()
    client.compile(text)
    first = time.perf_counter() - t0
    hits = plugin.compile_cache_stats()["hits"]
    t0 = time.perf_counter()
    client.compile(text)
    second = time.perf_counter() - t0
    print(f"decode program compile: first {first * 1e3:.1f} ms, again {second * 1e3:.1f} ms")
    assert plugin.compile_cache_stats()["hits"] == hits + 1


def test_byte_cap_evicts_least_recent(client, plugin, monkeypatch):
    """PJRTX_COMPILE_CACHE_BYTES caps the host bytes the cache holds: with
    room for one program, compiling a second evicts the first (compiling it
    again is a miss), and the held bytes stay under the cap."""
    a, b = _prog(f"capA{os.getpid()}"), _prog(f"capB{os.getpid()}")
    monkeypatch.setenv("PJRTX_COMPILE_CACHE_BYTES", str(len(a) + len(a) // 2))
    client.compile(a)
    s0 = plugin.compile_cache_stats()
    client.compile(b)
    s1 = plugin.compile_cache_stats()
    assert s1["evictions"] > s0["evictions"] and s1["bytes"] <= len(a) + len(a) // 2
    client.compile(a)
    assert plugin.compile_cache_stats()["misses"] == s1["misses"] + 1


def test_fingerprint_names_the_entry(plugin, monkeypatch):
    text = _prog("fp")
    f1 = plugin.compile_fingerprint(text)
    assert f1.startswith("pjrtx-") and len(f1) == 38 and f1 == plugin.compile_fingerprint(text)
    assert plugin.compile_fingerprint(_prog("fp2")) != f1
    monkeypatch.setenv("PJRTX_REDUCE_TARGET_BLOCKS", "64")
    assert plugin.compile_fingerprint(text) != f1
