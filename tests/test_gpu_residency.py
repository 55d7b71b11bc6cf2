"""Device residency budget (the reference's executable residency cache:
src/runtime/executable_cache.zig:118-300, client_residency_tests.zig): each
loaded executable's device bytes (code object, resident constants, kernel
scratch) count against a per-device cap; loading past it evicts idle
executables, largest first, then least recently used, and an evicted
executable loads again, with the same results, when it next runs."""
import gc

import numpy as np
import pytest

from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu

N = 1 << 16   # 256 KiB of f32 constant per program


def _prog(i):
    b = Builder(f"jit_resident_{i}")
    x = b.param((N,), "f32")
    vals = (np.arange(N, dtype=np.float32) % 97) * np.float32(i + 1)
    c = b.dense(vals.tolist(), "f32", (N,))
    return b.build([b.add(x, c)]), vals


@pytest.fixture
def uncapped(plugin):
    plugin.set_max_resident_bytes(0, 0)
    yield plugin
    plugin.set_max_resident_bytes(0, 0)


def test_eviction_under_a_small_cap(client, uncapped):
    p = uncapped
    x = np.random.default_rng(0).standard_normal(N).astype(np.float32)
    progs = [_prog(i) for i in range(3)]
    s0 = p.residency_stats(0)
    exes = [client.compile(progs[0][0])]   # compiling loads it
    s1 = p.residency_stats(0)
    (got,) = exes[0](x)
    np.testing.assert_array_equal(got, x + progs[0][1])
    one = s1["resident_bytes"] - s0["resident_bytes"]
    assert one >= 4 * N, s1   # the constant at least
    # Room for one of these executables only.
    cap = one + one // 2
    p.set_max_resident_bytes(0, cap)
    assert p.residency_stats(0)["max_resident_bytes"] == cap
    ev = p.residency_stats(0)["evictions"]
    exes += [client.compile(t) for t, _ in progs[1:]]   # each load evicts
    assert p.residency_stats(0)["resident_bytes"] <= cap
    for k in (1, 2, 0, 2, 1):
        (got,) = exes[k](x)
        np.testing.assert_array_equal(got, x + progs[k][1])
        st = p.residency_stats(0)
        assert st["resident_bytes"] <= cap, st
    st = p.residency_stats(0)
    assert st["evictions"] >= ev + 6 and st["evicted_bytes"] >= 6 * one, st
    # No cap: everything loads again and stays.
    p.set_max_resident_bytes(0, 0)
    for k in range(3):
        (got,) = exes[k](x)
        np.testing.assert_array_equal(got, x + progs[k][1])
    assert p.residency_stats(0)["resident_bytes"] >= 3 * one


def test_destroyed_executables_leave_the_budget(client, uncapped):
    p = uncapped
    text, vals = _prog(7)
    x = np.zeros(N, np.float32)
    before = p.residency_stats(0)["resident_bytes"]
    exe = client.compile(text)
    (got,) = exe(x)
    np.testing.assert_array_equal(got, vals)
    assert p.residency_stats(0)["resident_bytes"] >= before + 4 * N
    del exe
    gc.collect()
    assert p.residency_stats(0)["resident_bytes"] == before


def test_measured_mfma_peak_is_plausible(plugin):
    """The calibration kernel behind roofline.measured_peak: dense bf16 MFMA
    on every SIMD sustains most of the published 2.5 PFLOP/s and never more."""
    for shape in (0, 1):
        tf = plugin.mfma_peak_tflops(0, shape)
        assert 800.0 < tf < 2600.0, (shape, tf)
