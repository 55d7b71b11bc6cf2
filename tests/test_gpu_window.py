"""In-place dynamic_update_slice fused into the elementwise kernel that
computes its update (planner absorb_window_updates): the kernel stores the
update at the clamped window offset of the operand's buffer. Checked against
numpy with StableHLO's start clamping, including out-of-range starts."""
import json

import numpy as np
import pytest

from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


def _program():
    b = Builder()
    cache = b.param((2, 8, 16), "f32")
    x = b.param((2, 1, 16), "f32")
    pos = b.param((), "s32")
    op = b.add(cache, b.scalar_like(1.0, cache))          # an intermediate: updated in place
    u = b.multiply(x, b.scalar_like(2.0, x))              # the update, computed by a kernel
    z = b.constant(0, "s32")
    r = b.dynamic_update_slice(op, u, [z, pos, z])
    return b.build([r])


def test_window_update_is_fused_and_clamped(client):
    exe = client.compile(_program())
    steps = json.loads(exe.optimized_program())["steps"]
    assert "dynamic_update_slice" not in [s.get("library") for s in steps]
    assert sum(len(s.get("window_outputs", [])) for s in steps) == 1
    rng = np.random.default_rng(0)
    cache = rng.standard_normal((2, 8, 16)).astype(np.float32)
    x = rng.standard_normal((2, 1, 16)).astype(np.float32)
    for p in [-3, 0, 5, 7, 12]:
        (got,) = exe(cache, x, np.array(p, np.int32))
        want = cache + 1.0
        q = min(max(p, 0), 7)
        want[:, q:q + 1, :] = x * 2.0
        np.testing.assert_array_equal(got, want)


def test_shift_written_back_in_place_matches_numpy(client):
    # c[0:7] = -c[1:8] into the donated c: the update kernel reads c, so the
    # write must stay its own step (a fused window write would race).
    b = Builder()
    c_in = b.param((8, 16), "f32", donate=True)
    u = b.negate(b.slice(c_in, [1, 0], [8, 16]))
    z = b.constant(0, "s32")
    exe = client.compile(b.build([b.dynamic_update_slice(c_in, u, [z, z])]))
    steps = json.loads(exe.optimized_program())["steps"]
    assert not any(s.get("window_outputs") for s in steps)
    c = np.random.default_rng(1).standard_normal((8, 16)).astype(np.float32)
    (got,) = exe(c)
    want = c.copy()
    want[0:7] = -c[1:8]
    np.testing.assert_array_equal(got, want)
