"""The allocation-free execute (pjrtx_executable_execute_noalloc) against the
ordinary PJRT execute of the same executable: bit-identical outputs, on two
calls in a row (the second with a smaller input), for plans whose kernels use
scratch blocks (split-reduction partials, scatter keys / sort / segments,
top_k sort words, split-K GEMV partials). Inputs and outputs are caller-owned
device memory; every intermediate and scratch block comes from the fixed
per-GPU block."""
import numpy as np
import pytest

from oracle import ops
from pjrtx_amd import programs
from pjrtx_amd.hlo import Builder
from pjrtx_amd.pjrt import DeviceArray, PjrtError

pytestmark = pytest.mark.gpu


def _dot_gemv(m, k, n):
    b = Builder()
    x = b.param((m, k), "bf16")
    w = b.param((k, n), "bf16")
    return b.build([b.dot_general(x, w, contract=((1,), (0,)))])


def _cases():
    rng = np.random.default_rng(11)
    big_c2 = ops.c2_inputs(64, 128256, seed=5)
    small_c2 = ops.c2_inputs(8, 4096, seed=6)
    rows, dim, n = 4096, 256, 65536
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    idx = ops.zipf_indices(n, rows, seed=3)
    upd = rng.standard_normal((n, dim)).astype(np.float32)
    xs = rng.standard_normal((512, 64)).astype(np.float32)
    idxs = ops.zipf_indices(4096, 512, seed=4)
    upds = rng.standard_normal((4096, 64)).astype(np.float32)
    lg = ops.f32_to_bf16_bits(rng.standard_normal((64, 128256)).astype(np.float32))
    lgs = ops.f32_to_bf16_bits(rng.standard_normal((4, 8192)).astype(np.float32))
    xb = ops.f32_to_bf16_bits(rng.standard_normal((4, 4096)).astype(np.float32))
    wb = ops.f32_to_bf16_bits((0.02 * rng.standard_normal((4096, 1000))).astype(np.float32))
    xbs = ops.f32_to_bf16_bits(rng.standard_normal((2, 1024)).astype(np.float32))
    wbs = ops.f32_to_bf16_bits((0.02 * rng.standard_normal((1024, 200))).astype(np.float32))
    return {
        "c2_argmax_f16": ((programs.c2_argmax_f16_reductions(64, 128256), [big_c2], ["bf16"]),
                          (programs.c2_argmax_f16_reductions(8, 4096), [small_c2], ["bf16"])),
        "scatter_add_f32": ((programs.c4_scatter_add(rows, dim, n, "f32"), [x, idx, upd], [None] * 3),
                            (programs.c4_scatter_add(512, 64, 4096, "f32"), [xs, idxs, upds], [None] * 3)),
        "top_k": ((programs.topk_logits(64, 128256, 50), [lg], ["bf16"]),
                  (programs.topk_logits(4, 8192, 16), [lgs], ["bf16"])),
        "gemv_split_k": ((_dot_gemv(4, 4096, 1000), [xb, wb], ["bf16"] * 2),
                         (_dot_gemv(2, 1024, 200), [xbs, wbs], ["bf16"] * 2)),
    }


def _run_noalloc(client, exe, arrays):
    p = client.p
    args = [DeviceArray.from_numpy(p, a) for a in arrays]
    ref = exe(*arrays, dtypes=[("bf16" if a.dtype == np.uint16 else None) for a in arrays])
    outs = [DeviceArray(p, r.nbytes) for r in ref]
    used = exe.execute_noalloc([a.ptr for a in args], [o.ptr for o in outs])
    return args, outs, ref, used


@pytest.mark.parametrize("case", ["c2_argmax_f16", "scatter_add_f32", "top_k", "gemv_split_k"])
def test_noalloc_matches_execute_on_two_calls(client, case):
    (big_t, big_a, _), (small_t, small_a, _) = _cases()[case]
    big = client.compile(big_t)
    small = client.compile(small_t)
    # Both calls are queued back to back, the second with the smaller input;
    # the fixed block still holds the first call's contents when the second runs.
    a1, o1, ref1, used1 = _run_noalloc(client, big, big_a)
    a2, o2, ref2, used2 = _run_noalloc(client, small, small_a)
    client.p.hip_check(client.p.lib.pjrtx_hip_synchronize(0))
    assert 0 < used2 <= client.p.lib.pjrtx_noalloc_scratch_bytes()
    for outs, ref in ((o1, ref1), (o2, ref2)):
        for o, r in zip(outs, ref):
            np.testing.assert_array_equal(o.to_numpy(r.dtype, r.shape), r)
    # A third call of the big one after the small one: same bits again.
    o3 = [DeviceArray(client.p, r.nbytes) for r in ref1]
    big.execute_noalloc([a.ptr for a in a1], [o.ptr for o in o3])
    client.p.hip_check(client.p.lib.pjrtx_hip_synchronize(0))
    for o, r in zip(o3, ref1):
        np.testing.assert_array_equal(o.to_numpy(r.dtype, r.shape), r)
    for d in a1 + o1 + a2 + o2 + o3:
        d.free()


def test_noalloc_rejects_a_plan_beyond_the_fixed_block(client):
    # A 128 MiB parameter written in place (not donated) needs a 128 MiB copy.
    b = Builder()
    x = b.param((8192, 4096), "f32")
    u = b.param((1, 4096), "f32")
    z = b.constant(0, "s32")
    exe = client.compile(b.build([b.dynamic_update_slice(x, u, [z, z])]))
    p = client.p
    xd, ud, od = DeviceArray(p, 8192 * 4096 * 4), DeviceArray(p, 4096 * 4), DeviceArray(p, 8192 * 4096 * 4)
    with pytest.raises(PjrtError) as e:
        exe.execute_noalloc([xd.ptr, ud.ptr], [od.ptr])
    assert e.value.code == 8 and "too small" in e.value.message  # RESOURCE_EXHAUSTED
    for d in (xd, ud, od):
        d.free()
    # The entry point keeps working after the refusal.
    (t, arrays, _), _ = _cases()["c2_argmax_f16"]
    exe2 = client.compile(programs.c2_argmax_f16_reductions(8, 4096))
    arrays = [ops.c2_inputs(8, 4096, seed=9)]
    args, outs, ref, _ = _run_noalloc(client, exe2, arrays)
    client.p.hip_check(client.p.lib.pjrtx_hip_synchronize(0))
    for o, r in zip(outs, ref):
        np.testing.assert_array_equal(o.to_numpy(r.dtype, r.shape), r)


def test_noalloc_rejects_bad_arguments(client):
    exe = client.compile(programs.c2_argmax_f16_reductions(8, 4096))
    with pytest.raises(PjrtError) as e:
        exe.execute_noalloc([], [])
    assert e.value.code == 3  # INVALID_ARGUMENT: wrong argument count
