"""Host-to-device uploads: the direct path (small arrays) and the pinned
staging ring on its own copy stream (arrays of 64 MiB and more) return the
host bytes exactly, and an upload into a block that queued device work has
just released waits for that work (allocation is ordered on the compute
stream, the staged copy runs on another)."""
import numpy as np
import pytest

from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,dtype", [((1000,), np.float32), ((3, 5, 7), np.int8), ((4096, 4096), np.float32),
                                         ((40 * 2**20 + 3,), np.int16), ((70 * 2**20 + 1,), np.uint8),
                                         ((9 * 2**20 + 5,), np.float64)])
def test_upload_roundtrip(client, shape, dtype):
    rng = np.random.default_rng(1)
    a = rng.integers(-100, 100, shape).astype(dtype) if np.dtype(dtype).kind in "iu" else \
        rng.standard_normal(shape).astype(dtype)
    b = client.buffer(a)
    np.testing.assert_array_equal(b.to_numpy(), a)


def test_staged_upload_waits_for_queued_work(client):
    n = 64 * 2**20  # 256 MiB of f32: staged
    rng = np.random.default_rng(2)
    x = rng.standard_normal(n, dtype=np.float32)
    bld = Builder("jit_sq")
    p = bld.param((n,), "f32")
    r = bld.sum(bld.multiply(p, p), [0])
    exe = client.compile(bld.build([r]))
    want = float(np.sum(x.astype(np.float64) ** 2))
    xb = client.buffer(x)
    for _ in range(3):
        out = exe.execute_buffers([xb])[0]   # queued, not awaited
        xb.delete()                          # its block returns to the allocator
        y = rng.standard_normal(n, dtype=np.float32)
        xb = client.buffer(y)                # may reuse that block
        assert abs(float(out.to_numpy()) - want) <= 1e-4 * want
        np.testing.assert_array_equal(xb.to_numpy(), y)
        x, want = y, float(np.sum(y.astype(np.float64) ** 2))


def test_large_readback_through_pinned_ring(client):
    """Readbacks of 64 MiB and more go device -> pinned ring -> caller memory
    (chunks of 32 MiB, the DMA of the next chunks overlapping the host copy
    of the current one): byte-exact, including a ragged last chunk, and after
    queued device work that produces the source."""
    import time
    rng = np.random.default_rng(11)
    n = (100 << 20) + 4096 + 12          # 3 whole chunks and a ragged tail
    host = rng.integers(0, 256, n, dtype=np.uint8)
    buf = client.buffer(host)
    t0 = time.perf_counter()
    back = buf.to_numpy()
    el = time.perf_counter() - t0
    print(f"staged readback of {n >> 20} MiB: {n / el / 1e9:.1f} GB/s")
    assert np.array_equal(back, host)
    # The source produced by a kernel still queued when the readback starts.
    from pjrtx_amd.hlo import Builder
    b = Builder("jit_neg_u8")
    x = b.param((n,), "u8")
    exe = client.compile(b.build([b.xor(x, b.scalar_like(255, x))]))
    (y,) = exe.execute_buffers([buf])
    assert np.array_equal(y.to_numpy(), host ^ np.uint8(255))
