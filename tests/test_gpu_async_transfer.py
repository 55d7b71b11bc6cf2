"""PJRT_Client_CreateBuffersForAsyncHostToDevice and the transfer manager
(the reference's async host transfer: src/runtime/async_host_transfer.zig:
28-60, exercised by src/plugin/api_buffer_test.zig:86-160): device buffers
created empty, filled by chunks sent in any order and of any size (large
chunks through the pinned staging ring), ready once their last chunk is
sent. Reads and executions of a buffer wait for that; an error set on a
buffer, or a manager destroyed before the last chunk, fails them instead."""
import threading

import numpy as np
import pytest

from pjrtx_amd.hlo import Builder
from pjrtx_amd.pjrt import PjrtError

pytestmark = pytest.mark.gpu


def _chunks(nbytes, rng, sizes):
    """Splits [0, nbytes) into consecutive pieces of the given sizes (the
    last takes the rest), returned in a shuffled order."""
    cuts, at = [], 0
    for s in sizes:
        if at >= nbytes:
            break
        cuts.append((at, min(nbytes, at + s)))
        at += s
    if at < nbytes:
        cuts.append((at, nbytes))
    order = rng.permutation(len(cuts))
    return [cuts[i] for i in order]


def test_out_of_order_chunks_are_byte_exact(client):
    rng = np.random.default_rng(0)
    specs = [((1000, 37), "f32"), ((4099,), "bf16"), ((3, 5, 7), "s8"), ((0, 4), "f32"), ((1,), "f64")]
    host = [
        rng.standard_normal((1000, 37)).astype(np.float32),
        rng.integers(0, 1 << 16, 4099, dtype=np.uint16),
        rng.integers(-128, 128, (3, 5, 7), dtype=np.int8),
        np.zeros((0, 4), np.float32),
        np.array([np.pi]),
    ]
    t = client.async_transfer(specs)
    assert t.count() == len(specs)
    assert [t.size(i) for i in range(len(specs))] == [h.nbytes for h in host]
    bufs = [t.buffer(i) for i in range(len(specs))]
    for i, h in enumerate(host):
        raw = h.view(np.uint8).reshape(-1)
        pieces = _chunks(raw.size, rng, [1, 3, 4096, 7, 65536, 12345, 2])
        if not pieces:
            t.transfer(i, b"", 0, True)
            continue
        for k, (a, b) in enumerate(pieces):
            t.transfer(i, raw[a:b].copy(), a, k == len(pieces) - 1)
    t.close()
    for b, h in zip(bufs, host):
        got = b.to_numpy()
        assert got.shape == h.shape
        np.testing.assert_array_equal(got.view(np.uint8), h.view(np.uint8))


def test_large_chunks_through_the_staging_ring(client):
    """96 MiB in two chunks of 72 and 24 MiB, the larger sent second (the
    ring takes chunks of 64 MiB and more)."""
    rng = np.random.default_rng(1)
    n = 96 << 20
    data = rng.integers(0, 256, n, dtype=np.uint8)
    t = client.async_transfer([((n // 4,), "u32")])
    buf = t.buffer(0)
    split = 24 << 20
    t.transfer(0, data[:split], 0, False)
    t.transfer(0, data[split:], split, True)
    got = buf.to_numpy().view(np.uint8)
    assert np.array_equal(got, data)


def test_execute_waits_for_the_last_chunk(client):
    b = Builder("jit_async_exec")
    x = b.param((256, 1024), "f32")
    exe = client.compile(b.build([b.sum(b.multiply(x, x), [1])]))
    rng = np.random.default_rng(2)
    h = rng.standard_normal((256, 1024)).astype(np.float32)
    t = client.async_transfer([((256, 1024), "f32")])
    buf = t.buffer(0)
    raw = h.view(np.uint8).reshape(-1)
    half = raw.size // 2
    t.transfer(0, raw[half:].copy(), half, False)   # second half first
    result = {}

    def run():
        result["out"] = exe.execute_buffers([buf])[0].to_numpy()

    th = threading.Thread(target=run)
    th.start()
    th.join(0.5)
    assert th.is_alive(), "execute must wait for the buffer's last chunk"
    t.transfer(0, raw[:half].copy(), 0, True)
    th.join(60)
    assert not th.is_alive()
    want = (h.astype(np.float64) ** 2).sum(1)
    np.testing.assert_allclose(result["out"], want, rtol=1e-5)


def test_errors(client):
    t = client.async_transfer([((16,), "f32"), ((16,), "f32"), ((8,), "s32")])
    with pytest.raises(PjrtError, match="exceeds buffer size"):
        t.transfer(0, np.zeros(8, np.float32), 40, False)
    with pytest.raises(PjrtError, match="out of range"):
        t.size(3)
    t.transfer(0, np.ones(16, np.float32), 0, True)
    with pytest.raises(PjrtError, match="last chunk"):
        t.transfer(0, np.ones(1, np.float32), 0, True)
    np.testing.assert_array_equal(t.buffer(0).to_numpy(), np.ones(16, np.float32))
    b1 = t.buffer(1)
    t.set_error(1, 9, "producer went away")
    with pytest.raises(PjrtError, match="producer went away"):
        b1.to_numpy()
    b2 = t.buffer(2)
    t.close()   # buffer 2 never received its last chunk
    with pytest.raises(PjrtError, match="destroyed before"):
        b2.to_numpy()


def test_buffer_deleted_mid_transfer(client):
    """The holder deletes a buffer before its last chunk: the next chunk for
    it is refused (no write into memory the buffer gave back), the other
    buffers of the manager still fill."""
    t = client.async_transfer([((1024,), "f32"), ((1024,), "f32")])
    b0, b1 = t.buffer(0), t.buffer(1)
    t.transfer(0, np.ones(512, np.float32), 0, False)
    b0.delete_memory()
    assert b0.is_deleted()
    with pytest.raises(PjrtError, match="was deleted"):
        t.transfer(0, np.ones(512, np.float32), 2048, True)
    with pytest.raises(PjrtError, match="was deleted"):
        b0.to_numpy()
    t.transfer(1, np.full(1024, 3, np.float32), 0, True)
    np.testing.assert_array_equal(b1.to_numpy(), np.full(1024, 3, np.float32))
    t.close()
    b0.delete()
    assert b0.is_deleted()
