"""GPU parity of the library steps (gather, scatter, dot_general, dynamic
slices, concatenate, pad) through the PJRT C API, against the numpy oracle
and the reference's known answers.

Tolerances: gather / slices / integer scatter bit-exact; f32 scatter-add
bit-exact against the in-order oracle on rows with at most 256 updates (same
f32 additions in the same order) and within 1e-5 of the float64 sum, relative
to the row's scale, on longer rows (folded in 256-update chunks);
bf16 dot_general 2e-2 relative to the output scale (|ref| or the RMS of the
row, whichever is larger: bf16 outputs near zero have no relative precision).
"""
import json
import pathlib

import numpy as np
import pytest

from oracle import ops
from pjrtx_amd import programs
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu
KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())
bf = ops.f32_to_bf16_bits
fb = ops.bf16_bits_to_f32


def run(client, text, *args, dtypes=None):
    return client.compile(text)(*args, dtypes=dtypes)


def assert_bf16_close(got_bits, want, rtol=2e-2):
    got = fb(got_bits).astype(np.float64)
    want = np.asarray(want, np.float64)
    scale = np.sqrt(np.mean(want ** 2, axis=-1, keepdims=True)) + 1e-30
    err = np.abs(got - want) / np.maximum(np.abs(want), scale)
    assert err.max() <= rtol, f"max scaled error {err.max():.3g}"


# ------------------------------------------------------------------ gather

def test_gather_kats(client):
    k = KATS["gather_axis0"]
    b = Builder()
    x = b.param((3, 2), "f32")
    i = b.param((2, 1), "s32")
    t = b.build([b.gather(x, i, [1], [0], [0], 1, [1, 2])])
    (out,) = run(client, t, np.array(k["operand"], np.float32), np.array(k["indices"], np.int32)[:, None])
    np.testing.assert_array_equal(out, k["expected"])
    k = KATS["gather_axis1"]
    b = Builder()
    x = b.param((3, 2), "f32")
    i = b.param((2, 1), "s32")
    t = b.build([b.gather(x, i, [0], [1], [1], 1, [3, 1])])
    (out,) = run(client, t, np.array(k["operand"], np.float32), np.array(k["indices"], np.int32)[:, None])
    np.testing.assert_array_equal(out, k["expected"])
    k = KATS["gather_point"]
    b = Builder()
    x = b.param((3, 2), "f32")
    i = b.param((2, 2), "s32")
    t = b.build([b.gather(x, i, [], [0, 1], [0, 1], 1, [1, 1])])
    (out,) = run(client, t, np.array(k["operand"], np.float32), np.array(k["indices"], np.int32))
    np.testing.assert_array_equal(out, k["expected"])


def test_batched_gather(client):
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    idx = np.array([[2, 0], [1, 2]], np.int32)[..., None]
    b = Builder()
    xp = b.param((2, 3, 4), "f32")
    ip = b.param((2, 2, 1), "s32")
    t = b.build([b.gather(xp, ip, [2], [1], [1], 2, [1, 1, 4], operand_batching_dims=[0],
                          start_indices_batching_dims=[0])])
    (out,) = run(client, t, x, idx)
    np.testing.assert_array_equal(out, ops.gather_stablehlo(x, idx, [2], [1], [1], 2, [1, 1, 4], [0], [0]))


@pytest.mark.parametrize("vocab,dim,batch,seq", [(100, 64, 2, 7), (1000, 4096, 2, 64), (128256, 4096, 8, 2048),
                                                  (300, 6144, 1, 9), (50, 16384, 1, 3)])
def test_embedding_gather(client, vocab, dim, batch, seq):
    rng = np.random.default_rng(vocab)
    table = bf((0.02 * rng.standard_normal((vocab, dim))).astype(np.float32))
    idx = rng.integers(0, vocab, (batch, seq)).astype(np.int32)
    idx.flat[0] = -1  # wrapped to the last row, as jnp indexing does
    idx.flat[-1] = vocab - 1
    (out,) = run(client, programs.c4_embedding_gather(vocab, dim, batch, seq), table, idx, dtypes=["bf16", None])
    np.testing.assert_array_equal(out, ops.gather_rows(table, idx))


@pytest.mark.parametrize("idx_dtype", ["s32", "s64"])
@pytest.mark.parametrize("dim", [64, 5])
def test_gather_folded_index_wrap_edges(client, idx_dtype, dim):
    """JAX's negative-index normalization, folded into the gather, on the
    indices where it matters: -1 and -rows wrap to the last and first rows,
    indices still out of range after the wrap (and the type's extremes) are
    clamped; dim 5 takes the generic gather kernel, 64 the row kernel."""
    vocab, n = 1000, 64
    np_t = np.int32 if idx_dtype == "s32" else np.int64
    info = np.iinfo(np_t)
    rng = np.random.default_rng(dim)
    table = bf((0.02 * rng.standard_normal((vocab, dim))).astype(np.float32))
    idx = rng.integers(-2 * vocab, 2 * vocab, n).astype(np_t)
    idx[:10] = [-1, -vocab, -vocab - 1, -5000, 0, vocab - 1, vocab, vocab + 5, info.min, info.max]
    b = Builder()
    tp = b.param((vocab, dim), "bf16")
    ip = b.param((n,), idx_dtype)
    wrapped = b.select(b.compare("LT", ip, b.scalar_like(0, ip)), b.add(ip, b.scalar_like(vocab, ip)), ip)
    iv = b.broadcast_in_dim(wrapped, (n, 1), [0])
    t = b.build([b.gather(tp, iv, offset_dims=[1], collapsed_slice_dims=[0], start_index_map=[0],
                          index_vector_dim=1, slice_sizes=[1, dim])])
    (out,) = run(client, t, table, idx, dtypes=["bf16", None])
    np.testing.assert_array_equal(out, ops.gather_rows(table, idx))


# ----------------------------------------------------------------- scatter

@pytest.mark.parametrize("mode", ["set", "add"])
def test_scatter_kats(client, mode):
    combiner = "set" if mode == "set" else "add"
    k = KATS["scatter_1d"]
    b = Builder()
    x, i, u = b.param((4,), "f32"), b.param((2, 1), "s32"), b.param((2,), "f32")
    t = b.build([b.scatter(x, i, u, [], [0], [0], 1, combiner)])
    (out,) = run(client, t, np.array(k["operand"], np.float32), np.array(k["indices"], np.int32)[:, None],
                 np.array(k["updates"], np.float32))
    np.testing.assert_array_equal(out, k[mode])
    k = KATS["scatter_point"]
    b = Builder()
    x, i, u = b.param((3, 2), "f32"), b.param((2, 2), "s32"), b.param((2,), "f32")
    t = b.build([b.scatter(x, i, u, [], [0, 1], [0, 1], 1, combiner)])
    (out,) = run(client, t, np.array(k["operand"], np.float32), np.array(k["indices"], np.int32),
                 np.array(k["updates"], np.float32))
    np.testing.assert_array_equal(out, k[mode])
    k = KATS["scatter_window"]
    b = Builder()
    x, i, u = b.param((3, 4), "f32"), b.param((2, 1), "s32"), b.param((2, 2), "f32")
    t = b.build([b.scatter(x, i, u, [1], [0], [0], 1, combiner)])
    (out,) = run(client, t, np.array(k["operand"], np.float32), np.array(k["indices"], np.int32)[:, None],
                 np.array(k["updates"], np.float32))
    np.testing.assert_array_equal(out, k[mode])


def test_scatter_batched_kat(client):
    k = KATS["scatter_batched"]
    b = Builder()
    x, i, u = b.param((2, 3, 4), "f32"), b.param((2, 2, 1), "s32"), b.param((2, 2, 4), "f32")
    t = b.build([b.scatter(x, i, u, [2], [1], [1], 2, "set", input_batching_dims=[0],
                           scatter_indices_batching_dims=[0])])
    (out,) = run(client, t, np.array(k["operand"], np.float32).reshape(2, 3, 4), np.array(k["indices"], np.int32),
                 np.array(k["updates"], np.float32).reshape(2, 2, 4))
    np.testing.assert_array_equal(out.reshape(-1), k["set"])


def _check_scatter_f32(out, x, idx, upd):
    """Every row bit-exact against the sequential fold in update order (the
    loop a StableHLO scatter defines: np.add.at in index order); the float64
    sum bounds both by the recursive-summation error, as a sanity check."""
    rows = x.shape[0]
    seq = ops.scatter_rows_add(x, idx, upd)
    np.testing.assert_array_equal(out, seq)
    exact = ops.scatter_rows_add_f64(x, idx, upd)
    lens = ops.segment_lengths(idx, rows)
    absum = np.abs(x.astype(np.float64)).copy()
    valid = (idx >= 0) & (idx < rows)
    np.add.at(absum, idx[valid], np.abs(upd[valid].astype(np.float64)))
    bound = (lens[:, None] + 1) * 2.0 ** -24 * absum + 1e-30
    assert (np.abs(out.astype(np.float64) - exact) <= bound).all()
    return lens


@pytest.mark.parametrize("rows,dim,n", [(16, 8, 100), (4096, 256, 65536), (64, 20, 40000), (32, 6, 20000)])
def test_scatter_add_f32_in_update_order(client, rows, dim, n):
    # (64, 20): a row of 20 columns folds as two slices (16 + a partial one);
    # (32, 6): 24-byte rows are not 16-byte multiples, every row folds whole.
    rng = np.random.default_rng(rows)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    idx = ops.zipf_indices(n, rows, seed=rows)
    idx[:3] = [-1, rows, rows + 5]  # out of bounds: skipped
    upd = rng.standard_normal((n, dim)).astype(np.float32)
    (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "f32"), x, idx, upd)
    lens = _check_scatter_f32(out, x, idx, upd)
    if n > 1000:
        assert lens.max() > 256  # long segments: the sliced path ran
    (again,) = run(client, programs.c4_scatter_add(rows, dim, n, "f32"), x, idx, upd)
    np.testing.assert_array_equal(again, out)  # deterministic


def test_scatter_add_full_size_zipf(client):
    """C4b / C4c at the BASELINE size: [65536,256] operand, 1,048,576 Zipf(1.1)
    updates (the hottest row takes ~10^5 of them). int32 and f32 bit-exact on
    the whole output against the sequential fold in update order."""
    rows, dim, n = 65536, 256, 1048576
    rng = np.random.default_rng(4)
    idx = ops.zipf_indices(n, rows, seed=4)
    xi = rng.integers(-1000, 1000, (rows, dim)).astype(np.int32)
    ui = rng.integers(-1000, 1000, (n, dim)).astype(np.int32)
    (out_i,) = run(client, programs.c4_scatter_add(rows, dim, n, "s32"), xi, idx, ui)
    np.testing.assert_array_equal(out_i, ops.scatter_rows_add_int(xi, idx, ui))
    xf = np.zeros((rows, dim), np.float32)
    uf = rng.standard_normal((n, dim), dtype=np.float32)
    (out_f,) = run(client, programs.c4_scatter_add(rows, dim, n, "f32"), xf, idx, uf)
    np.testing.assert_array_equal(out_f, ops.scatter_rows_add(xf, idx, uf))
    assert ops.segment_lengths(idx, rows).max() > 90000


def test_scatter_add_f32_many_updates_scanned_early_lists(client):
    """More than 4M updates: the early rows' listing runs with a scan of the
    per-block counts between its count and write kernels (up to 4M the write
    kernel sums them itself). f32 bit-exact in update order; out-of-bounds
    indices skipped."""
    rows, dim, n = 2048, 4, 4_400_000
    rng = np.random.default_rng(31)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    idx = ops.zipf_indices(n, rows, seed=31)
    idx[:4] = [-1, rows, rows + 7, -rows]
    upd = rng.standard_normal((n, dim)).astype(np.float32)
    (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "f32"), x, idx, upd)
    np.testing.assert_array_equal(out, ops.scatter_rows_add(x, idx, upd))
    assert ops.segment_lengths(idx, rows).max() > 256 * 64  # early rows picked


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f64", "s64"])
def test_scatter_add_long_segments_other_types(client, dtype):
    """The sliced in-order fold for 2- and 8-byte elements: bf16/f16 round
    after every add (as the sequential loop in that type does), f64 and s64
    exact in update order."""
    rows, dim, n = 16, 64, 30000
    rng = np.random.default_rng(8)
    idx = ops.zipf_indices(n, rows, seed=8)
    if dtype == "s64":
        x = rng.integers(-10**12, 10**12, (rows, dim)).astype(np.int64)
        u = rng.integers(-10**12, 10**12, (n, dim)).astype(np.int64)
        (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "s64"), x, idx, u)
        np.testing.assert_array_equal(out, ops.scatter_rows_add(x, idx, u))
        return
    if dtype == "f64":
        x = rng.standard_normal((rows, dim))
        u = rng.standard_normal((n, dim))
        (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "f64"), x, idx, u)
        np.testing.assert_array_equal(out, ops.scatter_rows_add(x, idx, u))
        return
    xf = rng.standard_normal((rows, dim)).astype(np.float32)
    uf = (0.01 * rng.standard_normal((n, dim))).astype(np.float32)
    if dtype == "bf16":
        x, u = ops.f32_to_bf16_bits(xf), ops.f32_to_bf16_bits(uf)
        want = ops.scatter_rows_add_bf16_bits(x, idx, u)
    else:
        x, u = xf.astype(np.float16), uf.astype(np.float16)
        want = ops.scatter_rows_add(x, idx, u)
    (out,) = run(client, programs.c4_scatter_add(rows, dim, n, dtype), x, idx, u, dtypes=[dtype, None, dtype])
    np.testing.assert_array_equal(out, want)


@pytest.mark.parametrize("case", ["bf16_add", "f64_add", "f32_set", "f32_one_row", "f32_mostly_dropped"])
def test_scatter_early_rows(client, case):
    """Scatters of at least 65,536 updates fold their longest rows (picked from
    a sample of the keys) while the keys are sorted, and the sorted path skips
    them: other element types and combiners, every update on one row, and a
    majority of dropped (out-of-bounds) updates, whose key fills most of the
    sample but is never picked. Bit-exact against the sequential loop."""
    rows, n = 128, 70000
    rng = np.random.default_rng(21)
    idx = ops.zipf_indices(n, rows, seed=21)
    if case == "f32_one_row":
        idx = np.zeros(n, np.int32)
    if case == "f32_mostly_dropped":
        drop = rng.random(n) < 0.6
        idx = np.where(drop, rows + 7, idx).astype(np.int32)
    if case == "bf16_add":
        dim = 64
        x = ops.f32_to_bf16_bits(rng.standard_normal((rows, dim)).astype(np.float32))
        u = ops.f32_to_bf16_bits((0.01 * rng.standard_normal((n, dim))).astype(np.float32))
        (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "bf16"), x, idx, u, dtypes=["bf16", None, "bf16"])
        np.testing.assert_array_equal(out, ops.scatter_rows_add_bf16_bits(x, idx, u))
    elif case == "f64_add":
        dim = 16
        x = rng.standard_normal((rows, dim))
        u = rng.standard_normal((n, dim))
        (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "f64"), x, idx, u)
        np.testing.assert_array_equal(out, ops.scatter_rows_add(x, idx, u))
    elif case == "f32_set":
        dim = 32
        x = rng.standard_normal((rows, dim)).astype(np.float32)
        u = rng.standard_normal((n, dim)).astype(np.float32)
        (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "f32", combiner="set"), x, idx, u)
        want = x.copy()
        rev = idx[::-1]
        r, first = np.unique(rev, return_index=True)
        want[r] = u[n - 1 - first]
        np.testing.assert_array_equal(out, want)
    else:
        dim = 32
        x = rng.standard_normal((rows, dim)).astype(np.float32)
        u = rng.standard_normal((n, dim)).astype(np.float32)
        (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "f32"), x, idx, u)
        np.testing.assert_array_equal(out, ops.scatter_rows_add(x, idx, u))


@pytest.mark.parametrize("dtype,combiner", [("s32", "maximum"), ("s32", "minimum"), ("u32", "add"),
                                            ("s64", "maximum")])
def test_scatter_integer_long_segments_any_order_ops(client, dtype, combiner):
    """Integer add / max / min are exact in any order: long segments fold in
    parallel chunks merged with atomics; bit-exact against the sequential loop."""
    rows, dim, n = 64, 128, 60000
    rng = np.random.default_rng(14)
    npt = {"s32": np.int32, "u32": np.uint32, "s64": np.int64}[dtype]
    lo, hi = (0, 2**31) if dtype == "u32" else (-10**9, 10**9)
    x = rng.integers(lo, hi, (rows, dim)).astype(npt)
    u = rng.integers(lo, hi, (n, dim)).astype(npt)
    idx = ops.zipf_indices(n, rows, seed=14)
    (out,) = run(client, programs.c4_scatter_add(rows, dim, n, dtype, combiner=combiner), x, idx, u)
    want = x.copy()
    if combiner == "add":
        np.add.at(want, idx, u)
    elif combiner == "maximum":
        np.maximum.at(want, idx, u)
    else:
        np.minimum.at(want, idx, u)
    np.testing.assert_array_equal(out, want)
    assert ops.segment_lengths(idx, rows).max() > 1024  # several chunks per hot row


def test_scatter_add_in_place_on_donated_operand(client):
    """The operand donated (the result reuses its memory): hot slices and bulk
    rows read each element before writing it; rows without updates stay."""
    rows, dim, n = 512, 64, 50000
    b = Builder()
    x = b.param((rows, dim), "f32", donate=True)
    i = b.param((n,), "s32")
    u = b.param((n, dim), "f32")
    iv = b.broadcast_in_dim(i, (n, 1), [0])
    exe = client.compile(b.build([b.scatter(x, iv, u, [1], [0], [0], 1, "add")]))
    rng = np.random.default_rng(12)
    xv = rng.standard_normal((rows, dim)).astype(np.float32)
    idx = ops.zipf_indices(n, rows, seed=12)
    uv = rng.standard_normal((n, dim)).astype(np.float32)
    bx = client.buffer(xv)
    (out,) = exe.execute_buffers([bx, client.buffer(idx), client.buffer(uv)])
    np.testing.assert_array_equal(out.to_numpy(), ops.scatter_rows_add(xv, idx, uv))
    assert ops.segment_lengths(idx, rows).max() > 256


@pytest.mark.parametrize("combiner", ["set", "maximum", "minimum"])
def test_scatter_long_segments_order_free_ops(client, combiner):
    """Segments of ~600 updates (three chunks): set keeps the last update in
    update order; max/min are exact in any grouping."""
    rows, dim, n = 8, 64, 5000
    rng = np.random.default_rng(6)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    idx = rng.integers(0, rows, n).astype(np.int32)
    upd = rng.standard_normal((n, dim)).astype(np.float32)
    (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "f32", combiner=combiner), x, idx, upd)
    want = x.copy()
    for j in range(n):
        r = idx[j]
        want[r] = upd[j] if combiner == "set" else (np.maximum(want[r], upd[j]) if combiner == "maximum"
                                                   else np.minimum(want[r], upd[j]))
    np.testing.assert_array_equal(out, want)


def test_scatter_set_last_update_wins(client):
    rows, dim, n = 64, 16, 4096
    rng = np.random.default_rng(5)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    idx = rng.integers(0, rows, n).astype(np.int32)
    upd = rng.standard_normal((n, dim)).astype(np.float32)
    (out,) = run(client, programs.c4_scatter_add(rows, dim, n, "f32", combiner="set"), x, idx, upd)
    want = x.copy()
    for j in range(n):
        want[idx[j]] = upd[j]
    np.testing.assert_array_equal(out, want)


# ------------------------------------------------------------- dot_general

@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
def test_dot_kat(client, dtype):
    k = KATS["dot_2x2"]
    b = Builder()
    x, y = b.param((2, 2), dtype), b.param((2, 2), dtype)
    t = b.build([b.dot_general(x, y, contract=((1,), (0,)))])
    lhs, rhs = np.array(k["lhs"], np.float32), np.array(k["rhs"], np.float32)
    if dtype == "bf16":
        out = run(client, t, bf(lhs), bf(rhs), dtypes=["bf16", "bf16"])[0]
        out = fb(out)
    else:
        npd = np.float16 if dtype == "f16" else np.float32
        out = run(client, t, lhs.astype(npd), rhs.astype(npd))[0]
    np.testing.assert_array_equal(out.astype(np.float32), k["expected"])


@pytest.mark.parametrize("shape", [
    ("mk,kn", (64, 128), (128, 96)),            # NN, ragged N
    ("mk,nk", (200, 64), (136, 64)),            # NT (rhs contract last)
    ("bmk,bkn", (3, 130, 72), (3, 72, 40)),     # batched NN, ragged everything
    ("bmk,bnk", (4, 256, 128), (4, 256, 128)),  # batched NT (attention scores)
    ("mk,kn", (1, 2048), (2048, 2048)),         # GEMV (decode)
    ("mk,kn", (4, 512), (512, 1000)),           # GEMV M=4
    ("mk,nk", (1, 512), (300, 512)),            # GEMV K-major
    ("mk,kn", (1, 5632), (5632, 2048)),         # GEMV long K (FFN down), many K chunks
    ("mk,kn", (1, 2048), (2048, 32000)),        # GEMV wide N (lm_head)
    ("mk,kn", (3, 200), (200, 1030)),           # GEMV M=3, K not a chunk multiple, ragged N
    ("mk,kn", (8, 64), (64, 24)),               # GEMV M=8, tiny N, one K chunk
    ("bmk,bnk", (16, 1, 128), (16, 640, 128)),  # batched K-major GEMV (decode scores)
    ("bmk,bkn", (16, 1, 640), (16, 640, 128)),  # batched N-major GEMV (decode context)
    ("bmk,bnk", (2, 5, 2048), (2, 300, 2048)),  # batched K-major, M=5, long K
    ("mk,nk", (2, 8), (40, 8)),                 # K-major with K = 8
])
def test_dot_bf16_random(client, shape):
    spec, sa, sb = shape
    rng = np.random.default_rng(sum(sa) + sum(sb))
    a = bf(rng.standard_normal(sa).astype(np.float32))
    b_ = bf(rng.standard_normal(sb).astype(np.float32))
    lhs_s, rhs_s = spec.split(",")
    lb = tuple(i for i, c in enumerate(lhs_s) if c == "b")
    rb = tuple(i for i, c in enumerate(rhs_s) if c == "b")
    lc = (lhs_s.index("k"),)
    rc = (rhs_s.index("k"),)
    bld = Builder()
    x, y = bld.param(sa, "bf16"), bld.param(sb, "bf16")
    t = bld.build([bld.dot_general(x, y, batch=(lb, rb), contract=(lc, rc))])
    (out,) = run(client, t, a, b_, dtypes=["bf16", "bf16"])
    want = ops.dot_general_f64(fb(a), fb(b_), lb, rb, lc, rc)
    assert out.shape == want.shape
    assert_bf16_close(out, want)


def test_dot_f32_fallback_and_rank3_rank2(client):
    # jax_op_suite attention_scores_rhs_contract_last / attention_values_rhs_second_last
    q = ((np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5) - 11) / 7)
    kc = ((np.arange(2 * 6 * 5, dtype=np.float32).reshape(2, 6, 5) - 9) / 11)
    b = Builder()
    x, y = b.param(q.shape, "f32"), b.param(kc.shape, "f32")
    t = b.build([b.dot_general(x, y, batch=((0,), (0,)), contract=((3,), (2,)))])
    (out,) = run(client, t, q, kc)
    np.testing.assert_allclose(out, ops.dot_general_f64(q, kc, (0,), (0,), (3,), (2,)), rtol=1e-5, atol=1e-6)


def test_matmul_8192_sampled_rows(client):
    """C3d at full size on the default route, the hand-written MFMA kernel
    (gemm_nt_256, B read N-contiguous); sampled rows against float64, both
    ends and tile boundaries."""
    n = 8192
    rng = np.random.default_rng(9)
    a = bf((rng.standard_normal((n, n), dtype=np.float32) / np.float32(np.sqrt(n))))
    b_ = bf((rng.standard_normal((n, n), dtype=np.float32) / np.float32(np.sqrt(n))))
    (out,) = run(client, programs.c3_matmul(n, n, n), a, b_, dtypes=["bf16", "bf16"])
    rows = np.array([0, 1, 255, 256, 4095, 4096, 8190, 8191])
    want = fb(a[rows]).astype(np.float64) @ fb(b_).astype(np.float64)
    assert_bf16_close(out[rows], want)


def test_matmul_8192_library_route_sampled_rows(client, monkeypatch):
    """C3d at full size on the opt-in hipBLASLt route (PJRTX_BLASLT=1); rows
    sampled for the float64 reference."""
    monkeypatch.setenv("PJRTX_BLASLT", "1")
    n = 8192
    rng = np.random.default_rng(8)
    a = bf((rng.standard_normal((n, n), dtype=np.float32) / np.float32(np.sqrt(n))))
    b_ = bf((rng.standard_normal((n, n), dtype=np.float32) / np.float32(np.sqrt(n))))
    (out,) = run(client, programs.c3_matmul(n, n, n), a, b_, dtypes=["bf16", "bf16"])
    rows = np.array([0, 1, 127, 128, 4095, 8191])
    want = fb(a[rows]).astype(np.float64) @ fb(b_).astype(np.float64)
    assert_bf16_close(out[rows], want)


def test_attention_full_size_sampled_heads(client):
    """C3 attention at [8,32,2048,128] (causal, bf16) through the fused
    kernel; four (batch, head) pairs compared in full (every query tile, the
    first and the last included) against the oracle's bf16 arithmetic."""
    B, H, S, D = 8, 32, 2048, 128
    from bench import randn_bits
    q = randn_bits((B, H, S, D), 21, 1 / np.sqrt(D))
    k = randn_bits((B, H, S, D), 22, 1 / np.sqrt(D))
    v = randn_bits((B, H, S, D), 23, 1 / np.sqrt(D))
    exe = client.compile(programs.c3_attention(B, H, S, D))
    steps = json.loads(exe.optimized_program())["steps"]
    assert any("attention" in str(s_.get("library", "")) for s_ in steps)
    (out,) = exe(q, k, v, dtypes=["bf16"] * 3)
    for b_, h in [(0, 0), (3, 17), (5, 31), (7, 31)]:
        sl = (slice(b_, b_ + 1), slice(h, h + 1))
        want = fb(ops.attention_bf16(q[sl], k[sl], v[sl], causal=True))
        assert_bf16_close(out[sl], want)


@pytest.mark.parametrize("b,h,s,d", [(1, 2, 128, 64), (2, 2, 512, 128)])
def test_attention_small(client, b, h, s, d):
    rng = np.random.default_rng(s)
    q, k, v = (bf((rng.standard_normal((b, h, s, d)) / np.sqrt(d)).astype(np.float32)) for _ in range(3))
    (out,) = run(client, programs.c3_attention(b, h, s, d), q, k, v, dtypes=["bf16"] * 3)
    want = fb(ops.attention_bf16(q, k, v, causal=True))
    assert_bf16_close(out, want)


# ---------------------------------------------- dynamic slices, concat, pad

def test_dynamic_slice_and_update_clamped(client):
    x = np.arange(3 * 4, dtype=np.float32).reshape(3, 4)
    b = Builder()
    xp = b.param((3, 4), "f32")
    i0, i1 = b.param((), "s32"), b.param((), "s32")
    up = b.param((2, 2), "f32")
    ds = b.dynamic_slice(xp, [i0, i1], [2, 2])
    dus = b.dynamic_update_slice(xp, up, [i0, i1])
    exe = client.compile(b.build([ds, dus]))
    u = np.array([[100, 101], [102, 103]], np.float32)
    for s0, s1 in [(0, 0), (1, 2), (5, -3), (-1, 3)]:
        got_ds, got_dus = exe(x, np.array(s0, np.int32), np.array(s1, np.int32), u)
        c0, c1 = min(max(s0, 0), 1), min(max(s1, 0), 2)  # StableHLO clamps starts
        np.testing.assert_array_equal(got_ds, x[c0:c0 + 2, c1:c1 + 2])
        want = x.copy()
        want[c0:c0 + 2, c1:c1 + 2] = u
        np.testing.assert_array_equal(got_dus, want)


def test_kv_cache_update_in_place_chain(client):
    # cache' = DUS(DUS(cache + 0, k0, p), k1, p+1): the second update writes in place.
    L, H, D = 16, 2, 8
    b = Builder()
    cache = b.param((1, L, H, D), "bf16")
    k0 = b.param((1, 1, H, D), "bf16")
    pos = b.param((), "s32")
    z = b.constant(0, "s32")
    c1 = b.dynamic_update_slice(b.add(cache, b.scalar_like(0.0, cache)), k0, [z, pos, z, z])
    p1 = b.add(pos, b.constant(1, "s32"))
    c2 = b.dynamic_update_slice(c1, k0, [z, p1, z, z])
    exe = client.compile(b.build([c2]))
    plan = json.loads(exe.optimized_program())
    assert any(s.get("in_place") for s in plan["steps"]), plan
    rng = np.random.default_rng(0)
    cv = bf(rng.standard_normal((1, L, H, D)).astype(np.float32))
    kv = bf(rng.standard_normal((1, 1, H, D)).astype(np.float32))
    (out,) = exe(cv, kv, np.array(5, np.int32), dtypes=["bf16", "bf16", None])
    want = cv.copy()
    want[:, 5] = kv[:, 0]
    want[:, 6] = kv[:, 0]
    np.testing.assert_array_equal(out, want)


def test_concatenate_and_pad(client):
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    c = np.arange(8, dtype=np.float32).reshape(2, 4) + 100
    b = Builder()
    ap, cp = b.param((2, 3), "f32"), b.param((2, 4), "f32")
    cat = b.concatenate([ap, cp], 1)
    pad = b.pad(ap, b.constant(-1.0, "f32"), [1, 0], [0, 2], [1, 1])
    got_cat, got_pad = run(client, b.build([cat, pad]), a, c)
    np.testing.assert_array_equal(got_cat, np.concatenate([a, c], axis=1))
    want = np.full((4, 7), -1.0, np.float32)
    want[1::2, 0:5:2] = a
    np.testing.assert_array_equal(got_pad, want)


_BIG_GEMM_SHAPES = [
    ("bmk,bkn", (2, 300, 200), (2, 200, 520), "bf16", None),   # NN (B read N-contiguous), ragged M / N / K tail
    ("bmk,bnk", (3, 512, 136), (3, 264, 136), "bf16", None),   # NT, ragged N, K not a multiple of 64
    ("mk,kn", (256, 64), (64, 256), "f16", None),              # exactly one tile
    ("bmk,bnk", (2, 260, 72), (2, 300, 72), "bf16", "f32"),    # f32 output
    ("bmk,bkn", (2, 264, 72), (2, 72, 300), "bf16", None),     # NN with N % 8 != 0: transposed copy of B
    ("mk,kn", (520, 136), (136, 264), "bf16", "f32"),          # NN, f32 output, ragged M / N, K tail
    ("bmk,bkn", (2, 256, 128), (2, 128, 512), "f16", None),    # NN, f16, whole tiles
]


@pytest.mark.parametrize("shape", _BIG_GEMM_SHAPES)
def test_dot_large_tile_kernel(client, shape, monkeypatch):
    """The 256 x 256 tile kernel on shapes with ragged edges; the environment
    lowers its tile-count threshold so that these small problems take it."""
    monkeypatch.setenv("PJRTX_BIG_GEMM_MIN_TILES", "1")
    spec, sa, sb, dt, out_dt = shape
    rng = np.random.default_rng(sum(sa) + sum(sb))
    if dt == "bf16":
        to, fr = bf, fb
    else:
        to = lambda x: x.astype(np.float16).view(np.uint16)  # noqa: E731
        fr = lambda b: b.view(np.float16).astype(np.float32)  # noqa: E731
    a = to(rng.standard_normal(sa).astype(np.float32))
    b_ = to(rng.standard_normal(sb).astype(np.float32))
    ls, rs = spec.split(",")
    lb = tuple(i for i, c in enumerate(ls) if c == "b")
    rb = tuple(i for i, c in enumerate(rs) if c == "b")
    lc, rc = (ls.index("k"),), (rs.index("k"),)
    bld = Builder()
    x, y = bld.param(sa, dt), bld.param(sb, dt)
    t = bld.build([bld.dot_general(x, y, batch=(lb, rb), contract=(lc, rc), out_dtype=out_dt)])
    (out,) = run(client, t, a, b_, dtypes=[dt, dt])
    want = ops.dot_general_f64(fr(a), fr(b_), lb, rb, lc, rc)
    assert out.shape == want.shape
    if out_dt == "f32":
        np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())
    elif dt == "bf16":
        assert_bf16_close(out, want)
    else:
        got = fr(out).astype(np.float64)
        scale = np.sqrt(np.mean(want ** 2, axis=-1, keepdims=True))
        assert (np.abs(got - want) / np.maximum(np.abs(want), scale)).max() <= 2e-2


_LIBRARY_GEMM_SHAPES = [
    ("mk,kn", (4096, 512), (512, 4096), None),          # N-contiguous B
    ("mk,nk", (4096, 384), (4096, 384), None),          # K-contiguous B
    ("bmk,bkn", (4, 2048, 256), (4, 256, 2048), None),  # strided batches
    ("mk,kn", (4096, 256), (256, 4096), "f32"),         # f32 output
]


@pytest.mark.parametrize("shape", _LIBRARY_GEMM_SHAPES)
def test_dot_library_gemm_matches_own_kernels(client, shape, monkeypatch):
    """Plain products that fill the GPU on the opt-in hipBLASLt route
    (PJRTX_BLASLT=1): same tolerance to the float64 product as the own MFMA
    kernels (the default route), and the same bits on every call."""
    spec, sa, sb, out_dt = shape
    rng = np.random.default_rng(sum(sa) + sum(sb))
    a = bf(rng.standard_normal(sa).astype(np.float32))
    b_ = bf(rng.standard_normal(sb).astype(np.float32))
    ls, rs = spec.split(",")
    lb = tuple(i for i, c in enumerate(ls) if c == "b")
    rb = tuple(i for i, c in enumerate(rs) if c == "b")
    lc, rc = (ls.index("k"),), (rs.index("k"),)
    bld = Builder()
    x, y = bld.param(sa, "bf16"), bld.param(sb, "bf16")
    t = bld.build([bld.dot_general(x, y, batch=(lb, rb), contract=(lc, rc), out_dtype=out_dt)])
    want = ops.dot_general_f64(fb(a), fb(b_), lb, rb, lc, rc)
    monkeypatch.setenv("PJRTX_BLASLT", "1")
    exe = client.compile(t)
    (lib1,) = exe(a, b_, dtypes=["bf16", "bf16"])
    (lib2,) = exe(a, b_, dtypes=["bf16", "bf16"])
    np.testing.assert_array_equal(lib1, lib2)
    monkeypatch.setenv("PJRTX_BLASLT", "0")
    (own,) = client.compile(t)(a, b_, dtypes=["bf16", "bf16"])
    for out in (lib1, own):
        if out_dt == "f32":
            np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())
        else:
            assert_bf16_close(out, want)
