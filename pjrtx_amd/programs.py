"""The BASELINE workloads as StableHLO programs (what ``jax.jit`` lowers them
to), parameterized by shape so that tests can run the same program small.

C1  f32 elementwise chain + row reduction:
    out = sum(tanh(x*y + 0.5)*x - max(y, 0), axis=1)
C2  two-output max/index argmax (ZML style) over bf16 logits, plus f16
    sum / max / min of the logits cast to f16.
"""
from __future__ import annotations

from .hlo import Builder


def c1_elementwise_rowsum(rows: int = 4096, cols: int = 4096) -> str:
    b = Builder("jit_c1")
    x = b.param((rows, cols), "f32")
    y = b.param((rows, cols), "f32")
    t = b.multiply(x, y)
    t = b.add(t, b.scalar_like(0.5, t))
    t = b.tanh(t)
    t = b.multiply(t, x)
    r = b.maximum(y, b.scalar_like(0.0, y))
    t = b.subtract(t, r)
    out = b.sum(t, [1])
    return b.build([out])


def stream_negate(rows: int = 8192, cols: int = 4096) -> str:
    """out = -x over f32 [rows, cols]: a plain streaming kernel that reads and
    writes exactly rows*cols*4 bytes each. Used to calibrate the hardware
    byte counters (FETCH_SIZE / WRITE_SIZE) against a known size."""
    b = Builder("jit_stream_negate")
    x = b.param((rows, cols), "f32")
    return b.build([b.negate(x)])


def c2_argmax_f16_reductions(rows: int = 64, vocab: int = 128256) -> str:
    b = Builder("jit_c2")
    logits = b.param((rows, vocab), "bf16")
    vals, idx = b.argmax(logits, 1, "s32")
    h = b.convert(logits, "f16")
    s = b.sum(h, [1])
    mx = b.max(h, [1])
    mn = b.min(h, [1])
    return b.build([vals, idx, s, mx, mn])


def c2_argmax_only(rows: int, vocab: int, dtype: str = "bf16") -> str:
    b = Builder("jit_argmax")
    logits = b.param((rows, vocab), dtype)
    vals, idx = b.argmax(logits, 1, "s32")
    return b.build([vals, idx])


def c3_attention(batch: int = 8, heads: int = 32, seq: int = 2048, head_dim: int = 128, causal: bool = True,
                 dtype: str = "bf16") -> str:
    """scores = einsum('bhqd,bhkd->bhqk', q, k); causal mask via select;
    softmax in f32; context = einsum('bhqk,bhkd->bhqd', p, v) -> bf16."""
    b = Builder("jit_c3_attention")
    shp = (batch, heads, seq, head_dim)
    q, k, v = b.param(shp, dtype), b.param(shp, dtype), b.param(shp, dtype)
    s = b.dot_general(q, k, batch=((0, 1), (0, 1)), contract=((3,), (3,)))          # [B,H,S,S] bf16
    if causal:
        row = b.iota((seq, seq), 0)
        col = b.iota((seq, seq), 1)
        keep = b.broadcast_in_dim(b.compare("GE", row, col), s.shape, [2, 3])
        s = b.select(keep, s, b.scalar_like(float("-inf"), s))
    sf = b.convert(s, "f32")
    m = b.max(sf, [3])
    e = b.exp(b.subtract(sf, b.broadcast_in_dim(m, sf.shape, [0, 1, 2])))
    z = b.sum(e, [3])
    p = b.convert(b.divide(e, b.broadcast_in_dim(z, sf.shape, [0, 1, 2])), dtype)
    ctx = b.dot_general(p, v, batch=((0, 1), (0, 1)), contract=((3,), (2,)))        # [B,H,S,D]
    return b.build([ctx])


def c3_scores(batch: int, heads: int, seq: int, head_dim: int) -> str:
    b = Builder("jit_c3_scores")
    shp = (batch, heads, seq, head_dim)
    q, k = b.param(shp, "bf16"), b.param(shp, "bf16")
    return b.build([b.dot_general(q, k, batch=((0, 1), (0, 1)), contract=((3,), (3,)))])


def c3_context(batch: int, heads: int, seq: int, head_dim: int) -> str:
    b = Builder("jit_c3_context")
    p = b.param((batch, heads, seq, seq), "bf16")
    v = b.param((batch, heads, seq, head_dim), "bf16")
    return b.build([b.dot_general(p, v, batch=((0, 1), (0, 1)), contract=((3,), (2,)))])


def c3_matmul(m: int = 8192, k: int = 8192, n: int = 8192, dtype: str = "bf16") -> str:
    b = Builder("jit_c3_matmul")
    x, y = b.param((m, k), dtype), b.param((k, n), dtype)
    return b.build([b.dot_general(x, y, contract=((1,), (0,)))])


def c4_embedding_gather(vocab: int = 128256, dim: int = 4096, batch: int = 8, seq: int = 2048) -> str:
    """table[idx] as jnp indexing lowers it: negative indices wrapped, index
    vector dim appended, gather of [1, dim] slices."""
    b = Builder("jit_c4_gather")
    table = b.param((vocab, dim), "bf16")
    idx = b.param((batch, seq), "s32")
    neg = b.compare("LT", idx, b.scalar_like(0, idx))
    wrapped = b.select(neg, b.add(idx, b.scalar_like(vocab, idx)), idx)
    iv = b.broadcast_in_dim(wrapped, (batch, seq, 1), [0, 1])
    out = b.gather(table, iv, offset_dims=[2], collapsed_slice_dims=[0], start_index_map=[0], index_vector_dim=2,
                   slice_sizes=[1, dim])
    return b.build([out])


def c4_scatter_add(rows: int = 65536, dim: int = 256, n: int = 1048576, dtype: str = "f32",
                   combiner: str = "add") -> str:
    """operand.at[idx].add(updates) with idx [n] and updates [n, dim]."""
    b = Builder("jit_c4_scatter")
    x = b.param((rows, dim), dtype)
    idx = b.param((n,), "s32")
    upd = b.param((n, dim), dtype)
    iv = b.broadcast_in_dim(idx, (n, 1), [0])
    out = b.scatter(x, iv, upd, update_window_dims=[1], inserted_window_dims=[0], scatter_dims_to_operand_dims=[0],
                    index_vector_dim=1, combiner=combiner)
    return b.build([out])


def topk_logits(rows: int = 64, vocab: int = 128256, k: int = 50) -> str:
    """lax.top_k over bf16 logits (sampling's candidate set): chlo.top_k."""
    b = Builder("jit_topk")
    logits = b.param((rows, vocab), "bf16")
    v, i = b.top_k(logits, k)
    return b.build([v, i])
