"""Numpy restatement of the hot-path ops — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker; the plugin never calls it.

Parity pins (what each function is checked against in tests/test_oracle.py):
  argmax_rows      reference KAT api_test.cc:1016-1055 ({7,5},{1,1}); JAX tie
                   fixture jax_op_suite.py:125,258-269; numpy.argmax (same
                   first-max / first-NaN rule); brute-force pair comparator on
                   small random inputs with planted ties and NaNs.
  f16_row_reduce   reference KAT api_test.cc:930-1014 (sum {3,7}, max {2,4},
                   min {1,3}; bf16 sum {3,7}); closed form on constant rows.
  c1_rowsum        closed forms on special inputs (y <= 0 rows, x = 0 rows);
                   float64 brute force at small size.
Every function names the reference lines whose semantics it restates.
"""
from __future__ import annotations

import numpy as np


# ------------------------------------------------------------- bf16 helpers

def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round to nearest even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


# ------------------------------------------------------------------ argmax

def argmax_pair_better(va: float, ia: int, vb: float, ib: int, kind: str = "max") -> bool:
    """The (value, index) order of JAX's argmax comparator — NaN wins, larger
    (or smaller, for argmin) value wins, ties go to the lower index — which is
    also what the reference's MLX path computes (reference:
    src/backend/mlx_metal/api.cc:4101-4131: max, NaN-aware match, min index)."""
    na, nb = va != va, vb != vb
    if na != nb:
        return na
    if not na and va != vb:
        return va > vb if kind == "max" else va < vb
    return ia < ib


def argmax_rows_bruteforce(values: np.ndarray, kind: str = "max") -> tuple[np.ndarray, np.ndarray]:
    """Pure-python fold with argmax_pair_better over each row (small inputs)."""
    v = np.asarray(values, dtype=np.float64)
    out_v = np.empty(v.shape[0], dtype=np.float64)
    out_i = np.empty(v.shape[0], dtype=np.int64)
    for r in range(v.shape[0]):
        bv, bi = (-np.inf if kind == "max" else np.inf), np.iinfo(np.int64).max
        for i, x in enumerate(v[r]):
            if argmax_pair_better(float(x), i, bv, bi, kind):
                bv, bi = float(x), i
        if v.shape[1] == 0:
            bi = 0
        out_v[r], out_i[r] = bv, bi
    return out_v, out_i


def argmax_rows(values: np.ndarray, kind: str = "max") -> tuple[np.ndarray, np.ndarray]:
    """Vectorized restatement of the same rule (reference: api.cc:4101-4131):
    m = NaN-propagating max of the row; index = lowest position whose value
    equals m, or is NaN when m is NaN. Returns (values as float32, int32)."""
    v = np.asarray(values, dtype=np.float32)
    nan = np.isnan(v)
    any_nan = nan.any(axis=1)
    filled = np.where(nan, -np.inf if kind == "max" else np.inf, v)
    m = filled.max(axis=1) if kind == "max" else filled.min(axis=1)
    match = np.where(any_nan[:, None], nan, filled == m[:, None])
    idx = np.argmax(match, axis=1).astype(np.int32)
    m = np.where(any_nan, np.float32(np.nan), m).astype(np.float32)
    return m, idx


# --------------------------------------------------------- row reductions

def f16_row_reduce(x16: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """jnp.sum / max / min over the last axis of an f16 array. JAX lowers the
    f16 sum as convert->f32, reduce-add, convert->f16; max/min reduce in f16
    (reference reductions: api.cc:3982-4044; KATs api_test.cc:930-1014).
    The sum is accumulated in float64 here and rounded once to f16."""
    x = np.asarray(x16, dtype=np.float16)
    s = x.astype(np.float64).sum(axis=1).astype(np.float32).astype(np.float16)
    return s, x.max(axis=1), x.min(axis=1)


def c2_reference(logits_bf16_bits: np.ndarray):
    """Outputs of the C2 program: argmax (values bf16 bits, indices int32) of
    the bf16 logits and f16 sum/max/min of logits.astype(f16)."""
    vals = bf16_bits_to_f32(logits_bf16_bits)
    mv, mi = argmax_rows(vals)
    s, mx, mn = f16_row_reduce(vals.astype(np.float16))
    return f32_to_bf16_bits(mv), mi, s, mx, mn


# ---------------------------------------------------------------- C1 chain

def c1_rowsum(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """sum(tanh(x*y + 0.5)*x - max(y, 0), axis=1), evaluated in float64 from
    the f32 inputs (the elementwise chain of a `view_elementwise` group,
    reference program_build.zig:10-207, then a reduce_sum node)."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    return (np.tanh(x * y + 0.5) * x - np.maximum(y, 0.0)).sum(axis=1)


# ------------------------------------------------------------ input makers

def c1_inputs(rows: int, cols: int, seed: int = 0):
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    y = np.random.default_rng(seed + 1).uniform(-1, 1, (rows, cols)).astype(np.float32)
    return x, y


def c2_inputs(rows: int, vocab: int, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return f32_to_bf16_bits(rng.standard_normal((rows, vocab), dtype=np.float32))


# ------------------------------------------------------------------ gather

def gather_stablehlo(operand, indices, offset_dims, collapsed_slice_dims, start_index_map, index_vector_dim,
                     slice_sizes, operand_batching_dims=(), start_indices_batching_dims=()):
    """StableHLO gather by its definition, element by element (small inputs).
    Starts are clamped so each slice stays in bounds, the rule the reference's
    gather kernel applies (reference: executable_metal_graph_gather.zig:61-65)."""
    operand = np.asarray(operand)
    indices = np.asarray(indices)
    if index_vector_dim == indices.ndim:
        indices = indices[..., None]
    batch_idx_dims = [d for d in range(indices.ndim) if d != index_vector_dim]
    window = [d for d in range(operand.ndim) if d not in collapsed_slice_dims and d not in operand_batching_dims]
    out_rank = len(batch_idx_dims) + len(offset_dims)
    batch_out = [d for d in range(out_rank) if d not in offset_dims]
    shape = [0] * out_rank
    for o, d in zip(batch_out, batch_idx_dims):
        shape[o] = indices.shape[d]
    for o, d in zip(offset_dims, window):
        shape[o] = slice_sizes[d]
    out = np.zeros(shape, dtype=operand.dtype)
    for oi in np.ndindex(*shape):
        bcoord = [oi[o] for o in batch_out]
        start = [0] * operand.ndim
        for k, od in enumerate(start_index_map):
            sl = list(bcoord)
            sl.insert(index_vector_dim, k)
            start[od] = int(indices[tuple(sl)])
        for ob, ib in zip(operand_batching_dims, start_indices_batching_dims):
            start[ob] = bcoord[batch_idx_dims.index(ib)]
        src = []
        for d in range(operand.ndim):
            s = min(max(start[d], 0), operand.shape[d] - slice_sizes[d])
            src.append(s)
        for o, d in zip(offset_dims, window):
            src[d] += oi[o]
        out[oi] = operand[tuple(src)]
    return out


def gather_rows(table, idx):
    """table[idx] as jnp indexing lowers it: negative indices wrapped once,
    then starts clamped to [0, rows-1] (row-gather special case of
    gather_stablehlo)."""
    idx = np.asarray(idx, dtype=np.int64)
    n = table.shape[0]
    idx = np.where(idx < 0, idx + n, idx)
    return table[np.clip(idx, 0, n - 1)]


# ----------------------------------------------------------------- scatter

def scatter_stablehlo(operand, indices, updates, update_window_dims, inserted_window_dims,
                      scatter_dims_to_operand_dims, index_vector_dim, combiner="add", input_batching_dims=(),
                      scatter_indices_batching_dims=()):
    """StableHLO scatter by its definition, applied sequentially in update
    order (the order of XLA's CPU scatter loop); windows whose start is out of
    bounds are skipped (reference dimension numbers: api.cc:3158-3236)."""
    out = np.array(operand, copy=True)
    indices = np.asarray(indices)
    updates = np.asarray(updates)
    if index_vector_dim == indices.ndim:
        indices = indices[..., None]
    upd_scatter = [d for d in range(updates.ndim) if d not in update_window_dims]
    idx_batch = [d for d in range(indices.ndim) if d != index_vector_dim]
    window = [d for d in range(out.ndim) if d not in inserted_window_dims and d not in input_batching_dims]
    wsize = [1] * out.ndim
    for j, d in enumerate(window):
        wsize[d] = updates.shape[update_window_dims[j]]
    for ui in np.ndindex(*updates.shape):
        sc = [ui[d] for d in upd_scatter]
        start = [0] * out.ndim
        for k, od in enumerate(scatter_dims_to_operand_dims):
            sl = list(sc)
            sl.insert(index_vector_dim, k)
            start[od] = int(indices[tuple(sl)])
        for ob, ib in zip(input_batching_dims, scatter_indices_batching_dims):
            start[ob] = sc[idx_batch.index(ib)]
        if any(start[d] < 0 or start[d] > out.shape[d] - wsize[d] for d in range(out.ndim)):
            continue
        tgt = list(start)
        for j, d in enumerate(window):
            tgt[d] += ui[update_window_dims[j]]
        tgt = tuple(tgt)
        u = updates[ui]
        if combiner == "add":
            out[tgt] = out[tgt] + u
        elif combiner == "set":
            out[tgt] = u
        elif combiner == "maximum":
            out[tgt] = max(out[tgt], u)
        elif combiner == "minimum":
            out[tgt] = min(out[tgt], u)
        elif combiner == "multiply":
            out[tgt] = out[tgt] * u
    return out


def scatter_rows_add(operand, idx, updates):
    """Row scatter-add in update order: np.add.at applies the additions one by
    one in index order, in the operand's dtype (f32 adds for f32, wrapping
    adds for int32) — the sequential loop scatter_stablehlo defines."""
    out = np.array(operand, copy=True)
    idx = np.asarray(idx, dtype=np.int64)
    ok = (idx >= 0) & (idx < operand.shape[0])
    np.add.at(out, idx[ok], updates[ok])
    return out


def scatter_rows_add_bf16_bits(operand_bits, idx, update_bits):
    """Row scatter-add on bf16 bit patterns in update order, each addition
    done as XLA does bf16 arithmetic: widen both to f32, add in f32, round the
    sum to bf16 (nearest-even)."""
    out = bf16_bits_to_f32(np.asarray(operand_bits, np.uint16)).copy()
    upd = bf16_bits_to_f32(np.asarray(update_bits, np.uint16))
    idx = np.asarray(idx, dtype=np.int64)
    for j in np.flatnonzero((idx >= 0) & (idx < out.shape[0])):
        r = idx[j]
        out[r] = bf16_bits_to_f32(f32_to_bf16_bits((out[r] + upd[j]).astype(np.float32)))
    return f32_to_bf16_bits(out)


def scatter_rows_add_int(operand, idx, updates):
    """Integer row scatter-add, vectorized: integer addition is associative,
    so per-row sums in any order (int64, then wrapped) equal the sequential
    loop bit for bit."""
    idx = np.asarray(idx, dtype=np.int64)
    ok = (idx >= 0) & (idx < operand.shape[0])
    order = np.argsort(idx[ok], kind="stable")
    si = idx[ok][order]
    su = updates[ok][order].astype(np.int64)
    out = operand.astype(np.int64)
    if si.size:
        starts = np.flatnonzero(np.r_[True, si[1:] != si[:-1]])
        sums = np.add.reduceat(su, starts, axis=0)
        out[si[starts]] += sums
    return out.astype(operand.dtype)


def scatter_rows_add_f64(operand, idx, updates):
    """The exact (float64) value of the row scatter-add, for bounding the
    rounding of any summation order."""
    out = np.asarray(operand, np.float64).copy()
    idx = np.asarray(idx)
    valid = (idx >= 0) & (idx < out.shape[0])
    np.add.at(out, idx[valid], np.asarray(updates, np.float64)[valid])
    return out


def segment_lengths(idx, rows: int) -> np.ndarray:
    """Number of in-bounds updates per operand row."""
    idx = np.asarray(idx)
    valid = (idx >= 0) & (idx < rows)
    return np.bincount(idx[valid], minlength=rows)


def zipf_indices(n: int, rows: int, seed: int = 0, a: float = 1.1) -> np.ndarray:
    return ((np.random.default_rng(seed).zipf(a, n) - 1) % rows).astype(np.int32)


# --------------------------------------------------------------------- dot

def dot_general_f64(lhs, rhs, lhs_batch=(), rhs_batch=(), lhs_contract=(), rhs_contract=()):
    """dot_general in float64; output dims (batch..., lhs free..., rhs free...)
    (reference: api.cc:1562-1577, 3429-3492)."""
    letters = "abcdefghijklmnopqrstuvwxyz"
    li = [None] * lhs.ndim
    ri = [None] * rhs.ndim
    c = 0
    for lb, rb in zip(lhs_batch, rhs_batch):
        li[lb] = ri[rb] = letters[c]
        c += 1
    for lc, rc in zip(lhs_contract, rhs_contract):
        li[lc] = ri[rc] = letters[c]
        c += 1
    lf, rf = [], []
    for d in range(lhs.ndim):
        if li[d] is None:
            li[d] = letters[c]
            lf.append(letters[c])
            c += 1
    for d in range(rhs.ndim):
        if ri[d] is None:
            ri[d] = letters[c]
            rf.append(letters[c])
            c += 1
    out = "".join(letters[i] for i in range(len(lhs_batch))) + "".join(lf) + "".join(rf)
    return np.einsum(f"{''.join(li)},{''.join(ri)}->{out}", np.asarray(lhs, np.float64), np.asarray(rhs, np.float64))


def attention_bf16(q, k, v, causal=True):
    """The C3 program's arithmetic for one or more heads (bf16 bits in/out):
    scores rounded to bf16, masked, softmax in f32, P rounded to bf16,
    context accumulated in f32 and rounded to bf16."""
    qf, kf, vf = (bf16_bits_to_f32(t).astype(np.float64) for t in (q, k, v))
    s = np.einsum("...qd,...kd->...qk", qf, kf)
    s = bf16_bits_to_f32(f32_to_bf16_bits(s.astype(np.float32))).astype(np.float32)
    if causal:
        L = s.shape[-1]
        mask = np.tril(np.ones((L, L), dtype=bool))
        s = np.where(mask, s, np.float32(-np.inf))
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m, dtype=np.float32)
    p = e / e.sum(axis=-1, keepdims=True, dtype=np.float32)
    p = bf16_bits_to_f32(f32_to_bf16_bits(p.astype(np.float32))).astype(np.float64)
    ctx = np.einsum("...qk,...kd->...qd", p, vf)
    return f32_to_bf16_bits(ctx.astype(np.float32))
