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
