"""Numpy restatements of the widened frontend ops — TEST INFRASTRUCTURE ONLY.

Only tests/ use this module, as the checker; the plugin never calls it.

  reduce_precision  stablehlo.reduce_precision on the element type's own bits
                    (mantissa rounded to nearest even, then exponent clamped:
                    overflow to +-inf, underflow to +-0; NaN kept when
                    mantissa_bits > 0). The reference imports the op
                    (plan_instruction.zig:85, stablehlo_import_tests.zig:278,
                    e8m23 on f32, an identity) and executes it as a copy of its
                    operand (execution_node_structural.zig:34); this restates
                    the StableHLO definition, which equals the copy for a
                    format as wide as the type. Pins (tests/test_oracle_frontend.py):
                    e8m7 on f32 equals round-to-nearest-even bf16; e5m10 on f32
                    equals numpy's float16 conversion over the f16 normal range;
                    e8m23 is the identity; overflow, underflow and NaN cases.
  reduce_window     brute force over every window position in row-major
                    order from the init value; padded positions contribute the
                    init value (StableHLO). The reference computes sum or max
                    over a strided view of the input padded with 0 / -inf
                    (api.cc:4324-4437), the same for init 0 / -inf. Pins: the
                    reference's import case (window 2, padding [1, 0],
                    stablehlo_import_tests.zig:173-207); the cumulative-sum
                    closed form of a stride-1 window sum; numpy's
                    sliding_window_view max.
"""
from __future__ import annotations

import itertools

import numpy as np

_FORMATS = {  # dtype: (unsigned view, exponent bits, mantissa bits)
    "f32": (np.uint32, 8, 23),
    "f64": (np.uint64, 11, 52),
    "f16": (np.uint16, 5, 10),
    "bf16": (np.uint16, 8, 7),
}


def reduce_precision_bits(bits: np.ndarray, dtype: str, exponent_bits: int, mantissa_bits: int) -> np.ndarray:
    """The op on raw bit patterns of `dtype` (bf16 / f16 / f32 / f64)."""
    ut, E, Mn = _FORMATS[dtype]
    W = 1 + E + Mn
    u = np.asarray(bits).astype(ut)
    one = ut(1)
    sign = ut(one << ut(W - 1))
    expm = ut(((one << ut(E)) - one) << ut(Mn))
    manm = ut((one << ut(Mn)) - one)
    nan = ((u & expm) == expm) & ((u & manm) != 0)
    x = u.copy()
    with np.errstate(over="ignore"):
        if mantissa_bits < Mn:
            sh = ut(Mn - mantissa_bits)
            last = ut(one << sh)
            bias = ut((last >> one) - one) + ((u & last) >> sh)
            u = ((u + bias) & ut(~ut(last - one))).astype(ut)
        if exponent_bits < E:
            b = ut((one << ut(E - 1)) - one)
            rb = ut((one << ut(exponent_bits - 1)) - one)
            xe = u & expm
            over = xe > ut(ut(b + rb) << ut(Mn))
            under = xe <= ut(ut(b - rb) << ut(Mn))
            sz = u & sign
            u = np.where(over, sz | expm, np.where(under, sz, u)).astype(ut)
    if mantissa_bits > 0:
        u = np.where(nan, x, u).astype(ut)
    return u


def reduce_precision(x: np.ndarray, dtype: str, exponent_bits: int, mantissa_bits: int) -> np.ndarray:
    """Values in, values out: f32 / f64 arrays, f16 arrays, or bf16 given as
    uint16 bit patterns (returned as bit patterns)."""
    if dtype == "bf16":
        return reduce_precision_bits(np.asarray(x, np.uint16), "bf16", exponent_bits, mantissa_bits)
    npt = {"f32": np.float32, "f64": np.float64, "f16": np.float16}[dtype]
    ut = _FORMATS[dtype][0]
    v = np.ascontiguousarray(np.asarray(x, npt))
    return reduce_precision_bits(v.view(ut), dtype, exponent_bits, mantissa_bits).view(npt)


_FOLD = {
    "add": lambda a, b: a + b,
    "multiply": lambda a, b: a * b,
    "maximum": lambda a, b: a if np.isnan(a) else (b if np.isnan(b) else max(a, b)),
    "minimum": lambda a, b: a if np.isnan(a) else (b if np.isnan(b) else min(a, b)),
}


def reduce_window(x: np.ndarray, init, op: str, window, strides=None, window_dilations=None, padding=None,
                  acc_dtype=None) -> np.ndarray:
    """Brute force: every output element folds its window positions in
    row-major order, starting from init; positions in the padding contribute
    init. Accumulates in `acc_dtype` (default x's dtype), left to right.
    Small inputs only (pure Python loops)."""
    x = np.asarray(x)
    r = x.ndim
    strides = list(strides or [1] * r)
    wd = list(window_dilations or [1] * r)
    pad = [tuple(p) for p in (padding or [(0, 0)] * r)]
    at = np.dtype(acc_dtype or x.dtype)
    out_shape = []
    for d in range(r):
        padded = pad[d][0] + x.shape[d] + pad[d][1]
        span = (window[d] - 1) * wd[d] + 1
        out_shape.append(0 if padded < span else (padded - span) // strides[d] + 1)
    out = np.empty(out_shape, at)
    iv = at.type(init)
    f = _FOLD[op]
    for o in itertools.product(*[range(n) for n in out_shape]):
        acc = iv
        for w in itertools.product(*[range(n) for n in window]):
            c = [o[d] * strides[d] + w[d] * wd[d] - pad[d][0] for d in range(r)]
            inside = all(0 <= c[d] < x.shape[d] for d in range(r))
            v = at.type(x[tuple(c)]) if inside else iv
            if np.issubdtype(at, np.integer):
                with np.errstate(over="ignore"):
                    acc = at.type(f(acc, v))
            else:
                acc = at.type(f(acc, v))
        out[o] = acc
    return out
