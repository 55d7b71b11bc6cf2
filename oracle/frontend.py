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
                    order from the init value; padded positions and
                    base-dilation holes contribute the init value (StableHLO).
                    The reference computes sum or max over a strided view of
                    the input padded with 0 / -inf (api.cc:4324-4435), the
                    same for init 0 / -inf. Pins: the reference's import case
                    (window 2, padding [1, 0], stablehlo_import_tests.zig:
                    173-207); the cumulative-sum closed form of a stride-1
                    window sum; numpy's sliding_window_view max; base
                    dilation as numpy's strided placement into a zero array
                    (window 1) and the interleaving closed form (window 2);
                    negative padding as cropping.
  reduce_window_arg the (values, indices) pair form with jnp.argmax's rule
                    (reference: api.cc:4437-4620). Pins: numpy's argmax over
                    sliding_window_view (first maximum, NaN first) offset by
                    the window start; numpy padding with (-inf, 0); the
                    reference op suite's reduce_window_argmax_last input
                    (jax_op_suite.py:122,294-310).
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


def _window_geometry(shape, window, strides, window_dilations, padding, base_dilations):
    r = len(shape)
    strides = list(strides or [1] * r)
    wd = list(window_dilations or [1] * r)
    bd = list(base_dilations or [1] * r)
    pad = [tuple(p) for p in (padding or [(0, 0)] * r)]
    out_shape = []
    for d in range(r):
        dilated = (shape[d] - 1) * bd[d] + 1 if shape[d] else 0
        padded = pad[d][0] + dilated + pad[d][1]
        span = (window[d] - 1) * wd[d] + 1
        out_shape.append(0 if padded < span else (padded - span) // strides[d] + 1)
    return strides, wd, bd, pad, out_shape


def _source(o, w, shape, strides, wd, bd, pad):
    """Input coordinate read by window position w of output o, or None for a
    padding position or a base-dilation hole (StableHLO: the input dilated by
    base_dilation, then padded, pad_low possibly negative)."""
    src = []
    for d in range(len(shape)):
        c = o[d] * strides[d] + w[d] * wd[d] - pad[d][0]
        if c < 0 or c % bd[d] != 0 or c // bd[d] >= shape[d]:
            return None
        src.append(c // bd[d])
    return tuple(src)


def reduce_window(x: np.ndarray, init, op: str, window, strides=None, window_dilations=None, padding=None,
                  acc_dtype=None, base_dilations=None) -> np.ndarray:
    """Brute force: every output element folds its window positions in
    row-major order, starting from init; positions in the padding or in a
    base-dilation hole contribute init. Accumulates in `acc_dtype` (default
    x's dtype), left to right. Small inputs only (pure Python loops)."""
    x = np.asarray(x)
    strides, wd, bd, pad, out_shape = _window_geometry(x.shape, window, strides, window_dilations, padding,
                                                       base_dilations)
    at = np.dtype(acc_dtype or x.dtype)
    out = np.empty(out_shape, at)
    iv = at.type(init)
    f = _FOLD[op]
    for o in itertools.product(*[range(n) for n in out_shape]):
        acc = iv
        for w in itertools.product(*[range(n) for n in window]):
            c = _source(o, w, x.shape, strides, wd, bd, pad)
            v = at.type(x[c]) if c is not None else iv
            if np.issubdtype(at, np.integer):
                with np.errstate(over="ignore"):
                    acc = at.type(f(acc, v))
            else:
                acc = at.type(f(acc, v))
        out[o] = acc
    return out


def reduce_window_arg(values: np.ndarray, indices: np.ndarray, init_value, init_index, kind: str, window,
                      strides=None, window_dilations=None, padding=None, base_dilations=None):
    """Two-operand reduce_window over (values, indices) with jnp.argmax's
    pair rule (kind "max"; "min" for argmin): a NaN wins (the lowest index
    among NaNs), then the larger (smaller) value, ties to the lower index;
    the winner's own value and index. Padding and holes contribute
    (init_value, init_index). The rule is a selection, so the fold order does
    not matter; this folds in row-major window order. Brute force, small
    inputs. Reference: the max-pool-with-indices form,
    src/backend/mlx_metal/api.cc:4437-4620 (which breaks value ties by
    window position instead; the pair rule here is JAX's, the declared
    oracle's)."""
    values, indices = np.asarray(values), np.asarray(indices)
    strides, wd, bd, pad, out_shape = _window_geometry(values.shape, window, strides, window_dilations, padding,
                                                       base_dilations)
    ov = np.empty(out_shape, values.dtype)
    oi = np.empty(out_shape, indices.dtype)
    iv, ii = values.dtype.type(init_value), indices.dtype.type(init_index)

    def takes(xv, xi, av, ai):
        xn, an = np.isnan(xv), np.isnan(av)
        if xn or an:
            return bool(xn and (not an or xi < ai))
        if xv == av:
            return bool(xi < ai)
        return bool(xv > av) if kind == "max" else bool(xv < av)

    for o in itertools.product(*[range(n) for n in out_shape]):
        av, ai = iv, ii
        for w in itertools.product(*[range(n) for n in window]):
            c = _source(o, w, values.shape, strides, wd, bd, pad)
            xv, xi = (values[c], indices[c]) if c is not None else (iv, ii)
            if takes(xv, xi, av, ai):
                av, ai = xv, xi
        ov[o], oi[o] = av, ai
    return ov, oi
