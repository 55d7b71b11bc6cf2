"""Builder of StableHLO text modules in the form JAX prints for
``jax.jit(f).lower(*args).as_text()``.

JAX and jaxlib are not installed on these machines, so the programs that
JAX would hand the plugin are written with this builder instead: each method
emits the StableHLO op (pretty form, or the generic form JAX uses for
gather/scatter) that the corresponding ``jax.numpy`` / ``jax.lax`` call lowers
to, including JAX's conventions (f16 sums upcast to f32, argmax as a
two-operand reduce over (values, iota) with JAX's NaN/tie comparator,
explicit ``broadcast_in_dim`` of scalars).
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass

MLIR_TYPES = {
    "f32": "f32", "bf16": "bf16", "f16": "f16", "f64": "f64", "pred": "i1",
    "s8": "i8", "s16": "i16", "s32": "i32", "s64": "i64",
    "u8": "ui8", "u16": "ui16", "u32": "ui32", "u64": "ui64",
}
FLOATS = {"f32", "bf16", "f16", "f64"}


def tensor_type(shape, dtype: str) -> str:
    return "tensor<" + "".join(f"{d}x" for d in shape) + MLIR_TYPES[dtype] + ">"


@dataclass(frozen=True)
class T:
    name: str
    shape: tuple
    dtype: str

    @property
    def type(self) -> str:
        return tensor_type(self.shape, self.dtype)

    @property
    def rank(self) -> int:
        return len(self.shape)


def _fmt_float(v: float, dtype: str) -> str:
    if math.isnan(v):
        return {"f32": "0x7FC00000", "bf16": "0x7FC0", "f16": "0x7E00", "f64": "0x7FF8000000000000"}[dtype]
    if math.isinf(v):
        if dtype == "f32":
            return "0x7F800000" if v > 0 else "0xFF800000"
        if dtype == "bf16":
            return "0x7F80" if v > 0 else "0xFF80"
        if dtype == "f16":
            return "0x7C00" if v > 0 else "0xFC00"
        return "0x7FF0000000000000" if v > 0 else "0xFFF0000000000000"
    if dtype == "f32":
        v = struct.unpack("<f", struct.pack("<f", v))[0]
        return f"{v:.9e}"  # 9 significant digits round-trip every f32
    return repr(float(v))


def _literal(value, dtype: str) -> str:
    if dtype == "pred":
        return "true" if value else "false"
    if dtype in FLOATS:
        return _fmt_float(float(value), dtype)
    return str(int(value))


class Builder:
    """Accumulates one ``@main`` function; ``build()`` returns module text."""

    def __init__(self, name: str = "jit_f", mesh: str | None = None):
        """`mesh`: an `sdy.mesh` body such as '["x"=1]' to declare (Shardy
        prefix of a jax.jit module on one device); the arguments then carry
        replicated `sdy.sharding` attributes."""
        self.name = name
        self.mesh = mesh
        self.params: list[T] = []
        self.donated: set[str] = set()
        self.lines: list[str] = []
        self._n = 0
        self._c = 0

    # -------------------------------------------------------------- values
    def _fresh(self) -> str:
        n = f"%{self._n}"
        self._n += 1
        return n

    def _emit(self, text: str, shape, dtype) -> T:
        t = T(self._fresh(), tuple(shape), dtype)
        self.lines.append(f"    {t.name} = {text}")
        return t

    def param(self, shape, dtype: str, donate: bool = False) -> T:
        """Entry argument. `donate=True` is jax.jit's donate_argnums: the
        argument is marked `tf.aliasing_output = N` for the first unclaimed
        result of the same type, else `jax.buffer_donor = true`."""
        t = T(f"%arg{len(self.params)}", tuple(shape), dtype)
        self.params.append(t)
        if donate:
            self.donated.add(t.name)
        return t

    def constant(self, value, dtype: str, shape=()) -> T:
        name = f"%cst_{self._c}" if dtype in FLOATS else f"%c_{self._c}"
        self._c += 1
        t = T(name, tuple(shape), dtype)
        self.lines.append(f"    {name} = stablehlo.constant dense<{_literal(value, dtype)}> : {t.type}")
        return t

    def dense(self, values, dtype: str, shape) -> T:
        flat = [_literal(v, dtype) for v in values]
        if len(shape) == 1:
            body = "[" + ", ".join(flat) + "]"
        else:
            import numpy as np
            arr = np.array(flat, dtype=object).reshape(shape)

            def rec(a):
                if a.ndim == 1:
                    return "[" + ", ".join(a) + "]"
                return "[" + ", ".join(rec(x) for x in a) + "]"
            body = rec(arr)
        name = f"%c_{self._c}"
        self._c += 1
        t = T(name, tuple(shape), dtype)
        self.lines.append(f"    {name} = stablehlo.constant dense<{body}> : {t.type}")
        return t

    def scalar_like(self, value, like: T) -> T:
        """Scalar constant broadcast to `like`'s shape (JAX's lowering of
        python scalars in binary ops)."""
        c = self.constant(value, like.dtype)
        if like.rank == 0:
            return c
        return self.broadcast_in_dim(c, like.shape, [])

    # --------------------------------------------------------- elementwise
    def _unary(self, op: str, x: T, dtype: str | None = None) -> T:
        dt = dtype or x.dtype
        if dt == x.dtype:
            return self._emit(f"stablehlo.{op} {x.name} : {x.type}", x.shape, dt)
        return self._emit(f"stablehlo.{op} {x.name} : ({x.type}) -> {tensor_type(x.shape, dt)}", x.shape, dt)

    def _binary(self, op: str, a: T, b: T) -> T:
        assert a.shape == b.shape and a.dtype == b.dtype, (op, a, b)
        return self._emit(f"stablehlo.{op} {a.name}, {b.name} : {a.type}", a.shape, a.dtype)

    def add(self, a, b): return self._binary("add", a, b)
    def subtract(self, a, b): return self._binary("subtract", a, b)
    def multiply(self, a, b): return self._binary("multiply", a, b)
    def divide(self, a, b): return self._binary("divide", a, b)
    def maximum(self, a, b): return self._binary("maximum", a, b)
    def minimum(self, a, b): return self._binary("minimum", a, b)
    def power(self, a, b): return self._binary("power", a, b)
    def remainder(self, a, b): return self._binary("remainder", a, b)
    def and_(self, a, b): return self._binary("and", a, b)
    def or_(self, a, b): return self._binary("or", a, b)
    def xor(self, a, b): return self._binary("xor", a, b)
    def shift_left(self, a, b): return self._binary("shift_left", a, b)
    def shift_right_arithmetic(self, a, b): return self._binary("shift_right_arithmetic", a, b)
    def shift_right_logical(self, a, b): return self._binary("shift_right_logical", a, b)
    def atan2(self, a, b): return self._binary("atan2", a, b)

    def tanh(self, x): return self._unary("tanh", x)
    def exp(self, x): return self._unary("exponential", x)
    def log(self, x): return self._unary("log", x)
    def log1p(self, x): return self._unary("log_plus_one", x)
    def rsqrt(self, x): return self._unary("rsqrt", x)
    def sqrt(self, x): return self._unary("sqrt", x)
    def negate(self, x): return self._unary("negate", x)
    def abs(self, x): return self._unary("abs", x)
    def logistic(self, x): return self._unary("logistic", x)
    def sine(self, x): return self._unary("sine", x)
    def cosine(self, x): return self._unary("cosine", x)
    def floor(self, x): return self._unary("floor", x)
    def ceil(self, x): return self._unary("ceil", x)
    def sign(self, x): return self._unary("sign", x)
    def not_(self, x): return self._unary("not", x)
    def cbrt(self, x): return self._unary("cbrt", x)
    def round_nearest_afz(self, x): return self._unary("round_nearest_afz", x)
    def popcnt(self, x): return self._unary("popcnt", x)
    def clz(self, x): return self._unary("count_leading_zeros", x)
    def is_finite(self, x): return self._unary("is_finite", x, "pred")

    def reduce_precision(self, x: T, exponent_bits: int, mantissa_bits: int, generic: bool = False) -> T:
        if generic:
            return self._emit(f'"stablehlo.reduce_precision"({x.name}) <{{exponent_bits = {exponent_bits} : i32, '
                              f'mantissa_bits = {mantissa_bits} : i32}}> : ({x.type}) -> {x.type}', x.shape, x.dtype)
        return self._emit(f"stablehlo.reduce_precision {x.name}, format = e{exponent_bits}m{mantissa_bits} : {x.type}",
                          x.shape, x.dtype)

    def optimization_barrier(self, xs: list[T]) -> list[T]:
        """stablehlo.optimization_barrier: its results are its operands."""
        name = self._fresh()
        names = ", ".join(x.name for x in xs)
        types = ", ".join(x.type for x in xs)
        if len(xs) == 1:
            self.lines.append(f"    {name} = stablehlo.optimization_barrier {names} : {types}")
            return [T(name, xs[0].shape, xs[0].dtype)]
        self.lines.append(f'    {name}:{len(xs)} = "stablehlo.optimization_barrier"({names}) : ({types}) -> ({types})')
        return [T(f"{name}#{i}", x.shape, x.dtype) for i, x in enumerate(xs)]

    def sharding_constraint(self, x: T) -> T:
        """sdy.sharding_constraint to a replicated sharding (needs a mesh)."""
        rep = ", ".join("{}" for _ in x.shape)
        return self._emit(f"sdy.sharding_constraint {x.name} <@mesh, [{rep}]> : {x.type}", x.shape, x.dtype)

    def reduce_window(self, x: T, init: T, op: str, window, strides=None, window_dilations=None, padding=None,
                      base_dilations=None) -> T:
        """stablehlo.reduce_window (generic form, as jax.lax.reduce_window
        prints it) with a one-op region (add / maximum / minimum / multiply)."""
        r = len(x.shape)
        strides = list(strides or [1] * r)
        wd = list(window_dilations or [1] * r)
        bd = list(base_dilations or [1] * r)
        pad = [list(p) for p in (padding or [(0, 0)] * r)]
        shape = []
        for d in range(r):
            padded = pad[d][0] + (x.shape[d] - 1) * bd[d] + 1 + pad[d][1] if x.shape[d] else pad[d][0] + pad[d][1]
            span = (window[d] - 1) * wd[d] + 1
            shape.append(0 if padded < span else (padded - span) // strides[d] + 1)
        name = self._fresh()
        b = name[1:]
        sv = tensor_type((), x.dtype)
        arr = lambda v: "array<i64: " + ", ".join(str(int(e)) for e in v) + ">"  # noqa: E731
        pads = ", ".join(f"[{lo}, {hi}]" for lo, hi in pad)
        self.lines += [
            f'    {name} = "stablehlo.reduce_window"({x.name}, {init.name}) ({{',
            f"    ^bb0(%w{b}_a: {sv}, %w{b}_b: {sv}):",
            f"      %w{b}_c = stablehlo.{op} %w{b}_a, %w{b}_b : {sv}",
            f"      stablehlo.return %w{b}_c : {sv}",
            f"    }}) {{base_dilations = {arr(bd)}, padding = dense<[{pads}]> : tensor<{r}x2xi64>, "
            f"window_dimensions = {arr(window)}, window_dilations = {arr(wd)}, window_strides = {arr(strides)}}} : "
            f"({x.type}, {init.type}) -> {tensor_type(shape, x.dtype)}",
        ]
        return T(name, tuple(shape), x.dtype)

    def reduce_window_arg(self, x: T, idx: T, init_v: T, init_i: T, window, strides=None, window_dilations=None,
                          padding=None, base_dilations=None, kind: str = "max") -> tuple[T, T]:
        """Two-operand stablehlo.reduce_window over (values, indices) in the
        generic form, with the pair region jax.lax.reduce_window prints for
        the reference op suite's comparator (jax_op_suite.py:294-310):
        keep_left = (v_l > v_r) | ((v_l == v_r) & (i_l < i_r)), then a
        select of each operand (LT for kind "min")."""
        r = len(x.shape)
        strides = list(strides or [1] * r)
        wd = list(window_dilations or [1] * r)
        bd = list(base_dilations or [1] * r)
        pad = [list(p) for p in (padding or [(0, 0)] * r)]
        shape = []
        for d in range(r):
            padded = pad[d][0] + (x.shape[d] - 1) * bd[d] + 1 + pad[d][1] if x.shape[d] else pad[d][0] + pad[d][1]
            span = (window[d] - 1) * wd[d] + 1
            shape.append(0 if padded < span else (padded - span) // strides[d] + 1)
        name = self._fresh()
        b = name[1:]
        sv, si, pred = tensor_type((), x.dtype), tensor_type((), idx.dtype), tensor_type((), "pred")
        ik = "SIGNED" if idx.dtype.startswith("s") else "UNSIGNED"
        cmp = "GT" if kind == "max" else "LT"
        arr = lambda v: "array<i64: " + ", ".join(str(int(e)) for e in v) + ">"  # noqa: E731
        pads = ", ".join(f"[{lo}, {hi}]" for lo, hi in pad)
        self.lines += [
            f'    {name}:2 = "stablehlo.reduce_window"({x.name}, {idx.name}, {init_v.name}, {init_i.name}) ({{',
            f"    ^bb0(%w{b}_a: {sv}, %w{b}_b: {si}, %w{b}_c: {sv}, %w{b}_d: {si}):",
            f"      %w{b}_1 = stablehlo.compare  {cmp}, %w{b}_a, %w{b}_c,  FLOAT : ({sv}, {sv}) -> {pred}",
            f"      %w{b}_2 = stablehlo.compare  EQ, %w{b}_a, %w{b}_c,  FLOAT : ({sv}, {sv}) -> {pred}",
            f"      %w{b}_3 = stablehlo.compare  LT, %w{b}_b, %w{b}_d,  {ik} : ({si}, {si}) -> {pred}",
            f"      %w{b}_4 = stablehlo.and %w{b}_2, %w{b}_3 : {pred}",
            f"      %w{b}_5 = stablehlo.or %w{b}_1, %w{b}_4 : {pred}",
            f"      %w{b}_6 = stablehlo.select %w{b}_5, %w{b}_a, %w{b}_c : {pred}, {sv}",
            f"      %w{b}_7 = stablehlo.select %w{b}_5, %w{b}_b, %w{b}_d : {pred}, {si}",
            f"      stablehlo.return %w{b}_6, %w{b}_7 : {sv}, {si}",
            f"    }}) {{base_dilations = {arr(bd)}, padding = dense<[{pads}]> : tensor<{r}x2xi64>, "
            f"window_dimensions = {arr(window)}, window_dilations = {arr(wd)}, window_strides = {arr(strides)}}} : "
            f"({x.type}, {idx.type}, {init_v.type}, {init_i.type}) -> ({tensor_type(shape, x.dtype)}, "
            f"{tensor_type(shape, idx.dtype)})",
        ]
        return T(f"{name}#0", tuple(shape), x.dtype), T(f"{name}#1", tuple(shape), idx.dtype)

    def convert(self, x: T, dtype: str) -> T:
        return self._emit(f"stablehlo.convert {x.name} : ({x.type}) -> {tensor_type(x.shape, dtype)}", x.shape, dtype)

    def bitcast_convert(self, x: T, dtype: str) -> T:
        return self._emit(f"stablehlo.bitcast_convert {x.name} : ({x.type}) -> {tensor_type(x.shape, dtype)}",
                          x.shape, dtype)

    def compare(self, direction: str, a: T, b: T, kind: str | None = None) -> T:
        kind = kind or ("FLOAT" if a.dtype in FLOATS else ("UNSIGNED" if a.dtype.startswith("u") or a.dtype == "pred"
                                                            else "SIGNED"))
        out = tensor_type(a.shape, "pred")
        return self._emit(f"stablehlo.compare  {direction}, {a.name}, {b.name},  {kind} : ({a.type}, {b.type}) -> {out}",
                          a.shape, "pred")

    def select(self, p: T, a: T, b: T) -> T:
        return self._emit(f"stablehlo.select {p.name}, {a.name}, {b.name} : {p.type}, {a.type}", a.shape, a.dtype)

    def clamp(self, lo: T, x: T, hi: T) -> T:
        if lo.shape == x.shape and hi.shape == x.shape:
            return self._emit(f"stablehlo.clamp {lo.name}, {x.name}, {hi.name} : {x.type}", x.shape, x.dtype)
        return self._emit(f"stablehlo.clamp {lo.name}, {x.name}, {hi.name} : ({lo.type}, {x.type}, {hi.type}) -> "
                          f"{x.type}", x.shape, x.dtype)

    # ------------------------------------------------------------- views
    def broadcast_in_dim(self, x: T, shape, dims) -> T:
        d = ", ".join(str(v) for v in dims)
        return self._emit(f"stablehlo.broadcast_in_dim {x.name}, dims = [{d}] : ({x.type}) -> "
                          f"{tensor_type(shape, x.dtype)}", shape, x.dtype)

    def reshape(self, x: T, shape) -> T:
        return self._emit(f"stablehlo.reshape {x.name} : ({x.type}) -> {tensor_type(shape, x.dtype)}", shape, x.dtype)

    def transpose(self, x: T, perm) -> T:
        shape = tuple(x.shape[p] for p in perm)
        d = ", ".join(str(v) for v in perm)
        return self._emit(f"stablehlo.transpose {x.name}, dims = [{d}] : ({x.type}) -> {tensor_type(shape, x.dtype)}",
                          shape, x.dtype)

    def slice(self, x: T, start, limit, strides=None) -> T:
        strides = strides or [1] * x.rank
        shape = tuple((l - s + st - 1) // st for s, l, st in zip(start, limit, strides))
        rng = ", ".join(f"{s}:{l}" if st == 1 else f"{s}:{l}:{st}" for s, l, st in zip(start, limit, strides))
        return self._emit(f"stablehlo.slice {x.name} [{rng}] : ({x.type}) -> {tensor_type(shape, x.dtype)}",
                          shape, x.dtype)

    def iota(self, shape, dim: int, dtype: str = "s32") -> T:
        return self._emit(f"stablehlo.iota dim = {dim} : {tensor_type(shape, dtype)}", shape, dtype)

    def reverse(self, x: T, dims) -> T:
        d = ", ".join(str(v) for v in dims)
        return self._emit(f"stablehlo.reverse {x.name}, dims = [{d}] : {x.type}", x.shape, x.dtype)

    def concatenate(self, xs: list[T], dim: int) -> T:
        shape = list(xs[0].shape)
        shape[dim] = sum(x.shape[dim] for x in xs)
        names = ", ".join(x.name for x in xs)
        types = ", ".join(x.type for x in xs)
        return self._emit(f"stablehlo.concatenate {names}, dim = {dim} : ({types}) -> "
                          f"{tensor_type(shape, xs[0].dtype)}", shape, xs[0].dtype)

    # ------------------------------------------- materializing structural ops
    def dynamic_slice(self, x: T, starts: list[T], sizes) -> T:
        names = ", ".join([x.name] + [s.name for s in starts])
        types = ", ".join([x.type] + [s.type for s in starts])
        sz = ", ".join(str(v) for v in sizes)
        return self._emit(f"stablehlo.dynamic_slice {names}, sizes = [{sz}] : ({types}) -> "
                          f"{tensor_type(sizes, x.dtype)}", sizes, x.dtype)

    def dynamic_update_slice(self, x: T, update: T, starts: list[T]) -> T:
        names = ", ".join([x.name, update.name] + [s.name for s in starts])
        types = ", ".join([x.type, update.type] + [s.type for s in starts])
        return self._emit(f"stablehlo.dynamic_update_slice {names} : ({types}) -> {x.type}", x.shape, x.dtype)

    def custom_call(self, target: str, operands: list[T], shape, dtype: str, generic: bool = False) -> T:
        """stablehlo.custom_call as JAX prints it (pretty form), or the generic
        "stablehlo.custom_call"(...) {call_target_name = ...} form."""
        names = ", ".join(o.name for o in operands)
        types = ", ".join(o.type for o in operands)
        out = tensor_type(shape, dtype)
        if generic:
            return self._emit(f'"stablehlo.custom_call"({names}) {{api_version = 2 : i32, backend_config = "", '
                              f'call_target_name = "{target}"}} : ({types}) -> {out}', shape, dtype)
        return self._emit(f'stablehlo.custom_call @{target}({names}) {{api_version = 2 : i32, backend_config = ""}} : '
                          f"({types}) -> {out}", shape, dtype)

    def pad(self, x: T, value: T, low, high, interior) -> T:
        shape = tuple(lo + hi + d + max(d - 1, 0) * it for d, lo, hi, it in zip(x.shape, low, high, interior))
        f = lambda v: ", ".join(str(a) for a in v)  # noqa: E731
        return self._emit(f"stablehlo.pad {x.name}, {value.name}, low = [{f(low)}], high = [{f(high)}], interior = "
                          f"[{f(interior)}] : ({x.type}, {value.type}) -> {tensor_type(shape, x.dtype)}", shape, x.dtype)

    def dot_general(self, a: T, b: T, batch=((), ()), contract=((), ()), out_dtype: str | None = None) -> T:
        lb, rb = list(batch[0]), list(batch[1])
        lc, rc = list(contract[0]), list(contract[1])
        shape = [a.shape[d] for d in lb]
        shape += [a.shape[d] for d in range(a.rank) if d not in lb and d not in lc]
        shape += [b.shape[d] for d in range(b.rank) if d not in rb and d not in rc]
        f = lambda v: ", ".join(str(x) for x in v)  # noqa: E731
        bd = f"batching_dims = [{f(lb)}] x [{f(rb)}], " if lb else ""
        dt = out_dtype or a.dtype
        return self._emit(f"stablehlo.dot_general {a.name}, {b.name}, {bd}contracting_dims = [{f(lc)}] x [{f(rc)}], "
                          f"precision = [DEFAULT, DEFAULT] : ({a.type}, {b.type}) -> {tensor_type(shape, dt)}",
                          shape, dt)

    def gather(self, x: T, idx: T, offset_dims, collapsed_slice_dims, start_index_map, index_vector_dim, slice_sizes,
               operand_batching_dims=(), start_indices_batching_dims=()) -> T:
        f = lambda v: ", ".join(str(a) for a in v)  # noqa: E731
        batch_idx = [d for d in range(idx.rank) if d != index_vector_dim]
        out_rank = len(batch_idx) + len(offset_dims)
        window = [d for d in range(x.rank) if d not in collapsed_slice_dims and d not in operand_batching_dims]
        shape, bi, wi = [], 0, 0
        for o in range(out_rank):
            if o in offset_dims:
                shape.append(slice_sizes[window[wi]])
                wi += 1
            else:
                shape.append(idx.shape[batch_idx[bi]])
                bi += 1
        extra = ""
        if operand_batching_dims:
            extra = (f", operand_batching_dims = [{f(operand_batching_dims)}], start_indices_batching_dims = "
                     f"[{f(start_indices_batching_dims)}]")
        dn = (f"#stablehlo.gather<offset_dims = [{f(offset_dims)}], collapsed_slice_dims = [{f(collapsed_slice_dims)}]"
              f"{extra}, start_index_map = [{f(start_index_map)}], index_vector_dim = {index_vector_dim}>")
        return self._emit(f"\"stablehlo.gather\"({x.name}, {idx.name}) <{{dimension_numbers = {dn}, "
                          f"indices_are_sorted = false, slice_sizes = array<i64: {f(slice_sizes)}>}}> : "
                          f"({x.type}, {idx.type}) -> {tensor_type(shape, x.dtype)}", shape, x.dtype)

    def scatter(self, x: T, idx: T, upd: T, update_window_dims, inserted_window_dims, scatter_dims_to_operand_dims,
                index_vector_dim, combiner: str = "add", input_batching_dims=(), scatter_indices_batching_dims=()) -> T:
        f = lambda v: ", ".join(str(a) for a in v)  # noqa: E731
        extra = ""
        if input_batching_dims:
            extra = (f", input_batching_dims = [{f(input_batching_dims)}], scatter_indices_batching_dims = "
                     f"[{f(scatter_indices_batching_dims)}]")
        dn = (f"#stablehlo.scatter<update_window_dims = [{f(update_window_dims)}], inserted_window_dims = "
              f"[{f(inserted_window_dims)}]{extra}, scatter_dims_to_operand_dims = [{f(scatter_dims_to_operand_dims)}], "
              f"index_vector_dim = {index_vector_dim}>")
        name = self._fresh()
        st = tensor_type((), x.dtype)
        b = name[1:]
        if combiner == "set":
            body = [f"      stablehlo.return %s{b}_u : {st}"]
        else:
            body = [f"      %s{b}_r = stablehlo.{combiner} %s{b}_a, %s{b}_u : {st}",
                    f"      stablehlo.return %s{b}_r : {st}"]
        self.lines.extend([
            f"    {name} = \"stablehlo.scatter\"({x.name}, {idx.name}, {upd.name}) <{{indices_are_sorted = false, "
            f"scatter_dimension_numbers = {dn}, unique_indices = false}}> ({{",
            f"    ^bb0(%s{b}_a: {st}, %s{b}_u: {st}):",
            *body,
            f"    }}) : ({x.type}, {idx.type}, {upd.type}) -> {x.type}",
        ])
        return T(name, x.shape, x.dtype)

    # -------------------------------------------------------- reductions
    def reduce(self, x: T, init: T, dims, op: str) -> T:
        """Single-operand reduce in the `applies` form (op: add/maximum/minimum/...)."""
        shape = tuple(s for i, s in enumerate(x.shape) if i not in dims)
        d = ", ".join(str(v) for v in dims)
        return self._emit(f"stablehlo.reduce({x.name} init: {init.name}) applies stablehlo.{op} across dimensions = "
                          f"[{d}] : ({x.type}, {init.type}) -> {tensor_type(shape, x.dtype)}", shape, x.dtype)

    def argmax(self, x: T, axis: int, index_dtype: str = "s32", both: bool = True, kind: str = "max",
               idx: T | None = None):
        """Two-operand reduce over (x, iota) with JAX's argmax/argmin
        comparator (NaN wins, ties -> lowest index). Returns (values, indices).
        `idx` replaces the iota as the index operand."""
        if idx is None:
            idx = self.iota(x.shape, axis, index_dtype)
        init_v = self.constant(float("-inf") if kind == "max" else float("inf"), x.dtype)
        init_i = self.constant(0, index_dtype)
        shape = tuple(s for i, s in enumerate(x.shape) if i != axis)
        name = self._fresh()
        sv, si = tensor_type((), x.dtype), tensor_type((), index_dtype)
        cmp = "GT" if kind == "max" else "LT"
        fk = "FLOAT"
        ik = "SIGNED" if index_dtype.startswith("s") else "UNSIGNED"
        pred = tensor_type((), "pred")
        b = name[1:]
        body = [
            f"    {name}:2 = stablehlo.reduce({x.name} init: {init_v.name}), ({idx.name} init: {init_i.name}) across "
            f"dimensions = [{axis}] : ({x.type}, {idx.type}, {sv}, {si}) -> ({tensor_type(shape, x.dtype)}, "
            f"{tensor_type(shape, index_dtype)})",
            f"     reducer(%r{b}_a: {sv}, %r{b}_c: {sv}) (%r{b}_b: {si}, %r{b}_d: {si})  {{",
            f"      %r{b}_1 = stablehlo.compare  {cmp}, %r{b}_a, %r{b}_c,  {fk} : ({sv}, {sv}) -> {pred}",
            f"      %r{b}_2 = stablehlo.compare  NE, %r{b}_a, %r{b}_a,  {fk} : ({sv}, {sv}) -> {pred}",
            f"      %r{b}_3 = stablehlo.or %r{b}_1, %r{b}_2 : {pred}",
            f"      %r{b}_4 = stablehlo.compare  EQ, %r{b}_a, %r{b}_c,  {fk} : ({sv}, {sv}) -> {pred}",
            f"      %r{b}_5 = stablehlo.compare  LT, %r{b}_b, %r{b}_d,  {ik} : ({si}, {si}) -> {pred}",
            f"      %r{b}_6 = stablehlo.and %r{b}_4, %r{b}_5 : {pred}",
            f"      %r{b}_7 = stablehlo.or %r{b}_3, %r{b}_6 : {pred}",
            f"      %r{b}_8 = stablehlo.select %r{b}_3, %r{b}_a, %r{b}_c : {pred}, {sv}",
            f"      %r{b}_9 = stablehlo.select %r{b}_7, %r{b}_b, %r{b}_d : {pred}, {si}",
            f"      stablehlo.return %r{b}_8, %r{b}_9 : {sv}, {si}",
            "    }",
        ]
        self.lines.extend(body)
        return T(f"{name}#0", shape, x.dtype), T(f"{name}#1", shape, index_dtype)

    def sort(self, operands: list[T], dimension: int = -1, direction: str = "LT",
             compare_type: str | None = None, swap: bool = False) -> list[T]:
        """stablehlo.sort in the generic form jax.jit prints (jnp.sort,
        jnp.argsort): operands sorted together by operand 0 under
        `compare direction, lhs_0, rhs_0` (`swap` compares rhs_0 with lhs_0).
        compare_type defaults to TOTALORDER for floats, SIGNED/UNSIGNED for
        integers."""
        x = operands[0]
        dim = dimension % len(x.shape)
        if compare_type is None:
            if x.dtype in ("f32", "f16", "bf16", "f64"):
                compare_type = "TOTALORDER"
            else:
                compare_type = "UNSIGNED" if x.dtype.startswith("u") or x.dtype == "pred" else "SIGNED"
        name = self._fresh()
        b = name[1:]
        args = []
        for i, o in enumerate(operands):
            st = tensor_type((), o.dtype)
            args += [f"%s{b}_l{i}: {st}", f"%s{b}_r{i}: {st}"]
        sx = tensor_type((), x.dtype)
        lhs, rhs = (f"%s{b}_r0", f"%s{b}_l0") if swap else (f"%s{b}_l0", f"%s{b}_r0")
        ins = ", ".join(o.name for o in operands)
        in_t = ", ".join(o.type for o in operands)
        out_t = in_t if len(operands) == 1 else f"({in_t})"
        res = f"{name}:{len(operands)}" if len(operands) > 1 else name
        self.lines += [
            f'    {res} = "stablehlo.sort"({ins}) <{{dimension = {dim} : i64, is_stable = true}}> ({{',
            f"    ^bb0({', '.join(args)}):",
            f"      %s{b}_c = stablehlo.compare  {direction}, {lhs}, {rhs},  {compare_type} : ({sx}, {sx}) -> "
            f"{tensor_type((), 'pred')}",
            f"      stablehlo.return %s{b}_c : {tensor_type((), 'pred')}",
            f"    }}) : ({in_t}) -> {out_t}",
        ]
        if len(operands) == 1:
            return [T(name, x.shape, x.dtype)]
        return [T(f"{name}#{i}", o.shape, o.dtype) for i, o in enumerate(operands)]

    def top_k(self, x: T, k: int) -> tuple[T, T]:
        """chlo.top_k (lax.top_k): the k largest along the last dim, largest
        first, and their s32 positions."""
        name = self._fresh()
        shape = tuple(x.shape[:-1]) + (k,)
        vt, it = tensor_type(shape, x.dtype), tensor_type(shape, "s32")
        self.lines.append(f"    {name}:2 = chlo.top_k({x.name}, k = {k}) : {x.type} -> ({vt}, {it})")
        return T(f"{name}#0", shape, x.dtype), T(f"{name}#1", shape, "s32")

    def while_loop(self, state: list[T], cond_fn, body_fn) -> list[T]:
        """stablehlo.while in the pretty form jax.jit prints for lax.while_loop
        / fori_loop: `cond_fn(*args)` returns a pred scalar, `body_fn(*args)`
        the next state (same types). Values built before the loop may be
        used inside (captured)."""
        base = self._fresh()[1:]
        args = [T(f"%iterArg_{base}_{i}", s.shape, s.dtype) for i, s in enumerate(state)]
        outer = self.lines
        regions = []
        for fn in (cond_fn, body_fn):
            self.lines = []
            out = fn(*args)
            out = out if isinstance(out, (list, tuple)) else [out]
            names = ", ".join(o.name for o in out)
            types = ", ".join(o.type for o in out)
            regions.append(self.lines + [f"    stablehlo.return {names} : {types}"])
        self.lines = outer
        res = self._fresh()
        inits = ", ".join(f"{a.name} = {s.name}" for a, s in zip(args, state))
        types = ", ".join(s.type for s in state)
        count = f":{len(state)}" if len(state) > 1 else ""
        self.lines.append(f"    {res}{count} = stablehlo.while({inits}) : {types}")
        self.lines.append("     cond {")
        self.lines.extend("  " + line for line in regions[0])
        self.lines.append("    } do {")
        self.lines.extend("  " + line for line in regions[1])
        self.lines.append("    }")
        if len(state) == 1:
            return [T(res, state[0].shape, state[0].dtype)]
        return [T(f"{res}#{i}", s.shape, s.dtype) for i, s in enumerate(state)]

    # JAX-level helpers --------------------------------------------------
    def sum(self, x: T, axes) -> T:
        """jnp.sum: f16/bf16 inputs are summed in f32 and converted back."""
        axes = list(axes)
        if x.dtype in ("f16", "bf16"):
            xf = self.convert(x, "f32")
            r = self.reduce(xf, self.constant(0.0, "f32"), axes, "add")
            return self.convert(r, x.dtype)
        return self.reduce(x, self.constant(0, x.dtype), axes, "add")

    def max(self, x: T, axes) -> T:
        init = self.constant(float("-inf") if x.dtype in FLOATS else -(2 ** 31), x.dtype)
        return self.reduce(x, init, list(axes), "maximum")

    def min(self, x: T, axes) -> T:
        init = self.constant(float("inf") if x.dtype in FLOATS else 2 ** 31 - 1, x.dtype)
        return self.reduce(x, init, list(axes), "minimum")

    # ------------------------------------------------------------ output
    def build(self, outputs: list[T]) -> str:
        claimed: set[int] = set()
        parts = []
        for p in self.params:
            attr = ""
            if p.name in self.donated:
                match = next((i for i, o in enumerate(outputs) if i not in claimed and o.type == p.type), None)
                if match is None:
                    attr = " {jax.buffer_donor = true}"
                else:
                    claimed.add(match)
                    attr = f" {{tf.aliasing_output = {match} : i32}}"
            if self.mesh is not None:
                rep = ", ".join("{}" for _ in p.shape)
                shard = f"sdy.sharding = #sdy.sharding<@mesh, [{rep}]>"
                attr = f" {{{shard}}}" if not attr else attr[:-1] + f", {shard}}}"
            parts.append(f"{p.name}: {p.type}{attr}")
        args = ", ".join(parts)
        if len(outputs) == 1:
            res = f"({outputs[0].type} {{jax.result_info = \"result\"}})"
        else:
            res = "(" + ", ".join(f"{o.type} {{jax.result_info = \"result[{i}]\"}}" for i, o in enumerate(outputs)) + ")"
        ret_names = ", ".join(o.name for o in outputs)
        ret_types = ", ".join(o.type for o in outputs)
        return "\n".join([
            f"module @{self.name} attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{",
            *([f"  sdy.mesh @mesh = <{self.mesh}>"] if self.mesh is not None else []),
            f"  func.func public @main({args}) -> {res} {{",
            *self.lines,
            f"    return {ret_names} : {ret_types}",
            "  }",
            "}",
            "",
        ])
