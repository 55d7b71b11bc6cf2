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
