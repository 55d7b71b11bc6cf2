"""Numpy restatement of fused attention — TEST INFRASTRUCTURE ONLY.

Only tests/ use this module, as the checker; the plugin never calls it.

attention_f64(q, k, v, ...) is softmax(scale * q.k^T over the allowed keys) . v
in float64 for [B, H, S, D] operands with grouped heads (query head h reads
key/value head h // (Hq // Hkv)); allowed keys are k < Skv and, when causal,
k <= q_coef * q + offset. A row with no allowed key is NaN (0/0), which is
what the unfused softmax (max = -inf, exp(-inf - -inf)) produces.

sdpa_f64(q, k, v, token) is the reference's scaled-dot-product-attention
custom call (reference: src/backend/mlx_metal/api.cc:4928-5062): operands
[b, q, h, hd] or [q, h, hd], scale 1/sqrt(hd) computed in f32, the token
index cast to int32 (api.cc:947), key allowed iff key <= token + query
(api.cc:937-950).

attention_graph_ref(q, k, v, ...) evaluates the unfused graph the planner
rewrites (dot_general -> convert/scale/select -> f32 softmax -> convert ->
dot_general) with its roundings: scores and probabilities rounded to the
16-bit input type, f32 softmax, f32 accumulation.

Parity pins (tests/test_oracle_attention.py):
  * the reference's known answers api_test.cc:271-352 (one head, and four
    query heads over two key/value heads: pins the grouped-head mapping);
  * closed forms: equal scores give the running mean of the allowed value
    rows; one dominant score selects its value row; a first query under a
    causal mask with offset 0 returns value row 0 exactly; an empty allowed
    set gives NaN;
  * the rank-3 and rank-4 custom-call layouts agree; scale invariance
    (q * c with scale / c).
"""
from __future__ import annotations

import numpy as np

from oracle import ops


def _mask(sq: int, skv: int, causal: bool, q_coef: int, offset: int) -> np.ndarray:
    qi = np.arange(sq)[:, None]
    ki = np.arange(skv)[None, :]
    if not causal:
        return np.ones((sq, skv), dtype=bool)
    return ki <= q_coef * qi + offset


def attention_f64(q, k, v, *, scale: float = 1.0, causal: bool = False, q_coef: int = 1, offset: int = 0):
    """q [B, Hq, Sq, D], k/v [B, Hkv, Skv, D] (any float dtype) -> float64."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    assert Hq % Hkv == 0
    rep = Hq // Hkv
    k = np.repeat(k, rep, axis=1)
    v = np.repeat(v, rep, axis=1)
    s = scale * np.matmul(q, np.swapaxes(k, -1, -2))
    allowed = _mask(Sq, Skv, causal, q_coef, offset)
    s = np.where(allowed, s, -np.inf)
    with np.errstate(invalid="ignore"):
        m = s.max(-1, keepdims=True)
        e = np.exp(s - m)
        p = e / e.sum(-1, keepdims=True)
    return np.matmul(p, v)


def sdpa_f64(q, k, v, token: int):
    """The custom call on its own layouts ([b,q,h,hd] or [q,h,hd])."""
    q = np.asarray(q)
    rank3 = q.ndim == 3
    if rank3:
        q, k, v = q[None], np.asarray(k)[None], np.asarray(v)[None]
    hd = q.shape[-1]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    tok = int(np.array(token).astype(np.int64).astype(np.int32))
    t = lambda x: np.transpose(np.asarray(x), (0, 2, 1, 3))  # noqa: E731  [b,s,h,d] -> [b,h,s,d]
    out = attention_f64(t(q), t(k), t(v), scale=scale, causal=True, q_coef=1, offset=tok)
    out = np.transpose(out, (0, 2, 1, 3))
    return out[0] if rank3 else out


def _round16(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.asarray(x, np.float32)
    if dtype == "bf16":
        return ops.bf16_bits_to_f32(ops.f32_to_bf16_bits(x))
    return x.astype(np.float16).astype(np.float32)


def attention_graph_ref(q, k, v, dtype: str, *, scale: float = 1.0, causal: bool = False, q_coef: int = 1,
                        offset: int = 0) -> np.ndarray:
    """The unfused graph's arithmetic (f32 values of 16-bit q, k, v)."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    rep = q.shape[1] // k.shape[1]
    k = np.repeat(k, rep, axis=1)
    v = np.repeat(v, rep, axis=1)
    s = _round16(np.matmul(q.astype(np.float64), np.swapaxes(k, -1, -2)).astype(np.float32), dtype)
    s = (s * np.float32(scale)).astype(np.float32)
    s = np.where(_mask(q.shape[2], k.shape[2], causal, q_coef, offset), s, np.float32(-np.inf))
    with np.errstate(invalid="ignore"):
        m = s.max(-1, keepdims=True)
        e = np.exp(s - m, dtype=np.float32)
        p = _round16(e / e.sum(-1, keepdims=True, dtype=np.float32), dtype)
    return _round16(np.matmul(p.astype(np.float64), v).astype(np.float32), dtype)
