"""Numpy restatement of the llama-like decoder — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker; the plugin never calls it.

The restatement follows the program that pjrtx_amd.llama_like builds (the
form jax.jit lowers a llama block to), op by op. bf16 values are rounded to
bf16 exactly where the program stores a bf16 tensor:

* the results of dots (f32 accumulation, then one rounding);
* the results of bf16 elementwise ops (computed in f32, then rounded);
* the converts back to bf16.

f32 values stay f32. The reference's own numpy model
(src/plugin/jax/jax_llama_like_inference.py:206-237) is a one-block f32 toy
with the same pieces: RMS normalisation, q/k/v projections, softmax
attention and a gated MLP.

Parity pins (tests/test_oracle_llama.py):

* **RoPE.** It preserves each rotated pair's norm and is the identity at
  position 0. q·k after RoPE depends only on the position difference. It
  matches a complex-number form of the rotation.
* **RMSNorm.** It matches a float64 closed form.
* **Attention.** With zero query weights the scores are uniform, so the
  context is the running mean of V over positions ≤ pos.
* **The whole forward.** It matches an independent float64 einsum
  restatement, with no bf16 rounding, within bf16 tolerance.
* **The KV cache.** Prefill of n+1 tokens gives the last-position logits of
  prefill(n) followed by one decode step.
"""
from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round f32 values to the nearest bf16 (ties to even), returned as f32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) & np.uint32(0xFFFF0000)).astype(np.uint32)
    return r.view(np.float32)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def weights_f32(cfg, weight_bits: list[np.ndarray]) -> dict:
    """bf16 bit patterns -> f32 arrays, converted in row blocks on a thread
    pool (numpy releases the GIL inside the shifts)."""
    from concurrent.futures import ThreadPoolExecutor
    import os
    from pjrtx_amd.llama_like import weight_shapes
    out = {name: np.empty(w.shape, np.float32) for (name, _), w in zip(weight_shapes(cfg), weight_bits)}
    jobs = []
    for (name, _), w in zip(weight_shapes(cfg), weight_bits):
        src, dst = w.reshape(-1), out[name].reshape(-1)
        for lo in range(0, src.size, 1 << 22):
            jobs.append((src, dst, lo, min(src.size, lo + (1 << 22))))

    def conv(job):
        src, dst, lo, hi = job
        dst[lo:hi] = bf16_bits_to_f32(src[lo:hi])

    with ThreadPoolExecutor(max(1, min(16, os.cpu_count() or 1))) as ex:
        list(ex.map(conv, jobs))
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x [T,d] bf16 values (f32 array), w [d]: bf16(bf16(x*rsqrt(mean(x^2)+eps)) * w)."""
    xf = x.astype(np.float32)
    ss = np.sum(xf * xf, axis=1, dtype=np.float32)
    ms = ss / np.float32(x.shape[1])
    r = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    y = bf16_round(xf * r[:, None])
    return bf16_round(y * w[None, :])


def rope_tables(cfg, pos: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    from pjrtx_amd.llama_like import rope_inv_freq
    inv = rope_inv_freq(cfg)
    ang = pos.astype(np.float32)[:, None] * inv[None, :]
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    return np.concatenate([c, c], 1), np.concatenate([s, s], 1)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [H,T,D] bf16 values: bf16(x*cos + rotate_half(x)*sin) in f32."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], -1)
    return bf16_round(x * cos[None] + rot * sin[None])


def mm(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """bf16 x bf16 -> f32 accumulate -> bf16."""
    return bf16_round(np.matmul(a.astype(np.float32), w.astype(np.float32)))


def forward(cfg, W: dict, tokens: np.ndarray, start: int, kcache: list, vcache: list):
    """One program execution: tokens [T] at positions start..start+T-1.
    Caches are lists of [H, L, D] f32 arrays (bf16 values), updated in place.
    Returns (next_token int, logits [vocab] f32 with bf16 values)."""
    T = len(tokens)
    H, D = cfg.heads, cfg.head_dim
    tok = np.where(tokens < 0, tokens + cfg.vocab, tokens)
    tok = np.clip(tok, 0, cfg.vocab - 1)
    x = W["embed"][tok]
    pos = np.arange(start, start + T, dtype=np.int32)
    cos, sin = rope_tables(cfg, pos)
    scale = np.float32(1.0 / np.sqrt(D))
    key = np.arange(cfg.max_len)
    for layer in range(cfg.layers):
        w = lambda n: W[f"l{layer}.{n}"]  # noqa: E731
        h = rmsnorm(x, w("attn_norm"), cfg.eps)
        q = rope(mm(h, w("wq")).reshape(T, H, D).transpose(1, 0, 2), cos, sin)
        k = rope(mm(h, w("wk")).reshape(T, H, D).transpose(1, 0, 2), cos, sin)
        v = mm(h, w("wv")).reshape(T, H, D).transpose(1, 0, 2)
        s0 = min(max(start, 0), cfg.max_len - T)  # dynamic_update_slice clamps the start
        kcache[layer][:, s0:s0 + T] = k
        vcache[layer][:, s0:s0 + T] = v
        s = bf16_round(np.matmul(q, kcache[layer].transpose(0, 2, 1)))          # [H,T,L]
        sf = s * scale
        sf = np.where(key[None, None, :] <= pos[None, :, None], sf, np.float32(-np.inf))
        m = sf.max(axis=2, keepdims=True)
        e = np.exp(sf - m).astype(np.float32)
        p = bf16_round(e / e.sum(axis=2, keepdims=True, dtype=np.float32))
        ctx = bf16_round(np.matmul(p, vcache[layer]))                            # [H,T,D]
        ctx = ctx.transpose(1, 0, 2).reshape(T, H * D)
        x = bf16_round(x + mm(ctx, w("wo")))
        h = rmsnorm(x, w("ffn_norm"), cfg.eps)
        g = mm(h, w("w1"))
        silu = bf16_round(g * (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))))
        act = bf16_round(silu * mm(h, w("w3")))
        x = bf16_round(x + mm(act, w("w2")))
    h = rmsnorm(x[-1:], W["final_norm"], cfg.eps)
    logits = mm(h, W["lm_head"])[0]
    nan = np.isnan(logits)
    nxt = int(np.argmax(nan)) if nan.any() else int(np.argmax(logits))
    return nxt, logits


def empty_caches(cfg):
    shape = (cfg.heads, cfg.max_len, cfg.head_dim)
    return [np.zeros(shape, np.float32) for _ in range(cfg.layers)], \
        [np.zeros(shape, np.float32) for _ in range(cfg.layers)]


def generate(cfg, W: dict, prompt: np.ndarray, new_tokens: int, forced: np.ndarray | None = None):
    """Greedy decode: prefill, then one step per token. With `forced`, the
    given tokens are fed instead of the argmax (teacher forcing), so that
    logits can be compared step by step. Returns (tokens, logits list)."""
    kc, vc = empty_caches(cfg)
    t, lg = forward(cfg, W, np.asarray(prompt, np.int32), 0, kc, vc)
    toks, logits = [t], [lg]
    p = len(prompt)
    for i in range(new_tokens - 1):
        feed = int(forced[i]) if forced is not None else toks[-1]
        t, lg = forward(cfg, W, np.array([feed], np.int32), p + i, kc, vc)
        toks.append(t)
        logits.append(lg)
    return np.array(toks, np.int32), logits


# ------------------------------------------------- independent float64 form

def forward_f64(cfg, W: dict, tokens: np.ndarray) -> np.ndarray:
    """Full recompute over `tokens` (positions 0..T-1) in float64 with no bf16
    rounding, written independently (einsum, complex RoPE). Returns the
    last position's logits."""
    T = len(tokens)
    H, D = cfg.heads, cfg.head_dim
    Wd = {k: v.astype(np.float64) for k, v in W.items()}
    x = Wd["embed"][np.asarray(tokens) % cfg.vocab]
    half = D // 2
    inv = cfg.theta ** (-np.arange(half) * 2.0 / D)
    rot = np.exp(1j * np.arange(T)[:, None] * inv[None, :])                        # [T, half]

    def norm(v, g):
        return v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + cfg.eps) * g

    def rope_c(a):  # a [T, H, D]: pairs (i, i+half) as complex numbers
        z = (a[..., :half] + 1j * a[..., half:]) * rot[:, None, :]
        return np.concatenate([z.real, z.imag], -1)

    causal = np.tril(np.ones((T, T), bool))
    for layer in range(cfg.layers):
        w = lambda n: Wd[f"l{layer}.{n}"]  # noqa: E731
        h = norm(x, w("attn_norm"))
        q = rope_c((h @ w("wq")).reshape(T, H, D))
        k = rope_c((h @ w("wk")).reshape(T, H, D))
        v = (h @ w("wv")).reshape(T, H, D)
        s = np.einsum("qhd,khd->hqk", q, k) / np.sqrt(D)
        s = np.where(causal[None], s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        ctx = np.einsum("hqk,khd->qhd", p, v).reshape(T, H * D)
        x = x + ctx @ w("wo")
        h = norm(x, w("ffn_norm"))
        g = h @ w("w1")
        x = x + ((g / (1 + np.exp(-g))) * (h @ w("w3"))) @ w("w2")
    return norm(x[-1], Wd["final_norm"]) @ Wd["lm_head"]


class DecoderF64:
    """Incremental float64 decode with float64 KV caches and no bf16 rounding:
    the exact model (the same arithmetic as `forward_f64`) evaluated one
    program execution at a time, so that every step of a long decode can be
    compared with the exact logits without recomputing the whole prefix.
    `step(tokens)` runs tokens at the next positions (the prompt as one call,
    then one token per call) and returns the last position's logits.

    Pinned by tests/test_oracle_llama.py: after a prefill and each decode
    step its logits equal `forward_f64` over the whole prefix (float64
    rounding only)."""

    def __init__(self, cfg, W: dict):
        self.cfg = cfg
        self.Wd = {k: v.astype(np.float64) for k, v in W.items()}
        H, D = cfg.heads, cfg.head_dim
        self.k = [np.zeros((cfg.max_len, H, D)) for _ in range(cfg.layers)]
        self.v = [np.zeros((cfg.max_len, H, D)) for _ in range(cfg.layers)]
        self.n = 0
        half = D // 2
        self.inv = cfg.theta ** (-np.arange(half) * 2.0 / D)

    def step(self, tokens) -> np.ndarray:
        cfg, Wd = self.cfg, self.Wd
        tokens = np.asarray(tokens)
        T = len(tokens)
        H, D = cfg.heads, cfg.head_dim
        half = D // 2
        p0 = self.n
        assert p0 + T <= cfg.max_len, "the exact decoder has no clamped positions"
        pos = np.arange(p0, p0 + T)
        rot = np.exp(1j * pos[:, None] * self.inv[None, :])                     # [T, half]
        x = Wd["embed"][tokens % cfg.vocab]

        def norm(v, g):
            return v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + cfg.eps) * g

        def rope_c(a):
            z = (a[..., :half] + 1j * a[..., half:]) * rot[:, None, :]
            return np.concatenate([z.real, z.imag], -1)

        L = p0 + T
        allowed = np.arange(L)[None, :] <= pos[:, None]                          # [T, L]
        for layer in range(cfg.layers):
            w = lambda n: Wd[f"l{layer}.{n}"]  # noqa: E731
            h = norm(x, w("attn_norm"))
            q = rope_c((h @ w("wq")).reshape(T, H, D))
            self.k[layer][p0:L] = rope_c((h @ w("wk")).reshape(T, H, D))
            self.v[layer][p0:L] = (h @ w("wv")).reshape(T, H, D)
            s = np.einsum("qhd,khd->hqk", q, self.k[layer][:L]) / np.sqrt(D)
            s = np.where(allowed[None], s, -np.inf)
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            ctx = np.einsum("hqk,khd->qhd", p, self.v[layer][:L]).reshape(T, H * D)
            x = x + ctx @ w("wo")
            h = norm(x, w("ffn_norm"))
            g = h @ w("w1")
            x = x + ((g / (1 + np.exp(-g))) * (h @ w("w3"))) @ w("w2")
        self.n = L
        return norm(x[-1], Wd["final_norm"]) @ Wd["lm_head"]
