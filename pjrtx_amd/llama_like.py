"""Llama-like decoder inference on the pjrtx plugin.

The model, in the form `jax.jit` lowers it to StableHLO:

* Embedding lookup: a gather over [vocab, d] with negative-index wrap.
* Each of `layers` blocks:
  * RMSNorm in f32 (sum of squares / d, rsqrt(ms + eps)), cast to bf16,
    times the bf16 gain.
  * Q/K/V projections [d, heads*head_dim].
  * RoPE of the rotate-half form, computed in f32. The angles are
    position * theta^(-2i/head_dim).
  * A static KV cache [1, heads, max_len, head_dim] per layer, written with
    dynamic_update_slice at the token position.
  * Scores q·kᵀ over the whole cache, scaled by 1/sqrt(head_dim) and masked
    to key position <= query position.
  * Softmax in f32 and the context p·v.
  * The output projection and the residual add.
  * RMSNorm, then the SwiGLU FFN: silu(h·w1) * (h·w3), then ·w2, then the
    residual add.
* The final RMSNorm, the lm_head [d, vocab], and a greedy argmax (JAX's
  comparator: ties go to the lowest index).

Weights are program arguments, as a jitted function of a params pytree
receives them. The caches are donated (`donate_argnums`), so each decode
step updates them in place. The reference's own llama-like fixture
(src/plugin/jax/jax_llama_like_inference.py:206-237, 304-330) is a one-block
f32 toy. This module is the larger bf16 decoder that C5 names, built with
the same pieces.

Two programs:

* **prefill** takes `(weights..., tokens [P] s32, caches...)` and returns
  `(next_token [1] s32, logits [1, vocab] bf16, caches...)`.
* **decode** takes `(weights..., token [1] s32, pos s32, caches...)` and
  returns the same outputs.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass

import numpy as np

from .hlo import Builder, T


@dataclass(frozen=True)
class LlamaConfig:
    layers: int = 8
    d_model: int = 2048
    heads: int = 16
    head_dim: int = 128
    ffn: int = 5632
    vocab: int = 32000
    eps: float = 1e-5
    theta: float = 10000.0
    max_len: int = 640
    prompt: int = 512
    new_tokens: int = 128

    @property
    def qdim(self) -> int:
        return self.heads * self.head_dim


FULL = LlamaConfig()
# Small enough for the numpy oracle in a unit test; same structure.
TINY = LlamaConfig(layers=2, d_model=128, heads=4, head_dim=32, ffn=320, vocab=512, max_len=40, prompt=12,
                   new_tokens=10)

LAYER_WEIGHTS = ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w1", "w3", "w2")


def weight_shapes(cfg: LlamaConfig) -> list[tuple[str, tuple[int, ...]]]:
    d, q, f = cfg.d_model, cfg.qdim, cfg.ffn
    shapes = {"attn_norm": (d,), "wq": (d, q), "wk": (d, q), "wv": (d, q), "wo": (q, d),
              "ffn_norm": (d,), "w1": (d, f), "w3": (d, f), "w2": (f, d)}
    out = [("embed", (cfg.vocab, d))]
    for layer in range(cfg.layers):
        out += [(f"l{layer}.{n}", shapes[n]) for n in LAYER_WEIGHTS]
    out += [("final_norm", (d,)), ("lm_head", (d, cfg.vocab))]
    return out


def num_params(cfg: LlamaConfig) -> int:
    return sum(int(np.prod(s)) for _, s in weight_shapes(cfg))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


_INIT_CHUNK = 1 << 22  # elements per independently seeded block


def init_weights(cfg: LlamaConfig, seed: int = 0) -> list[np.ndarray]:
    """Random-init bf16 weights (as uint16 bit patterns): matrices
    0.02*N(0,1), RMSNorm gains 1.0 (the usual llama init). Each block of
    2^22 elements of tensor t draws from its own generator seeded with
    (seed, t, block), so the result does not depend on how many threads
    fill it."""
    from concurrent.futures import ThreadPoolExecutor
    import os

    out, jobs = [], []
    for t, (name, shape) in enumerate(weight_shapes(cfg)):
        if name.endswith("norm"):
            out.append(np.full(shape, 0x3F80, np.uint16))  # 1.0
            continue
        arr = np.empty(shape, np.uint16)
        out.append(arr)
        flat = arr.reshape(-1)
        for blk, lo in enumerate(range(0, flat.size, _INIT_CHUNK)):
            jobs.append((flat, lo, min(flat.size, lo + _INIT_CHUNK), (seed, t, blk)))

    def fill(job):
        flat, lo, hi, key = job
        w = np.random.default_rng(list(key)).standard_normal(hi - lo, dtype=np.float32)
        w *= np.float32(0.02)
        flat[lo:hi] = f32_to_bf16_bits(w)

    with ThreadPoolExecutor(max(1, min(16, os.cpu_count() or 1))) as ex:
        list(ex.map(fill, jobs))
    return out


def prompt_tokens(cfg: LlamaConfig, seed: int = 1) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, cfg.vocab, cfg.prompt).astype(np.int32)


def rope_inv_freq(cfg: LlamaConfig) -> np.ndarray:
    """theta^(-2i/head_dim), i < head_dim/2, computed in float64 and stored as
    an f32 constant (what a numpy-precomputed table in the model code is)."""
    i = np.arange(0, cfg.head_dim, 2, dtype=np.float64)
    return (1.0 / (cfg.theta ** (i / cfg.head_dim))).astype(np.float32)


# ----------------------------------------------------------------- programs

class _Model:
    def __init__(self, b: Builder, cfg: LlamaConfig):
        self.b, self.cfg = b, cfg
        self.w = {name: b.param(shape, "bf16") for name, shape in weight_shapes(cfg)}

    def rmsnorm(self, x: T, w: T) -> T:
        b, cfg = self.b, self.cfg
        xf = b.convert(x, "f32")
        ss = b.reduce(b.multiply(xf, xf), b.constant(0.0, "f32"), [1], "add")
        ms = b.divide(ss, b.scalar_like(float(cfg.d_model), ss))
        r = b.rsqrt(b.add(ms, b.scalar_like(cfg.eps, ms)))
        y = b.convert(b.multiply(xf, b.broadcast_in_dim(r, xf.shape, [0])), "bf16")
        return b.multiply(y, b.broadcast_in_dim(w, y.shape, [1]))

    def rope_tables(self, pos: T) -> tuple[T, T]:
        """cos/sin [T, head_dim] f32 for positions pos [T] s32."""
        b, cfg = self.b, self.cfg
        n, half = pos.shape[0], cfg.head_dim // 2
        inv = b.dense(rope_inv_freq(cfg).tolist(), "f32", (half,))
        ang = b.multiply(b.broadcast_in_dim(b.convert(pos, "f32"), (n, half), [0]),
                         b.broadcast_in_dim(inv, (n, half), [1]))
        c, s = b.cosine(ang), b.sine(ang)
        return b.concatenate([c, c], 1), b.concatenate([s, s], 1)

    def rope(self, x: T, cos: T, sin: T) -> T:
        """x [1, H, T, D] bf16: x*cos + rotate_half(x)*sin in f32, to bf16."""
        b, cfg = self.b, self.cfg
        _, h, n, d = x.shape
        half = d // 2
        xf = b.convert(x, "f32")
        x1 = b.slice(xf, [0, 0, 0, 0], [1, h, n, half])
        x2 = b.slice(xf, [0, 0, 0, half], [1, h, n, d])
        rot = b.concatenate([b.negate(x2), x1], 3)
        c = b.broadcast_in_dim(cos, xf.shape, [2, 3])
        s = b.broadcast_in_dim(sin, xf.shape, [2, 3])
        return b.convert(b.add(b.multiply(xf, c), b.multiply(rot, s)), "bf16")

    def heads(self, x: T) -> T:
        """[T, H*D] -> [1, H, T, D]."""
        cfg = self.cfg
        n = x.shape[0]
        r = self.b.reshape(x, (1, n, cfg.heads, cfg.head_dim))
        return self.b.transpose(r, [0, 2, 1, 3])

    def block(self, layer: int, x: T, pos: T, start: T, cos: T, sin: T, kc: T, vc: T):
        b, cfg = self.b, self.cfg
        w = lambda n: self.w[f"l{layer}.{n}"]  # noqa: E731
        n = x.shape[0]
        h = self.rmsnorm(x, w("attn_norm"))
        mm = lambda a, m: b.dot_general(a, m, contract=((1,), (0,)))  # noqa: E731
        q = self.rope(self.heads(mm(h, w("wq"))), cos, sin)
        k = self.rope(self.heads(mm(h, w("wk"))), cos, sin)
        v = self.heads(mm(h, w("wv")))
        zero = b.constant(0, "s32")
        kc = b.dynamic_update_slice(kc, k, [zero, zero, start, zero])
        vc = b.dynamic_update_slice(vc, v, [zero, zero, start, zero])
        s = b.dot_general(q, kc, batch=((0, 1), (0, 1)), contract=((3,), (3,)))      # [1,H,T,L]
        sf = b.convert(s, "f32")
        sf = b.multiply(sf, b.scalar_like(1.0 / math.sqrt(cfg.head_dim), sf))
        key = b.iota(sf.shape, 3)
        qpos = b.broadcast_in_dim(pos, sf.shape, [2])
        sf = b.select(b.compare("LE", key, qpos), sf, b.scalar_like(float("-inf"), sf))
        m = b.max(sf, [3])
        e = b.exp(b.subtract(sf, b.broadcast_in_dim(m, sf.shape, [0, 1, 2])))
        den = b.reduce(e, b.constant(0.0, "f32"), [3], "add")
        p = b.convert(b.divide(e, b.broadcast_in_dim(den, e.shape, [0, 1, 2])), "bf16")
        ctx = b.dot_general(p, vc, batch=((0, 1), (0, 1)), contract=((3,), (2,)))    # [1,H,T,D]
        ctx = b.reshape(b.transpose(ctx, [0, 2, 1, 3]), (n, cfg.qdim))
        x = b.add(x, mm(ctx, w("wo")))
        h = self.rmsnorm(x, w("ffn_norm"))
        g = b.convert(mm(h, w("w1")), "f32")
        act = b.multiply(b.convert(b.multiply(g, b.logistic(g)), "bf16"), mm(h, w("w3")))
        x = b.add(x, mm(act, w("w2")))
        return x, kc, vc

    def forward(self, tokens: T, pos: T, start: T, caches: list[T]):
        b, cfg = self.b, self.cfg
        n = tokens.shape[0]
        wrapped = b.select(b.compare("LT", tokens, b.scalar_like(0, tokens)),
                           b.add(tokens, b.scalar_like(cfg.vocab, tokens)), tokens)
        x = b.gather(self.w["embed"], b.reshape(wrapped, (n, 1)), offset_dims=[1], collapsed_slice_dims=[0],
                     start_index_map=[0], index_vector_dim=1, slice_sizes=[1, cfg.d_model])
        cos, sin = self.rope_tables(pos)
        new_caches = []
        for layer in range(cfg.layers):
            x, kc, vc = self.block(layer, x, pos, start, cos, sin, caches[2 * layer], caches[2 * layer + 1])
            new_caches += [kc, vc]
        last = b.slice(x, [n - 1, 0], [n, cfg.d_model]) if n > 1 else x
        h = self.rmsnorm(last, self.w["final_norm"])
        logits = b.dot_general(h, self.w["lm_head"], contract=((1,), (0,)))          # [1, vocab]
        _, tok = b.argmax(logits, 1, "s32")
        return [tok, logits] + new_caches


def cache_shape(cfg: LlamaConfig) -> tuple[int, ...]:
    return (1, cfg.heads, cfg.max_len, cfg.head_dim)


def prefill_program(cfg: LlamaConfig) -> str:
    b = Builder("jit_llama_prefill")
    m = _Model(b, cfg)
    tokens = b.param((cfg.prompt,), "s32")
    caches = [b.param(cache_shape(cfg), "bf16", donate=True) for _ in range(2 * cfg.layers)]
    pos = b.iota((cfg.prompt,), 0)
    return b.build(m.forward(tokens, pos, b.constant(0, "s32"), caches))


def decode_program(cfg: LlamaConfig) -> str:
    b = Builder("jit_llama_decode")
    m = _Model(b, cfg)
    token = b.param((1,), "s32")
    pos = b.param((), "s32")
    caches = [b.param(cache_shape(cfg), "bf16", donate=True) for _ in range(2 * cfg.layers)]
    return b.build(m.forward(token, b.reshape(pos, (1,)), pos, caches))


def generate_program(cfg: LlamaConfig, steps: int) -> str:
    """`steps` greedy decode steps in one program (a fori_loop: stablehlo.while
    over a constant count). Arguments: the weights, the token the prefill
    produced, its position, the caches (donated). Results: the `steps` tokens
    that follow, then the caches."""
    b = Builder("jit_llama_generate")
    m = _Model(b, cfg)
    token = b.param((1,), "s32")
    pos0 = b.param((), "s32")
    caches = [b.param(cache_shape(cfg), "bf16", donate=True) for _ in range(2 * cfg.layers)]
    outs0 = b.broadcast_in_dim(b.constant(0, "s32"), (steps,), [])
    n = b.constant(steps, "s32")

    def body(i, tok, *rest):
        cs, outs = list(rest[:-1]), rest[-1]
        pos = b.add(pos0, i)
        res = m.forward(tok, b.reshape(pos, (1,)), pos, cs)
        nxt, new_caches = res[0], res[2:]
        outs = b.dynamic_update_slice(outs, nxt, [i])
        return [b.add(i, b.constant(1, "s32")), nxt] + list(new_caches) + [outs]

    state = [b.constant(0, "s32"), token] + caches + [outs0]
    final = b.while_loop(state, lambda i, *rest: b.compare("LT", i, n), body)
    return b.build([final[-1]] + final[2:-1])


# ------------------------------------------------------------------ driver

class LlamaRunner:
    """Greedy generation through the plugin: one prefill execute, then one
    decode execute per token. Weights stay resident as device buffers; the
    caches are donated to each step and come back as its outputs."""

    def __init__(self, client, cfg: LlamaConfig, weights: list[np.ndarray]):
        self.client, self.cfg = client, cfg
        self.prefill = client.compile(prefill_program(cfg))
        self.decode = client.compile(decode_program(cfg))
        self.weights = [client.buffer(w, "bf16") for w in weights]
        for wb in self.weights:
            wb.block_until_ready()

    def fresh_caches(self):
        z = np.zeros(cache_shape(self.cfg), np.uint16)
        return [self.client.buffer(z, "bf16") for _ in range(2 * self.cfg.layers)]

    def start(self, prompt: np.ndarray):
        """Runs the prefill. Returns (first generated token buffer, logits
        buffer, caches)."""
        toks = self.client.buffer(np.asarray(prompt, np.int32))
        outs = self.prefill.execute_buffers(self.weights + [toks] + self.fresh_caches())
        return outs[0], outs[1], outs[2:]

    def step(self, token_buf, pos: int, caches):
        return self.step_with(token_buf, self.client.buffer(np.array(pos, np.int32)), caches)

    def step_with(self, token_buf, pos_buf, caches):
        """One decode step at the position held by `pos_buf` (a device s32
        scalar). The caches are donated; the new ones are returned."""
        outs = self.decode.execute_buffers(self.weights + [token_buf, pos_buf] + caches)
        return outs[0], outs[1], outs[2:]

    def generate_in_one_execute(self, prompt: np.ndarray, new_tokens: int):
        """Greedy decode as one prefill execute plus one execute of
        generate_program (all decode steps in an on-device loop). Returns
        (tokens int32 [new_tokens], timings dict)."""
        if not hasattr(self, "looped") or self.looped[0] != new_tokens:
            self.looped = (new_tokens, self.client.compile(generate_program(self.cfg, new_tokens - 1)))
        pos = self.client.buffer(np.array(len(prompt), np.int32))
        t0 = time.perf_counter()
        tok, _, caches = self.start(prompt)
        tok.block_until_ready()
        t1 = time.perf_counter()
        outs = self.looped[1].execute_buffers(self.weights + [tok, pos] + caches)
        outs[0].block_until_ready()
        t2 = time.perf_counter()
        rest = outs[0].to_numpy()
        toks = np.concatenate([tok.to_numpy().astype(np.int32), rest.astype(np.int32)])
        return toks, {"prefill_s": t1 - t0, "decode_s": t2 - t1, "decode_steps": new_tokens - 1}

    def generate(self, prompt: np.ndarray, new_tokens: int, keep_logits: bool = False):
        """Greedy decode of `new_tokens` tokens after `prompt`. Returns
        (tokens int32 [new_tokens], timings dict, logits list or None). The
        next token's buffer feeds the next step without a host round trip;
        tokens are read back at the end."""
        p = len(prompt)
        pos_bufs = [self.client.buffer(np.array(p + i, np.int32)) for i in range(new_tokens - 1)]
        t0 = time.perf_counter()
        tok, logits, caches = self.start(prompt)
        tok.block_until_ready()
        t1 = time.perf_counter()
        toks = [tok]
        all_logits = [logits.to_numpy()] if keep_logits else None
        for i in range(new_tokens - 1):
            tok, logits, caches = self.step_with(tok, pos_bufs[i], caches)
            toks.append(tok)
            if keep_logits:
                all_logits.append(logits.to_numpy())
        toks[-1].block_until_ready()
        t2 = time.perf_counter()
        out = np.array([int(t.to_numpy()[0]) for t in toks], np.int32)
        return out, {"prefill_s": t1 - t0, "decode_s": t2 - t1, "decode_steps": new_tokens - 1}, all_logits
