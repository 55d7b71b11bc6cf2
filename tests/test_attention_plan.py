"""Host-side tests of the fused-attention rewrite (attention.cc): the
scaled-dot-product-attention custom call of the reference
(src/backend/mlx_metal/custom_call.zig:119-150, legality rules of
lowering_custom_call.zig:216-300) and the unfused softmax-attention pattern
become one `attention` library step; everything else stays as it was."""
import dataclasses
import json

import pytest

from pjrtx_amd import llama_like as L
from pjrtx_amd import programs
from pjrtx_amd.hlo import Builder
from pjrtx_amd.pjrt import PjrtError

SDPA = "pjrtx.mlx_metal.scaled_dot_product_attention"


def plan(plugin, text):
    return json.loads(plugin.plan_json(text))


def kinds(p):
    return [s.get("library") or s["kind"] for s in p["steps"]]


def test_c3_attention_is_one_step(plugin, monkeypatch):
    p = plan(plugin, programs.c3_attention(2, 4, 256, 128))
    assert kinds(p) == ["attention"]
    s = p["steps"][0]
    assert s["causal"] and s["q_coef"] == 1 and s["offset"] == 0 and not s["offset_operand"]
    assert s["scale"] == 1.0 and s["inputs"] == [0, 1, 2] and s["flops"] == 4 * 2 * 4 * 256 * 256 * 128
    assert s["effective_flops"] == 4 * 2 * 4 * 128 * (256 * 257 // 2)  # causal: query i reads i + 1 keys
    monkeypatch.setenv("PJRTX_FUSED_ATTENTION", "0")
    assert kinds(plan(plugin, programs.c3_attention(2, 4, 256, 128))) == ["dot_general", "rowfused", "dot_general"]


def test_llama_prefill_fuses_every_layer(plugin):
    cfg = dataclasses.replace(L.TINY, prompt=20)  # 20 queries per head: worth fusing
    pre = plan(plugin, L.prefill_program(cfg))
    att = [s for s in pre["steps"] if s.get("library") == "attention"]
    assert len(att) == L.TINY.layers
    for s in att:
        assert s["causal"] and s["q_coef"] == 1 and s["offset"] == 0 and not s["offset_operand"]
        assert abs(s["scale"] - 1 / L.TINY.head_dim ** 0.5) < 1e-7  # an f32 constant in the program
    assert "rowfused" not in [s["kind"] for s in pre["steps"] if s.get("row_len") == L.TINY.max_len]


def test_llama_decode_fuses_every_layer(plugin):
    dec = plan(plugin, L.decode_program(L.TINY))
    att = [s for s in dec["steps"] if s.get("library") == "attention"]
    assert len(att) == L.TINY.layers
    for s in att:  # key <= pos, pos read on the device
        assert s["causal"] and s["q_coef"] == 0 and s["offset"] == 0 and s["offset_operand"] and len(s["inputs"]) == 4


def test_decode_mask_reads_position_on_device(plugin):
    """The decode step's mask (key <= pos, pos a program argument) as a
    pattern with 16 queries: q_coef 0 and the position as a 4th operand."""
    b = Builder()
    shp, L_ = (1, 2, 16, 64), 48
    q, kc, vc = b.param(shp, "bf16"), b.param((1, 2, L_, 64), "bf16"), b.param((1, 2, L_, 64), "bf16")
    pos = b.param((), "s32")
    s = b.dot_general(q, kc, batch=((0, 1), (0, 1)), contract=((3,), (3,)))
    sf = b.multiply(b.convert(s, "f32"), b.scalar_like(0.125, b.convert(s, "f32")))
    key = b.iota(sf.shape, 3)
    qpos = b.broadcast_in_dim(b.reshape(pos, (1,)), sf.shape, [2])
    sf = b.select(b.compare("LE", key, qpos), sf, b.scalar_like(float("-inf"), sf))
    m = b.max(sf, [3])
    e = b.exp(b.subtract(sf, b.broadcast_in_dim(m, sf.shape, [0, 1, 2])))
    z = b.sum(e, [3])
    p = b.convert(b.divide(e, b.broadcast_in_dim(z, sf.shape, [0, 1, 2])), "bf16")
    ctx = b.dot_general(p, vc, batch=((0, 1), (0, 1)), contract=((3,), (2,)))
    st = plan(plugin, b.build([ctx]))["steps"]
    att = [x for x in st if x.get("library") == "attention"]
    assert len(att) == 1 and att[0]["q_coef"] == 0 and att[0]["offset_operand"] and len(att[0]["inputs"]) == 4
    assert att[0]["scale"] == 0.125


def _attention_graph(mask=None, extra_output=False, scale_bf16=False):
    b = Builder()
    shp = (1, 2, 32, 64)
    q, k, v = b.param(shp, "bf16"), b.param(shp, "bf16"), b.param(shp, "bf16")
    s = b.dot_general(q, k, batch=((0, 1), (0, 1)), contract=((3,), (3,)))
    if scale_bf16:
        s = b.multiply(s, b.scalar_like(0.5, s))
    sf = b.convert(s, "f32")
    if mask is not None:
        row, col = b.iota((32, 32), 0), b.iota((32, 32), 1)
        keep = b.broadcast_in_dim(mask(b, row, col), sf.shape, [2, 3])
        sf = b.select(keep, sf, b.scalar_like(float("-inf"), sf))
    m = b.max(sf, [3])
    e = b.exp(b.subtract(sf, b.broadcast_in_dim(m, sf.shape, [0, 1, 2])))
    z = b.sum(e, [3])
    p = b.convert(b.divide(e, b.broadcast_in_dim(z, sf.shape, [0, 1, 2])), "bf16")
    ctx = b.dot_general(p, v, batch=((0, 1), (0, 1)), contract=((3,), (2,)))
    return b.build([ctx, s] if extra_output else [ctx])


def test_mask_forms(plugin):
    # no mask
    s = plan(plugin, _attention_graph())["steps"]
    assert kinds({"steps": s}) == ["attention"] and not s[0]["causal"]
    # key < query  ->  key <= query - 1
    s = plan(plugin, _attention_graph(lambda b, r, c: b.compare("LT", c, r)))["steps"]
    assert s[0]["causal"] and s[0]["q_coef"] == 1 and s[0]["offset"] == -1
    # query + 3 >= key
    s = plan(plugin, _attention_graph(
        lambda b, r, c: b.compare("GE", b.add(r, b.scalar_like(3, r)), c)))["steps"]
    assert s[0]["offset"] == 3 and s[0]["q_coef"] == 1
    # a mask the kernel cannot express (key >= query) stays unfused
    assert "attention" not in kinds(plan(plugin, _attention_graph(lambda b, r, c: b.compare("GE", c, r))))


def test_pattern_with_other_uses_or_bf16_scaling_stays_unfused(plugin):
    assert "attention" not in kinds(plan(plugin, _attention_graph(extra_output=True)))
    assert "attention" not in kinds(plan(plugin, _attention_graph(scale_bf16=True)))


def _sdpa(dt="bf16", qs=(5, 4, 64), kvs=(9, 2, 64), tok=("s32", ()), out=None, generic=False):
    b = Builder()
    q, k, v = b.param(qs, dt), b.param(kvs, dt), b.param(kvs, dt)
    t = b.param(tok[1], tok[0])
    o = b.custom_call(SDPA, [q, k, v, t], out or qs, dt, generic=generic)
    return b.build([o])


@pytest.mark.parametrize("generic", [False, True])
def test_sdpa_custom_call_lowers(plugin, generic):
    s = plan(plugin, _sdpa(generic=generic))["steps"]
    assert kinds({"steps": s}) == ["attention"]
    assert s[0]["layout"] == 2 and s[0]["offset_operand"] and abs(s[0]["scale"] - 0.125) < 1e-12
    s = plan(plugin, _sdpa(qs=(2, 5, 4, 64), kvs=(2, 9, 2, 64), tok=("u32", (1,))))["steps"]
    assert s[0]["layout"] == 1


@pytest.mark.parametrize("kw", [
    dict(dt="f64"),
    dict(qs=(5, 64), kvs=(9, 64)),
    dict(kvs=(9, 3, 64)),                    # 4 query heads over 3 kv heads
    dict(kvs=(9, 2, 32)),                    # head dims differ
    dict(tok=("f32", ())),
    dict(tok=("s32", (2,))),
    dict(out=(5, 4, 32)),
])
def test_sdpa_custom_call_legality(plugin, kw):
    with pytest.raises(PjrtError) as e:
        plugin.plan_json(_sdpa(**kw))
    assert e.value.code == 3 and "attention custom_call" in e.value.message


def test_attention_kernels_build(plugin):
    assert plugin.compile_check(programs.c3_attention(1, 2, 128, 64), "gfx950") == 0  # library step: no fusion kernel
