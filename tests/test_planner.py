"""Host-side tests of the StableHLO importer, the fusion planner and the
kernel generator (no GPU). Structural counterparts of the reference's planner
tests (reference: src/backend/mlx_metal/program_fusion.zig:116-227,
executable_metal_graph_lowering_tests.zig:8-204)."""
import json

import pytest

from pjrtx_amd import programs
from pjrtx_amd.hlo import Builder
from pjrtx_amd.pjrt import PjrtError


def plan(plugin, text):
    return json.loads(plugin.plan_json(text))


def test_c1_is_one_fused_reduction(plugin):
    p = plan(plugin, programs.c1_elementwise_rowsum(64, 256))
    assert len(p["steps"]) == 1
    s = p["steps"][0]
    assert s["kind"] == "reduce" and s["reducers"] == ["sum"]
    # the whole elementwise chain is the reduction's prologue
    for op in ("multiply", "add", "tanh", "maximum", "subtract"):
        assert op in s["ops"]
    assert s["inputs"] == [0, 1]  # x and y read once; splat constants inlined
    assert p["constants"] == []


def test_c2_siblings_fuse_into_one_kernel(plugin):
    p = plan(plugin, programs.c2_argmax_f16_reductions(64, 128256))
    assert len(p["steps"]) == 1
    s = p["steps"][0]
    assert sorted(s["reducers"]) == ["argmax", "max", "min", "sum"]
    assert s["epilogue"] == ["convert"]  # f32 sum -> f16 inside the kernel
    assert s["inputs"] == [0]            # iota synthesized, not read
    assert len(s["outputs"]) == 5
    assert s["splits"] > 1 and s["grid"] >= 256  # 64 rows spread over the chip


def test_full_reduce_and_middle_axis(plugin):
    b = Builder()
    x = b.param((2, 3, 4), "f32")
    s_all = b.sum(x, [0, 1, 2])
    s_mid = b.sum(x, [1])
    m = b.max(x, [0, 2])
    p = plan(plugin, b.build([s_all, s_mid, m]))
    kinds = [st["kind"] for st in p["steps"]]
    assert kinds == ["reduce", "reduce", "reduce"]
    assert all(not st["row_schedule"] for st in p["steps"])


def test_multi_use_cheap_value_is_recomputed(plugin, monkeypatch):
    # softmax-like: exp(x - max) feeds both the sum and the divide (row
    # fusion off, so that the three passes stay separate steps).
    monkeypatch.setenv("PJRTX_ROW_FUSE_MAX", "0")
    b = Builder()
    x = b.param((8, 128), "f32")
    mx = b.max(x, [1])
    sh = b.subtract(x, b.broadcast_in_dim(mx, (8, 128), [0]))
    e = b.exp(sh)
    s = b.sum(e, [1])
    out = b.divide(e, b.broadcast_in_dim(s, (8, 128), [0]))
    p = plan(plugin, b.build([out]))
    kinds = [st["kind"] for st in p["steps"]]
    assert kinds == ["reduce", "reduce", "loop"]
    # exp is evaluated inside both the second reduction and the final loop
    assert "exponential" in p["steps"][1]["ops"] and "exponential" in p["steps"][2]["ops"]


def _softmax(b, x, via=None):
    mx = b.max(x, [1])
    if via is not None:
        mx = via(mx)
    e = b.exp(b.subtract(x, b.broadcast_in_dim(mx, x.shape, [0])))
    s = b.sum(e, [1])
    return b.divide(e, b.broadcast_in_dim(s, x.shape, [0]))


def test_softmax_is_one_row_kernel(plugin):
    b = Builder()
    x = b.param((8, 128), "f32")
    p = plan(plugin, b.build([_softmax(b, x)]))
    assert [st["kind"] for st in p["steps"]] == ["rowfused"]
    assert p["steps"][0]["phases"] == 3 and p["steps"][0]["rows"] == 8 and p["steps"][0]["row_len"] == 128
    # the row max and sum stay in registers: only the softmax output is stored
    assert len(p["steps"][0]["outputs"]) == 1


def test_row_fusion_refuses_reindexed_row_values(plugin):
    # the max is reversed before it is broadcast: row r would need row 7-r's
    # value, so the phases cannot share one workgroup per row.
    b = Builder()
    x = b.param((8, 128), "f32")
    p = plan(plugin, b.build([_softmax(b, x, via=lambda m: b.reverse(m, [0]))]))
    # max stays its own reduction; sum -> divide still fuse (the reversed max
    # is read from memory there, like any input).
    assert [st["kind"] for st in p["steps"]] == ["reduce", "rowfused"]
    assert p["steps"][0]["reducers"] == ["max"] and p["steps"][1]["phases"] == 2


def test_liveness_releases_intermediates(plugin, monkeypatch):
    monkeypatch.setenv("PJRTX_ROW_FUSE_MAX", "0")  # keep the max as a buffer between two steps
    b = Builder()
    x = b.param((4, 256), "f32")
    mx = b.max(x, [1])
    y = b.subtract(x, b.broadcast_in_dim(mx, (4, 256), [0]))
    s = b.sum(b.exp(y), [1])
    p = plan(plugin, b.build([s]))
    released = [v for st in p["steps"] for v in st["release_after"]]
    assert released, "the max intermediate must be released after its last use"


def test_reshape_of_materialized_value_is_alias(plugin):
    b = Builder()
    x = b.param((4, 6), "f32")
    s = b.sum(x, [1])
    r = b.reshape(s, (2, 2))
    p = plan(plugin, b.build([r]))
    assert [st["kind"] for st in p["steps"]] == ["reduce", "alias"]


def test_unsupported_op_fails_closed(plugin):
    text = """module @m {
  func.func public @main(%arg0: tensor<4xf32>) -> tensor<4xf32> {
    %0 = stablehlo.custom_call @foo(%arg0) : (tensor<4xf32>) -> tensor<4xf32>
    return %0 : tensor<4xf32>
  }
}"""
    with pytest.raises(PjrtError) as e:
        plugin.plan_json(text)
    assert e.value.code == 12 and "custom_call" in e.value.message


def test_parse_error_reports_line(plugin):
    text = "module @m {\n  func.func public @main(%arg0: tensor<4xf32>) -> tensor<4xf32> {\n    return %zz : tensor<4xf32>\n  }\n}"
    with pytest.raises(PjrtError) as e:
        plugin.plan_json(text)
    assert e.value.code == 3 and "line 3" in e.value.message


def test_private_function_calls_are_inlined(plugin):
    text = """module @jit_f attributes {mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32} {
  func.func public @main(%arg0: tensor<8xf32>) -> (tensor<8xf32> {jax.result_info = ""}) {
    %0 = call @relu(%arg0) : (tensor<8xf32>) -> tensor<8xf32>
    %1 = call @relu(%0) : (tensor<8xf32>) -> tensor<8xf32>
    return %1 : tensor<8xf32>
  }
  func.func private @relu(%arg0: tensor<8xf32>) -> tensor<8xf32> {
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = stablehlo.broadcast_in_dim %cst, dims = [] : (tensor<f32>) -> tensor<8xf32>
    %1 = stablehlo.maximum %arg0, %0 : tensor<8xf32>
    return %1 : tensor<8xf32>
  }
}"""
    p = plan(plugin, text)
    assert len(p["steps"]) == 1 and p["steps"][0]["kind"] == "loop"
    assert p["steps"][0]["ops"].count("maximum") == 2


def test_multi_partition_module_rejected_at_compile(plugin):
    text = programs.c1_elementwise_rowsum(4, 64).replace("mhlo.num_partitions = 1", "mhlo.num_partitions = 2")
    # planning alone accepts it; the PJRT compile path rejects (one device)
    plan(plugin, text)


@pytest.mark.parametrize("text_fn", [
    lambda: programs.c1_elementwise_rowsum(64, 256),
    lambda: programs.c2_argmax_f16_reductions(4, 1024),
    lambda: programs.c2_argmax_f16_reductions(64, 128256),
])
def test_generated_kernels_compile_for_gfx950(plugin, text_fn):
    assert plugin.compile_check(text_fn(), "gfx950") > 0


def test_generated_code_has_no_packed_f32(plugin):
    src = plugin.kernel_source(programs.c1_elementwise_rowsum(64, 256))
    assert "v_pk_" not in src
    assert "pjrtx_fusion_reduce_0" in src


def test_decode_dots_sharing_an_lhs_form_groups(plugin, monkeypatch):
    from pjrtx_amd import llama_like as L
    steps = plan(plugin, L.decode_program(L.TINY))["steps"]
    groups = [s["members"] for s in steps if s["kind"] == "gemv" and s["members"] > 1]
    assert groups == [3, 2] * L.TINY.layers  # q/k/v and gate/up of every layer
    monkeypatch.setenv("PJRTX_GEMV_FUSION", "0")
    steps = plan(plugin, L.decode_program(L.TINY))["steps"]
    groups = [s["group_size"] for s in steps if s.get("library") == "dot_group"]
    assert groups == [3, 2] * L.TINY.layers
    monkeypatch.setenv("PJRTX_DOT_GROUPS", "0")
    assert not [s for s in plan(plugin, L.decode_program(L.TINY))["steps"] if s.get("library") == "dot_group"]


def test_dot_group_refuses_a_member_that_depends_on_another(plugin):
    b = Builder()
    x = b.param((1, 64), "bf16")
    w = b.param((64, 64), "bf16")
    y = b.dot_general(x, w, contract=((1,), (0,)))
    w2 = b.multiply(w, b.broadcast_in_dim(b.reshape(y, (64,)), (64, 64), [1]))  # depends on the first dot
    z = b.dot_general(x, w2, contract=((1,), (0,)))
    steps = plan(plugin, b.build([y, z]))["steps"]
    assert "dot_group" not in [s.get("library") for s in steps]


def test_residual_add_merges_into_decode_dot(plugin, monkeypatch):
    from pjrtx_amd import llama_like as L
    steps = plan(plugin, L.decode_program(L.FULL))["steps"]
    merged = [s for s in steps if "residual_add" in s]
    assert len(merged) >= 2 * L.FULL.layers - 1  # o-proj and down-proj residuals
    assert all(s["kind"] == "gemv" for s in merged)
    monkeypatch.setenv("PJRTX_GEMV_FUSION", "0")
    steps = plan(plugin, L.decode_program(L.FULL))["steps"]
    merged = [s for s in steps if "residual_add" in s]
    assert len(merged) >= 2 * L.FULL.layers - 1
    assert all(s.get("library") == "dot_general" for s in merged)
    monkeypatch.setenv("PJRTX_DOT_RESIDUAL", "0")
    assert not [s for s in plan(plugin, L.decode_program(L.FULL))["steps"] if "residual_add" in s]


def test_decode_layer_is_five_launches(plugin):
    """Per layer: q/k/v GEMV (RMSNorm prologue, RoPE and both KV-row writes
    in its epilogue), attention, o-projection (+ residual), gate/up GEMV
    (RMSNorm prologue, SwiGLU epilogue), down projection (+ residual)."""
    from pjrtx_amd import llama_like as L
    steps = plan(plugin, L.decode_program(L.FULL))["steps"]
    units = [s for s in steps if s["kind"] != "alias"]
    gemv = [s for s in steps if s["kind"] == "gemv"]
    assert len(gemv) == 4 * L.FULL.layers + 1  # + lm_head
    qkv = [s for s in gemv if s["members"] == 3]
    assert len(qkv) == L.FULL.layers
    for s in qkv:
        assert s["prologue"] == "rowfused" and s["joint"] and s["seg_cols"] == L.FULL.head_dim
        assert "concatenate" in s["epilogue_loop"] and len(s["window_outputs"]) == 2
    up = [s for s in gemv if s["members"] == 2]
    assert all(s["prologue"] == "rowfused" and "logistic" in s["epilogue_loop"] for s in up)
    assert gemv[-1]["prologue"] == "rowfused" and gemv[-1]["N"] == [L.FULL.vocab]  # final norm + lm_head
    assert len(units) <= 5 * L.FULL.layers + 5
    # Every split GEMV folds in-launch (no combine kernel).
    assert all(s["direct"] or s["fused_combine"] for s in gemv)
    # The attention writes its 10 key splits' partials and the o-projection
    # merges them while staging its input.
    attn = [s for s in steps if s.get("library") == "attention"]
    assert len(attn) == L.FULL.layers and all(s["partials_out"] for s in attn)
    oproj = [s for s in gemv if s.get("attention_splits_merged")]
    assert len(oproj) == L.FULL.layers
    assert all(s["attention_splits_merged"] == 10 and s["members"] == 1 and "residual_add" in s for s in oproj)


def test_attention_merge_stays_in_attention_without_splits_or_when_off(plugin, monkeypatch):
    """40-slot caches give one key split: nothing to merge, the attention
    writes its rows. PJRTX_ATTN_MERGE_GEMV=0 keeps the merge in the attention
    launch."""
    from pjrtx_amd import llama_like as L
    steps = plan(plugin, L.decode_program(L.TINY))["steps"]
    assert not any(s.get("partials_out") or s.get("attention_splits_merged") for s in steps)
    monkeypatch.setenv("PJRTX_ATTN_MERGE_GEMV", "0")
    steps = plan(plugin, L.decode_program(L.FULL))["steps"]
    assert not any(s.get("partials_out") or s.get("attention_splits_merged") for s in steps)


def test_gemv_epilogue_must_stay_inside_segments(plugin):
    """A loop that reads a result across the whole row (a reverse) cannot
    run per segment: it stays its own launch."""
    b = Builder()
    x = b.param((1, 256), "bf16")
    w = b.param((256, 1024), "bf16")
    y = b.dot_general(x, w, contract=((1,), (0,)))
    z = b.multiply(b.reverse(y, [1]), y)
    steps = plan(plugin, b.build([z]))["steps"]
    assert [s["kind"] for s in steps] == ["gemv", "loop"]
    # Elementwise over the same index fuses.
    steps = plan(plugin, b.build([b.multiply(y, y)]))["steps"]
    assert [s["kind"] for s in steps] == ["gemv"] and steps[0]["epilogue_loop"] == ["multiply"]


def _shift_in_place_program():
    # c donated; c[0:7] = -c[1:8] written back into c (a roll-like shift).
    b = Builder()
    c = b.param((8, 16), "f32", donate=True)
    u = b.negate(b.slice(c, [1, 0], [8, 16]))
    z = b.constant(0, "s32")
    return b.build([b.dynamic_update_slice(c, u, [z, z])])


def test_window_write_not_absorbed_into_kernel_reading_operand(plugin):
    # The kernel computing the update reads the operand at other rows than it
    # would write: fusing the window write would race across workgroups.
    steps = plan(plugin, _shift_in_place_program())["steps"]
    assert not any(s.get("window_outputs") for s in steps)
    dus = [s for s in steps if s.get("library") == "dynamic_update_slice"]
    assert len(dus) == 1


@pytest.mark.parametrize("dt", ["s8", "u8", "s16", "u16", "s32", "u32", "s64", "u64"])
def test_popcnt_and_clz_kernels_compile_at_every_width(plugin, dt):
    """Generated popcnt / count_leading_zeros code compiles (hiprtc, no GPU)
    for every integer width (the 32-bit popcnt once emitted an extra ')')."""
    b = Builder()
    x = b.param((4, 8), dt)
    assert plugin.compile_check(b.build([b.popcnt(x), b.clz(x)])) > 0


def _wrapped_gather(vocab, dim, n, idx_dtype="s32", add_value=None):
    """table[idx] as jnp indexing lowers it (select(i < 0, i + add, i)), with
    `add` the table's row count unless given."""
    b = Builder()
    table = b.param((vocab, dim), "bf16")
    idx = b.param((n,), idx_dtype)
    add = vocab if add_value is None else add_value
    wrapped = b.select(b.compare("LT", idx, b.scalar_like(0, idx)), b.add(idx, b.scalar_like(add, idx)), idx)
    iv = b.broadcast_in_dim(wrapped, (n, 1), [0])
    return b.build([b.gather(table, iv, offset_dims=[1], collapsed_slice_dims=[0], start_index_map=[0],
                             index_vector_dim=1, slice_sizes=[1, dim])])


@pytest.mark.parametrize("idx_dtype", ["s32", "s64"])
def test_gather_index_wrap_folds_into_the_gather(plugin, monkeypatch, idx_dtype):
    # the normalization's loop kernel goes away: the gather reads the raw
    # indices through a view and applies i < 0 ? i + rows : i itself
    p = plan(plugin, _wrapped_gather(1000, 64, 16, idx_dtype))
    assert [st["kind"] for st in p["steps"]] == ["alias", "library"]
    assert p["steps"][0]["inputs"] == [1]
    monkeypatch.setenv("PJRTX_GATHER_WRAP", "0")
    p = plan(plugin, _wrapped_gather(1000, 64, 16, idx_dtype))
    kinds = [st["kind"] for st in p["steps"]]
    assert kinds == ["loop", "library"] and "select" in p["steps"][0]["ops"]


def test_gather_index_wrap_needs_the_row_count(plugin):
    # a wrap by anything but the gathered dimension's size is not JAX's
    # normalization and stays an elementwise kernel
    p = plan(plugin, _wrapped_gather(1000, 64, 16, add_value=999))
    assert [st["kind"] for st in p["steps"]] == ["loop", "library"]
