"""Custom-call target registration without a GPU: the PJRT GPU custom-call
extension on PJRT_Api.extension_start, the PjRTx_* exports, and the lowering
of registered targets to elementwise ops with the reference's legality rules
(reference: src/plugin/custom_call.zig:35-185, the walk of the extension chain
in src/plugin/pjrt/plugin_ctypes_smoke.py:117-147,
src/backend/mlx_metal/custom_call.zig:155-238 and its two tests at :241-293,
lowering_custom_call.zig:17-215)."""
import json
import pathlib
import re

import pytest

from pjrtx_amd.hlo import Builder
from pjrtx_amd.pjrt import PjrtError

ROOT = pathlib.Path(__file__).resolve().parents[1]
INVALID, UNIMPLEMENTED = 3, 12


def plan(plugin, text):
    return json.loads(plugin.plan_json(text))


def one_call(target, n_in=1, dtype="f32", out_dtype=None, shape=(8, 16)):
    b = Builder()
    xs = [b.param(shape, dtype) for _ in range(n_in)]
    return b.build([b.custom_call(target, xs, shape, out_dtype or dtype)])


def ops_of(p):
    return [o for s in p["steps"] for o in s.get("ops", [])]


def test_header_declares_what_the_library_exports(plugin):
    text = (ROOT / "include" / "pjrtx_custom_call.h").read_text()
    names = re.findall(r"PJRTX_CC_API\s+[\w\s\*]+?\b(PjRTx_\w+)\s*\(", text)
    assert len(names) == 7
    for n in names:
        assert hasattr(plugin.lib, n), n


def test_extension_chain_holds_the_gpu_custom_call_extension(plugin):
    ext = plugin.gpu_custom_call_extension()
    assert ext is not None
    assert ext.base.type == 0 and ext.base.struct_size >= 24 and ext.custom_call
    # The three marker handlers are distinct functions.
    marks = {plugin.marker(n) for n in ("PjRTx_CustomCall_Identity", "PjRTx_CustomCall_UnarySqrt",
                                        "PjRTx_CustomCall_BinaryAdd")}
    assert len(marks) == 3


def test_unregistered_target_is_unimplemented(plugin):
    with pytest.raises(PjrtError) as e:
        plan(plugin, one_call("pjrtx.test.never_registered"))
    assert e.value.code == UNIMPLEMENTED and "custom_call" in e.value.message


def test_registry_lowers_and_unregisters(plugin):
    t = "pjrtx.test.cc.dynamic"
    plugin.unregister_custom_call(t)
    v0 = plugin.compile_fingerprint(one_call(t))
    plugin.register_custom_call_unary(t, "exp")
    try:
        p = plan(plugin, one_call(t))
        assert ops_of(p) == ["exponential"] or "exponential" in ops_of(p)
        # the registry is part of the executable-cache key
        assert plugin.compile_fingerprint(one_call(t)) != v0
        plugin.register_custom_call_binary(t, "maximum")  # replaces the registration
        assert "maximum" in ops_of(plan(plugin, one_call(t, n_in=2)))
    finally:
        plugin.unregister_custom_call(t)
    with pytest.raises(PjrtError) as e:
        plan(plugin, one_call(t, n_in=2))
    assert e.value.code == UNIMPLEMENTED


def test_extension_registers_by_marker(plugin):
    t_sqrt, t_add, t_id = "pjrtx.test.cc.sqrt", "pjrtx.test.cc.add", "pjrtx.test.cc.id"
    try:
        plugin.register_custom_call_handler(t_sqrt, plugin.marker("PjRTx_CustomCall_UnarySqrt"))
        plugin.register_custom_call_handler(t_add, plugin.marker("PjRTx_CustomCall_BinaryAdd"))
        plugin.register_custom_call_handler(t_id, plugin.marker("PjRTx_CustomCall_Identity"))
        assert "sqrt" in ops_of(plan(plugin, one_call(t_sqrt)))
        assert "add" in ops_of(plan(plugin, one_call(t_add, n_in=2)))
        p = plan(plugin, one_call(t_id))
        assert all(s["kind"] == "alias" for s in p["steps"])  # the output is its input
    finally:
        for t in (t_sqrt, t_add, t_id):
            plugin.unregister_custom_call(t)


@pytest.mark.parametrize("how,code", [
    ("api_version", UNIMPLEMENTED),   # only the untyped API version 0
    ("foreign_handler", UNIMPLEMENTED),
    ("null_handler", INVALID),
    ("small_struct", INVALID),
])
def test_extension_registration_errors(plugin, how, code):
    h = plugin.marker("PjRTx_CustomCall_BinaryAdd")
    kw = {}
    if how == "api_version":
        kw["api_version"] = 1
    elif how == "foreign_handler":
        h = plugin.marker("GetPjrtApi")
    elif how == "null_handler":
        h = None
    else:
        kw["struct_size"] = 16
    with pytest.raises(PjrtError) as e:
        plugin.register_custom_call_handler("pjrtx.test.cc.bad", h, **kw)
    assert e.value.code == code


def test_registration_rejects_empty_target_and_unknown_ops(plugin):
    for fn, args in [(plugin.register_custom_call_identity, ("",)),
                     (plugin.register_custom_call_unary, ("pjrtx.test.cc.x", "bogus")),
                     (plugin.register_custom_call_binary, ("pjrtx.test.cc.x", "exp"))]:
        with pytest.raises(PjrtError) as e:
            fn(*args)
        assert e.value.code == INVALID


def test_builtin_targets(plugin):
    # annotate_device_placement is an identity; the built-in f32 add takes f32
    # tensors only.
    p = plan(plugin, one_call("annotate_device_placement", dtype="bf16"))
    assert all(s["kind"] == "alias" for s in p["steps"])
    assert "add" in ops_of(plan(plugin, one_call("pjrtx.mlx_metal.custom_binary_add_f32", n_in=2)))
    with pytest.raises(PjrtError) as e:
        plan(plugin, one_call("pjrtx.mlx_metal.custom_binary_add_f32", n_in=2, dtype="f16"))
    assert e.value.code == INVALID


@pytest.mark.parametrize("kind,op,n_in,dtype,out_dtype", [
    ("unary", "sqrt", 1, "s32", None),         # floating op on an integer
    ("unary", "popcnt", 1, "f32", None),       # integer op on a float
    ("unary", "is_finite", 1, "f32", "f32"),   # must produce pred
    ("unary", "exp", 2, "f32", None),          # arity
    ("binary", "shift_left", 2, "f32", None),  # shifts take integers
    ("binary", "atan2", 2, "s32", None),       # atan2 takes floats
    ("binary", "add", 1, "f32", None),         # arity
    ("binary", "add", 2, "f32", "f16"),        # output dtype
    ("identity", None, 1, "f32", "f16"),       # identity keeps the dtype
])
def test_lowering_legality(plugin, kind, op, n_in, dtype, out_dtype):
    t = "pjrtx.test.cc.legality"
    if kind == "unary":
        plugin.register_custom_call_unary(t, op)
    elif kind == "binary":
        plugin.register_custom_call_binary(t, op)
    else:
        plugin.register_custom_call_identity(t)
    try:
        with pytest.raises(PjrtError) as e:
            plan(plugin, one_call(t, n_in=n_in, dtype=dtype, out_dtype=out_dtype))
        assert e.value.code == INVALID
    finally:
        plugin.unregister_custom_call(t)


def test_is_finite_and_logical_ops_lower(plugin):
    t1, t2 = "pjrtx.test.cc.isfinite", "pjrtx.test.cc.xor"
    plugin.register_custom_call_unary(t1, "is_finite")
    plugin.register_custom_call_binary(t2, "xor")
    try:
        assert "is_finite" in ops_of(plan(plugin, one_call(t1, out_dtype="pred")))
        assert "xor" in ops_of(plan(plugin, one_call(t2, n_in=2, dtype="pred")))
        assert "xor" in ops_of(plan(plugin, one_call(t2, n_in=2, dtype="u8")))
    finally:
        plugin.unregister_custom_call(t1)
        plugin.unregister_custom_call(t2)
