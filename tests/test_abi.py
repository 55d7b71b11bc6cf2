"""The plugin library loads, exports every symbol its headers declare, and its
PJRT table / ctypes mirror agree — without a GPU (no compute calls)."""
import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def header_functions(name: str) -> list[str]:
    text = (ROOT / "include" / name).read_text()
    return re.findall(r"PJRTX_HIP_API\s+[\w\s\*]+?\b(pjrtx_\w+)\s*\(", text)


def test_exports_every_declared_symbol(plugin):
    lib = plugin.lib
    names = header_functions("pjrtx_hip.h")
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/pjrtx_hip.h but not exported"
    assert hasattr(lib, "GetPjrtApi")


def test_pjrt_table_layout_matches_header(plugin):
    from pjrtx_amd.pjrt import Api
    api = plugin.api
    assert api.struct_size == ctypes.sizeof(Api)
    assert api.pjrt_api_version.major_version == 0
    assert api.pjrt_api_version.minor_version > 0
    # Every slot is populated (unimplemented families answer UNIMPLEMENTED).
    for field, _ in Api._fields_[3:]:
        assert getattr(api, field), f"{field} is null"


def test_plugin_attributes(plugin):
    attrs = plugin.attributes()
    assert attrs["stablehlo_current_version"] == [1, 16, 0]
    assert attrs["stablehlo_minimum_version"] == [1, 0, 0]
    assert "xla_version" in attrs


def test_client_create_fails_closed_without_gpu(plugin):
    from pjrtx_amd.pjrt import Client, PjrtError
    if plugin.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(PjrtError) as e:
        Client()
    assert e.value.code == 9  # FAILED_PRECONDITION
    assert "no HIP device" in e.value.message


def test_unknown_client_option_rejected(plugin):
    from pjrtx_amd.pjrt import Client, PjrtError
    with pytest.raises(PjrtError) as e:
        Client(backend="metal_mlx")
    assert e.value.code in (3, 9)


def test_unimplemented_slot_returns_error(plugin):
    from pjrtx_amd.pjrt import PjrtError, _args, _mk
    Args = _args("SerializeArgs", [("executable", ctypes.c_void_p)])
    with pytest.raises(PjrtError) as e:
        plugin.call("Executable_Serialize", _mk(Args()))
    assert e.value.code == 12


def test_compile_fingerprint_needs_no_gpu(plugin, monkeypatch):
    """The compile-cache key: stable for a text, different for another text
    or another PJRTX_* environment (the switches change plans)."""
    from pjrtx_amd.hlo import Builder
    b = Builder("jit_fp")
    x = b.param((8, 16), "f32")
    text = b.build([b.sum(x, [1])])
    f1 = plugin.compile_fingerprint(text)
    assert f1.startswith("pjrtx-") and len(f1) == 38 and f1 == plugin.compile_fingerprint(text)
    assert plugin.compile_fingerprint(text + " ") != f1
    monkeypatch.setenv("PJRTX_GEMV_FUSION", "0")
    assert plugin.compile_fingerprint(text) != f1


def test_residency_setters_reject_bad_devices(plugin):
    """Without a GPU the residency calls fail with an error code, not a crash."""
    if plugin.device_count() > 0:
        pytest.skip("covered by the GPU residency tests")
    with pytest.raises(Exception):
        plugin.set_max_resident_bytes(0, 1 << 20)
