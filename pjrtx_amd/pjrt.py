"""ctypes client of the pjrtx PJRT plugin: the host-side mirror of what
jaxlib's PJRT C-API client does after ``xb.register_plugin("pjrtx", ...)``.

It dlopens ``libpjrtx_rocm_plugin.so``, calls ``GetPjrtApi`` and drives the
same PJRT calls JAX makes on the hot path: Client_Create -> BufferFromHostBuffer
-> Compile (StableHLO text, format "mlir") -> LoadedExecutable_Execute ->
Buffer_ToHostBuffer. Modelled on the reference's ctypes harness
(reference: src/plugin/pjrt/plugin_ctypes_smoke.py:103-173) and on the
CPU-vs-plugin runner (src/plugin/jax/jax_op_suite.py:98-109).

bf16 arrays are exchanged as numpy ``uint16`` holding the raw bf16 bits
(numpy has no bfloat16 and ml_dtypes is not installed); pass
``dtype="bf16"`` where a uint16 array means bf16.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import threading
from ctypes import POINTER, Structure, c_bool, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_uint, c_void_p

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = pathlib.Path(os.environ.get("PJRTX_PLUGIN_PATH", PKG / "libpjrtx_rocm_plugin.so"))

# PJRT_Buffer_Type values.
DTYPES = {
    "pred": 1, "s8": 2, "s16": 3, "s32": 4, "s64": 5, "u8": 6, "u16": 7, "u32": 8, "u64": 9,
    "f16": 10, "f32": 11, "f64": 12, "bf16": 13,
}
_NP = {
    "pred": np.bool_, "s8": np.int8, "s16": np.int16, "s32": np.int32, "s64": np.int64,
    "u8": np.uint8, "u16": np.uint16, "u32": np.uint32, "u64": np.uint64, "f16": np.float16,
    "f32": np.float32, "f64": np.float64, "bf16": np.uint16,
}
_FROM_NP = {np.dtype(v): k for k, v in _NP.items() if k not in ("bf16",)}
_CODE_TO_NAME = {v: k for k, v in DTYPES.items()}


class PjrtError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[PJRT error {code}] {message}")
        self.code = code
        self.message = message


# ----------------------------------------------------------------- structs

class ExtBase(Structure):
    pass


ExtBase._fields_ = [("struct_size", c_size_t), ("type", c_uint), ("next", POINTER(ExtBase))]


class GpuRegisterCustomCallArgs(Structure):
    """PJRT_Gpu_Register_Custom_Call_Args (include/pjrt_c_api.h)."""
    _fields_ = [("struct_size", c_size_t), ("function_name", c_char_p), ("function_name_size", c_size_t),
                ("api_version", c_int), ("handler_instantiate", c_void_p), ("handler_prepare", c_void_p),
                ("handler_initialize", c_void_p), ("handler_execute", c_void_p)]


class GpuCustomCallExtension(Structure):
    """PJRT_Gpu_Custom_Call: the extension header and its registration function."""
    _fields_ = [("base", ExtBase),
                ("custom_call", ctypes.CFUNCTYPE(c_void_p, POINTER(GpuRegisterCustomCallArgs)))]


def _args(name: str, fields: list[tuple[str, object]]):
    return type(name, (Structure,), {"_fields_": [("struct_size", c_size_t), ("extension_start", c_void_p)] + fields})


class ApiVersion(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("major_version", c_int),
                ("minor_version", c_int)]


class NamedValueUnion(ctypes.Union):
    _fields_ = [("string_value", c_char_p), ("int64_value", c_int64), ("int64_array_value", POINTER(c_int64)),
                ("float_value", c_float), ("bool_value", c_bool)]


class NamedValue(Structure):
    _anonymous_ = ("u",)
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("name", c_char_p),
                ("name_size", c_size_t), ("type", c_int), ("u", NamedValueUnion), ("value_size", c_size_t)]


ErrorDestroyArgs = _args("ErrorDestroyArgs", [("error", c_void_p)])
ErrorMessageArgs = _args("ErrorMessageArgs", [("error", c_void_p), ("message", c_void_p), ("message_size", c_size_t)])
ErrorGetCodeArgs = _args("ErrorGetCodeArgs", [("error", c_void_p), ("code", c_int)])
PluginAttributesArgs = _args("PluginAttributesArgs", [("attributes", POINTER(NamedValue)), ("num_attributes", c_size_t)])
ClientCreateArgs = _args("ClientCreateArgs", [
    ("create_options", POINTER(NamedValue)), ("num_options", c_size_t),
    ("kv_get_callback", c_void_p), ("kv_get_user_arg", c_void_p),
    ("kv_put_callback", c_void_p), ("kv_put_user_arg", c_void_p),
    ("client", c_void_p), ("kv_try_get_callback", c_void_p), ("kv_try_get_user_arg", c_void_p)])
ClientDestroyArgs = _args("ClientDestroyArgs", [("client", c_void_p)])
ClientTopologyDescriptionArgs = _args("ClientTopologyDescriptionArgs", [("client", c_void_p), ("topology", c_void_p)])
TopologySerializeArgs = _args("TopologySerializeArgs", [
    ("topology", c_void_p), ("serialized_bytes", c_void_p), ("serialized_bytes_size", c_size_t),
    ("serialized_topology", c_void_p), ("serialized_topology_deleter", ctypes.CFUNCTYPE(None, c_void_p))])
ClientPlatformNameArgs = _args("ClientPlatformNameArgs", [("client", c_void_p), ("platform_name", c_void_p),
                                                          ("platform_name_size", c_size_t)])
ClientDevicesArgs = _args("ClientDevicesArgs", [("client", c_void_p), ("devices", POINTER(c_void_p)),
                                                ("num_devices", c_size_t)])
Program = _args("Program", [("code", c_void_p), ("code_size", c_size_t), ("format", c_char_p), ("format_size", c_size_t)])
ClientCompileArgs = _args("ClientCompileArgs", [("client", c_void_p), ("program", POINTER(Program)),
                                                ("compile_options", c_char_p), ("compile_options_size", c_size_t),
                                                ("executable", c_void_p)])
BufferFromHostArgs = _args("BufferFromHostArgs", [
    ("client", c_void_p), ("data", c_void_p), ("type", c_int), ("dims", POINTER(c_int64)), ("num_dims", c_size_t),
    ("byte_strides", POINTER(c_int64)), ("num_byte_strides", c_size_t), ("host_buffer_semantics", c_int),
    ("device", c_void_p), ("memory", c_void_p), ("device_layout", c_void_p), ("done_with_host_buffer", c_void_p),
    ("buffer", c_void_p)])
ExecuteOptions = _args("ExecuteOptions", [
    ("send_callbacks", c_void_p), ("recv_callbacks", c_void_p), ("num_send_ops", c_size_t), ("num_recv_ops", c_size_t),
    ("launch_id", c_int), ("non_donatable_input_indices", POINTER(c_int64)),
    ("num_non_donatable_input_indices", c_size_t), ("context", c_void_p)])
ExecuteArgs = _args("ExecuteArgs", [
    ("executable", c_void_p), ("options", POINTER(ExecuteOptions)), ("argument_lists", POINTER(POINTER(c_void_p))),
    ("num_devices", c_size_t), ("num_args", c_size_t), ("output_lists", POINTER(POINTER(c_void_p))),
    ("device_complete_events", POINTER(c_void_p)), ("execute_device", c_void_p)])
ExecNumOutputsArgs = _args("ExecNumOutputsArgs", [("executable", c_void_p), ("num_outputs", c_size_t)])
LoadedGetExecutableArgs = _args("LoadedGetExecutableArgs", [("loaded_executable", c_void_p), ("executable", c_void_p)])
ExecutableDestroyArgs = _args("ExecutableDestroyArgs", [("executable", c_void_p)])
LoadedDestroyArgs = _args("LoadedDestroyArgs", [("executable", c_void_p)])
OptimizedProgramArgs = _args("OptimizedProgramArgs", [("executable", c_void_p), ("program", POINTER(Program))])
BufferDestroyArgs = _args("BufferDestroyArgs", [("buffer", c_void_p)])
BufferElementTypeArgs = _args("BufferElementTypeArgs", [("buffer", c_void_p), ("type", c_int)])
BufferIsDeletedArgs = _args("BufferIsDeletedArgs", [("buffer", c_void_p), ("is_deleted", ctypes.c_bool)])
BufferDimensionsArgs = _args("BufferDimensionsArgs", [("buffer", c_void_p), ("dims", POINTER(c_int64)),
                                                      ("num_dims", c_size_t)])
ToHostArgs = _args("ToHostArgs", [("src", c_void_p), ("host_layout", c_void_p), ("dst", c_void_p),
                                  ("dst_size", c_size_t), ("event", c_void_p)])
BufferReadyEventArgs = _args("BufferReadyEventArgs", [("buffer", c_void_p), ("event", c_void_p)])
EventAwaitArgs = _args("EventAwaitArgs", [("event", c_void_p)])
EventDestroyArgs = _args("EventDestroyArgs", [("event", c_void_p)])
EventIsReadyArgs = _args("EventIsReadyArgs", [("event", c_void_p), ("is_ready", c_bool)])
DeviceMemoryStatsArgs = _args("DeviceMemoryStatsArgs", [("device", c_void_p), ("bytes_in_use", c_int64)])
ShapeSpec = _args("ShapeSpec", [("dims", POINTER(c_int64)), ("num_dims", c_size_t), ("element_type", c_int)])
AsyncCreateArgs = _args("AsyncCreateArgs", [
    ("client", c_void_p), ("shape_specs", POINTER(ShapeSpec)), ("num_shape_specs", c_size_t),
    ("device_layouts", c_void_p), ("num_device_layouts", c_size_t), ("memory", c_void_p), ("transfer_manager", c_void_p)])
AsyncManagerArgs = _args("AsyncManagerArgs", [("transfer_manager", c_void_p)])
AsyncTransferDataArgs = _args("AsyncTransferDataArgs", [
    ("transfer_manager", c_void_p), ("buffer_index", c_int), ("data", c_void_p), ("offset", c_int64),
    ("transfer_size", c_int64), ("is_last_transfer", c_bool), ("done_with_h2d_transfer", c_void_p)])
AsyncRetrieveArgs = _args("AsyncRetrieveArgs", [("transfer_manager", c_void_p), ("buffer_index", c_int),
                                                ("buffer_out", c_void_p)])
AsyncCountArgs = _args("AsyncCountArgs", [("transfer_manager", c_void_p), ("buffer_count", c_size_t)])
AsyncSizeArgs = _args("AsyncSizeArgs", [("transfer_manager", c_void_p), ("buffer_index", c_int),
                                        ("buffer_size", c_size_t)])
AsyncSetErrorArgs = _args("AsyncSetErrorArgs", [
    ("transfer_manager", c_void_p), ("buffer_index", c_int), ("error_code", c_int), ("error_message", c_char_p),
    ("error_message_size", c_size_t)])

# PJRT_Api function-pointer order (include/pjrt_c_api.h).
API_FIELDS = """
Error_Destroy Error_Message Error_GetCode Plugin_Initialize Plugin_Attributes
Event_Destroy Event_IsReady Event_Error Event_Await Event_OnReady
Client_Create Client_Destroy Client_PlatformName Client_ProcessIndex Client_PlatformVersion Client_Devices
Client_AddressableDevices Client_LookupDevice Client_LookupAddressableDevice Client_AddressableMemories
Client_Compile Client_DefaultDeviceAssignment Client_BufferFromHostBuffer
DeviceDescription_Id DeviceDescription_ProcessIndex DeviceDescription_Attributes DeviceDescription_Kind
DeviceDescription_DebugString DeviceDescription_ToString
Device_GetDescription Device_IsAddressable Device_LocalHardwareId Device_AddressableMemories Device_DefaultMemory
Device_MemoryStats
Memory_Id Memory_Kind Memory_DebugString Memory_ToString Memory_AddressableByDevices
Executable_Destroy Executable_Name Executable_NumReplicas Executable_NumPartitions Executable_NumOutputs
Executable_SizeOfGeneratedCodeInBytes Executable_GetCostAnalysis Executable_OutputMemoryKinds
Executable_OptimizedProgram Executable_Serialize
LoadedExecutable_Destroy LoadedExecutable_GetExecutable LoadedExecutable_AddressableDevices LoadedExecutable_Delete
LoadedExecutable_IsDeleted LoadedExecutable_Execute Executable_DeserializeAndLoad LoadedExecutable_Fingerprint
Buffer_Destroy Buffer_ElementType Buffer_Dimensions Buffer_UnpaddedDimensions Buffer_DynamicDimensionIndices
Buffer_GetMemoryLayout Buffer_OnDeviceSizeInBytes Buffer_Device Buffer_Memory Buffer_Delete Buffer_IsDeleted
Buffer_CopyToDevice Buffer_ToHostBuffer Buffer_IsOnCpu Buffer_ReadyEvent Buffer_UnsafePointer
Buffer_IncreaseExternalReferenceCount Buffer_DecreaseExternalReferenceCount Buffer_OpaqueDeviceMemoryDataPointer
CopyToDeviceStream_Destroy CopyToDeviceStream_AddChunk CopyToDeviceStream_TotalBytes CopyToDeviceStream_GranuleSize
CopyToDeviceStream_CurrentBytes
TopologyDescription_Create TopologyDescription_Destroy TopologyDescription_PlatformName
TopologyDescription_PlatformVersion TopologyDescription_GetDeviceDescriptions TopologyDescription_Serialize
TopologyDescription_Attributes
Compile
Executable_OutputElementTypes Executable_OutputDimensions Buffer_CopyToMemory Client_CreateViewOfDeviceBuffer
Executable_Fingerprint Client_TopologyDescription Executable_GetCompiledMemoryStats Memory_Kind_Id
ExecuteContext_Create ExecuteContext_Destroy Buffer_CopyRawToHost AsyncHostToDeviceTransferManager_Destroy
AsyncHostToDeviceTransferManager_TransferData Client_CreateBuffersForAsyncHostToDevice
AsyncHostToDeviceTransferManager_RetrieveBuffer AsyncHostToDeviceTransferManager_Device
AsyncHostToDeviceTransferManager_BufferCount AsyncHostToDeviceTransferManager_BufferSize
AsyncHostToDeviceTransferManager_SetBufferError AsyncHostToDeviceTransferManager_AddMetadata
Client_DmaMap Client_DmaUnmap
""".split()


class Api(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("pjrt_api_version", ApiVersion)] + [
        ("PJRT_" + n, c_void_p) for n in API_FIELDS]


def _mk(args: Structure) -> Structure:
    args.struct_size = ctypes.sizeof(args)
    return args


# ------------------------------------------------------------------ plugin

_lock = threading.Lock()
_plugin: "Plugin | None" = None


def load_library(path: pathlib.Path | str | None = None) -> ctypes.CDLL:
    p = pathlib.Path(path or LIB_PATH)
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is not built; run `python -m pjrtx_amd.build` (or __graft_entry__.build()) first")
    return ctypes.CDLL(str(p))


class Plugin:
    """Loaded plugin library plus its PJRT_Api table."""

    def __init__(self, path: pathlib.Path | str | None = None):
        self.lib = load_library(path)
        get = self.lib.GetPjrtApi
        get.restype = c_void_p
        get.argtypes = []
        ptr = get()
        if not ptr:
            raise RuntimeError("GetPjrtApi returned null")
        self.api = ctypes.cast(ptr, POINTER(Api)).contents
        self._fns: dict[str, object] = {}
        self._setup_hip_abi()

    def _setup_hip_abi(self) -> None:
        L = self.lib
        L.pjrtx_hip_last_error.restype = c_char_p
        for name, argtypes in {
            "pjrtx_plan_json": [c_char_p, c_size_t, c_char_p, c_size_t, POINTER(c_size_t)],
            "pjrtx_kernel_source": [c_char_p, c_size_t, c_char_p, c_size_t, POINTER(c_size_t)],
            "pjrtx_compile_check": [c_char_p, c_size_t, c_char_p, POINTER(c_size_t)],
            "pjrtx_hip_device_count": [POINTER(c_int)],
            "pjrtx_executable_time_steps": [c_void_p, POINTER(c_void_p), c_size_t, c_int, POINTER(c_double), c_size_t,
                                            POINTER(c_size_t)],
            "pjrtx_executable_step_names": [c_void_p, c_char_p, c_size_t, POINTER(c_size_t)],
            "pjrtx_executable_graph_stats": [c_void_p, POINTER(c_int64)],
            "pjrtx_executable_run": [c_void_p, POINTER(c_void_p), c_size_t, c_int, POINTER(c_double)],
            "pjrtx_executable_run_pjrt": [c_void_p, POINTER(c_void_p), c_size_t, c_int, POINTER(c_double)],
            "pjrtx_executable_stats": [c_void_p, POINTER(c_int64)],
            "pjrtx_compile_cache_stats": [POINTER(c_int64), POINTER(c_int64), POINTER(c_int64)],
            "pjrtx_compile_cache_usage": [POINTER(c_int64), POINTER(c_int64)],
            "pjrtx_mfma_peak_tflops": [c_int, c_int, POINTER(c_double)],
            "pjrtx_compile_fingerprint": [c_char_p, c_size_t, c_char_p, c_size_t, POINTER(c_size_t)],
            "pjrtx_set_max_resident_bytes": [c_int, c_int64],
            "pjrtx_residency_stats": [c_int, POINTER(c_int64)],
            "pjrtx_hip_malloc": [c_int, c_size_t, POINTER(c_void_p)],
            "pjrtx_hip_free": [c_int, c_void_p],
            "pjrtx_hip_copy_h2d": [c_int, c_void_p, c_void_p, c_size_t],
            "pjrtx_hip_copy_d2h": [c_int, c_void_p, c_void_p, c_size_t],
            "pjrtx_hip_synchronize": [c_int],
            "pjrtx_executable_execute_noalloc": [c_void_p, c_int, POINTER(c_void_p), c_size_t, POINTER(c_void_p),
                                                 c_size_t, POINTER(c_size_t)],
        }.items():
            f = getattr(L, name)
            f.argtypes = argtypes
            f.restype = c_int
        L.pjrtx_noalloc_scratch_bytes.argtypes = []
        L.pjrtx_noalloc_scratch_bytes.restype = c_size_t

    def hip_check(self, rc: int) -> None:
        if rc != 0:
            raise PjrtError(rc, self.lib.pjrtx_hip_last_error().decode(errors="replace"))

    def call(self, name: str, args: Structure) -> None:
        fn = self._fns.get(name)
        if fn is None:
            raw = getattr(self.api, "PJRT_" + name)
            if not raw:
                raise PjrtError(12, f"PJRT_{name} is not installed")
            proto = ctypes.CFUNCTYPE(c_void_p, POINTER(type(args)))
            fn = proto(raw)
            self._fns[name] = fn
        err = fn(ctypes.byref(args))
        if err:
            raise self._error(err)

    def _error(self, err: int) -> PjrtError:
        m = _mk(ErrorMessageArgs())
        m.error = err
        ctypes.CFUNCTYPE(None, POINTER(ErrorMessageArgs))(self.api.PJRT_Error_Message)(ctypes.byref(m))
        msg = ctypes.string_at(m.message, m.message_size).decode(errors="replace") if m.message else ""
        c = _mk(ErrorGetCodeArgs())
        c.error = err
        ctypes.CFUNCTYPE(c_void_p, POINTER(ErrorGetCodeArgs))(self.api.PJRT_Error_GetCode)(ctypes.byref(c))
        d = _mk(ErrorDestroyArgs())
        d.error = err
        ctypes.CFUNCTYPE(None, POINTER(ErrorDestroyArgs))(self.api.PJRT_Error_Destroy)(ctypes.byref(d))
        return PjrtError(c.code, msg)

    # Custom-call targets (include/pjrtx_custom_call.h; host only).
    def _cc_call(self, fn, *names: bytes) -> None:
        argv = []
        for n in names:
            argv += [n, len(n) if n is not None else 0]
        fn.restype = c_void_p
        err = fn(*argv)
        if err:
            raise self._error(err)

    def register_custom_call_identity(self, target: str) -> None:
        self._cc_call(self.lib.PjRTx_RegisterCustomCallIdentity, target.encode())

    def register_custom_call_unary(self, target: str, op: str) -> None:
        self._cc_call(self.lib.PjRTx_RegisterCustomCallUnary, target.encode(), op.encode())

    def register_custom_call_binary(self, target: str, op: str) -> None:
        self._cc_call(self.lib.PjRTx_RegisterCustomCallBinary, target.encode(), op.encode())

    def unregister_custom_call(self, target: str) -> None:
        b = target.encode()
        self.lib.PjRTx_UnregisterCustomCall.argtypes = [c_char_p, c_size_t]
        self.lib.PjRTx_UnregisterCustomCall.restype = None
        self.lib.PjRTx_UnregisterCustomCall(b, len(b))

    def gpu_custom_call_extension(self):
        """The PJRT GPU custom-call extension from PJRT_Api.extension_start's
        chain (type 0), or None."""
        ext = ctypes.cast(self.api.extension_start, POINTER(ExtBase)) if self.api.extension_start else None
        while ext:
            if ext.contents.type == 0:
                return ctypes.cast(ext, POINTER(GpuCustomCallExtension)).contents
            ext = ext.contents.next
        return None

    def register_custom_call_handler(self, target: str, handler: int, api_version: int = 0,
                                     struct_size: int | None = None) -> None:
        """PJRT_Gpu_Register_Custom_Call through the extension; `handler` is the
        handler_execute address (a PjRTx_CustomCall_* marker)."""
        ext = self.gpu_custom_call_extension()
        if ext is None:
            raise PjrtError(12, "PJRT GPU custom-call extension not found")
        b = target.encode()
        a = GpuRegisterCustomCallArgs(struct_size=struct_size or ctypes.sizeof(GpuRegisterCustomCallArgs),
                                      function_name=b, function_name_size=len(b), api_version=api_version,
                                      handler_execute=handler)
        err = ext.custom_call(ctypes.byref(a))
        if err:
            raise self._error(err)

    def marker(self, name: str) -> int:
        """Address of a PjRTx_CustomCall_* marker handler."""
        return ctypes.cast(getattr(self.lib, name), c_void_p).value

    # Host-only compiler entry points (no GPU needed).
    def plan_json(self, text: str) -> str:
        return self._string_call(self.lib.pjrtx_plan_json, text)

    def kernel_source(self, text: str) -> str:
        return self._string_call(self.lib.pjrtx_kernel_source, text)

    def compile_check(self, text: str, arch: str = "gfx950") -> int:
        b = text.encode()
        n = c_size_t(0)
        self.hip_check(self.lib.pjrtx_compile_check(b, len(b), arch.encode(), ctypes.byref(n)))
        return n.value

    def _string_call(self, fn, text: str) -> str:
        b = text.encode()
        need = c_size_t(0)
        self.hip_check(fn(b, len(b), None, 0, ctypes.byref(need)))
        buf = ctypes.create_string_buffer(need.value)
        self.hip_check(fn(b, len(b), buf, need.value, ctypes.byref(need)))
        return buf.value.decode()

    def attributes(self) -> dict:
        a = _mk(PluginAttributesArgs())
        self.call("Plugin_Attributes", a)
        out = {}
        for i in range(a.num_attributes):
            nv = a.attributes[i]
            name = ctypes.string_at(nv.name, nv.name_size).decode()
            if nv.type == 0:
                out[name] = ctypes.string_at(nv.string_value, nv.value_size).decode()
            elif nv.type == 1:
                out[name] = nv.int64_value
            elif nv.type == 2:
                out[name] = [nv.int64_array_value[k] for k in range(nv.value_size)]
        return out

    def device_count(self) -> int:
        n = c_int(0)
        self.hip_check(self.lib.pjrtx_hip_device_count(ctypes.byref(n)))
        return n.value

    def compile_cache_stats(self) -> dict:
        """{"hits", "misses", "entries"} of the process's compile cache."""
        h, m, e = c_int64(0), c_int64(0), c_int64(0)
        self.hip_check(self.lib.pjrtx_compile_cache_stats(ctypes.byref(h), ctypes.byref(m), ctypes.byref(e)))
        b, ev = c_int64(0), c_int64(0)
        self.hip_check(self.lib.pjrtx_compile_cache_usage(ctypes.byref(b), ctypes.byref(ev)))
        return {"hits": h.value, "misses": m.value, "entries": e.value, "bytes": b.value, "evictions": ev.value}

    def compile_fingerprint(self, text: str) -> str:
        """The compile-cache key of `text` under the current PJRTX_* environment."""
        raw = text.encode()
        buf = ctypes.create_string_buffer(64)
        need = c_size_t(0)
        self.hip_check(self.lib.pjrtx_compile_fingerprint(raw, len(raw), buf, 64, ctypes.byref(need)))
        return buf.value.decode()

    def mfma_peak_tflops(self, device: int = 0, shape: int = 0) -> float:
        """Measured dense bf16 MFMA throughput (shape 0: 16x16x32, 1: 32x32x16)."""
        out = c_double(0.0)
        self.hip_check(self.lib.pjrtx_mfma_peak_tflops(device, shape, ctypes.byref(out)))
        return out.value

    def set_max_resident_bytes(self, device: int, nbytes: int) -> None:
        """Caps the device memory loaded executables hold (0: no cap)."""
        self.hip_check(self.lib.pjrtx_set_max_resident_bytes(device, nbytes))

    def residency_stats(self, device: int = 0) -> dict:
        out = (c_int64 * 6)()
        self.hip_check(self.lib.pjrtx_residency_stats(device, out))
        keys = ("resident_bytes", "peak_resident_bytes", "entries", "evictions", "evicted_bytes", "max_resident_bytes")
        return dict(zip(keys, list(out)))


def plugin() -> Plugin:
    global _plugin
    with _lock:
        if _plugin is None:
            _plugin = Plugin()
        return _plugin


# ------------------------------------------------------------------ client

def np_dtype_name(a: np.ndarray, dtype: str | None) -> str:
    if dtype:
        return dtype
    return _FROM_NP[a.dtype]


class Buffer:
    def __init__(self, client: "Client", handle: int):
        self.client = client
        self.handle = handle

    @property
    def dtype(self) -> str:
        a = _mk(BufferElementTypeArgs())
        a.buffer = self.handle
        self.client.p.call("Buffer_ElementType", a)
        return _CODE_TO_NAME[a.type]

    @property
    def shape(self) -> tuple[int, ...]:
        a = _mk(BufferDimensionsArgs())
        a.buffer = self.handle
        self.client.p.call("Buffer_Dimensions", a)
        return tuple(a.dims[i] for i in range(a.num_dims))

    def block_until_ready(self) -> "Buffer":
        a = _mk(BufferReadyEventArgs())
        a.buffer = self.handle
        self.client.p.call("Buffer_ReadyEvent", a)
        ev = a.event
        try:
            w = _mk(EventAwaitArgs())
            w.event = ev
            self.client.p.call("Event_Await", w)
        finally:
            d = _mk(EventDestroyArgs())
            d.event = ev
            self.client.p.call("Event_Destroy", d)
        return self

    def to_numpy(self) -> np.ndarray:
        dt = self.dtype
        out = np.empty(self.shape, dtype=_NP[dt])
        a = _mk(ToHostArgs())
        a.src = self.handle
        a.dst = out.ctypes.data if out.nbytes else None
        a.dst_size = out.nbytes
        if out.nbytes == 0:
            return out
        self.client.p.call("Buffer_ToHostBuffer", a)
        if a.event:
            w = _mk(EventAwaitArgs())
            w.event = a.event
            self.client.p.call("Event_Await", w)
            d = _mk(EventDestroyArgs())
            d.event = a.event
            self.client.p.call("Event_Destroy", d)
        return out

    def is_deleted(self) -> bool:
        """PJRT_Buffer_IsDeleted: true after Delete or after the buffer was
        donated to an execution."""
        if not self.handle:
            return True
        a = _mk(BufferIsDeletedArgs())
        a.buffer = self.handle
        self.client.p.call("Buffer_IsDeleted", a)
        return bool(a.is_deleted)

    def delete_memory(self) -> None:
        """PJRT_Buffer_Delete: gives the device memory back; the handle
        stays valid (is_deleted() turns true) until delete()."""
        if self.handle:
            a = _mk(BufferDestroyArgs())   # same layout as PJRT_Buffer_Delete_Args
            a.buffer = self.handle
            self.client.p.call("Buffer_Delete", a)

    def delete(self) -> None:
        """PJRT_Buffer_Destroy: releases the handle (and its memory)."""
        if self.handle:
            a = _mk(BufferDestroyArgs())
            a.buffer = self.handle
            self.client.p.call("Buffer_Destroy", a)
            self.handle = None

    def __del__(self):
        try:
            self.delete()
        except Exception:
            pass


class Executable:
    def __init__(self, client: "Client", handle: int, text: str):
        self.client = client
        self.handle = handle
        self.text = text
        a = _mk(LoadedGetExecutableArgs())
        a.loaded_executable = handle
        client.p.call("LoadedExecutable_GetExecutable", a)
        n = _mk(ExecNumOutputsArgs())
        n.executable = a.executable
        client.p.call("Executable_NumOutputs", n)
        self.num_outputs = n.num_outputs
        self._exe_view = a.executable

    def optimized_program(self) -> str:
        prog = _mk(Program())
        a = _mk(OptimizedProgramArgs())
        a.executable = self._exe_view
        a.program = ctypes.pointer(prog)
        self.client.p.call("Executable_OptimizedProgram", a)
        buf = ctypes.create_string_buffer(prog.code_size)
        prog.code = ctypes.cast(buf, c_void_p)
        self.client.p.call("Executable_OptimizedProgram", a)
        return buf.raw[: prog.code_size].decode()

    def execute_buffers(self, args: list[Buffer], non_donatable: list[int] | None = None) -> list[Buffer]:
        """PJRT_LoadedExecutable_Execute on one device. Arguments whose
        parameters are marked donated (and not listed in `non_donatable`)
        are consumed: their buffers read as deleted afterwards."""
        p = self.client.p
        arg_arr = (c_void_p * max(1, len(args)))(*[b.handle for b in args])
        arg_lists = (POINTER(c_void_p) * 1)(ctypes.cast(arg_arr, POINTER(c_void_p)))
        out_arr = (c_void_p * max(1, self.num_outputs))()
        out_lists = (POINTER(c_void_p) * 1)(ctypes.cast(out_arr, POINTER(c_void_p)))
        events = (c_void_p * 1)()
        opts = _mk(ExecuteOptions())
        if non_donatable:
            nd = (c_int64 * len(non_donatable))(*non_donatable)
            opts.non_donatable_input_indices = nd
            opts.num_non_donatable_input_indices = len(non_donatable)
        a = _mk(ExecuteArgs())
        a.executable = self.handle
        a.options = ctypes.pointer(opts)
        a.argument_lists = arg_lists
        a.num_devices = 1
        a.num_args = len(args)
        a.output_lists = out_lists
        a.device_complete_events = events
        p.call("LoadedExecutable_Execute", a)
        if events[0]:
            d = _mk(EventDestroyArgs())
            d.event = events[0]
            p.call("Event_Destroy", d)
        return [Buffer(self.client, out_arr[i]) for i in range(self.num_outputs)]

    def __call__(self, *arrays, dtypes: list[str | None] | None = None) -> list[np.ndarray]:
        dtypes = dtypes or [None] * len(arrays)
        bufs = [a if isinstance(a, Buffer) else self.client.buffer(a, dt) for a, dt in zip(arrays, dtypes)]
        outs = self.execute_buffers(bufs)
        return [o.to_numpy() for o in outs]

    def time_steps(self, args: list[Buffer], iters: int = 20) -> list[float]:
        L = self.client.p.lib
        arr = (c_void_p * max(1, len(args)))(*[b.handle for b in args])
        cap = 4096
        ms = (c_double * cap)()
        n = c_size_t(0)
        self.client.p.hip_check(L.pjrtx_executable_time_steps(self.handle, arr, len(args), iters, ms, cap,
                                                              ctypes.byref(n)))
        return [ms[i] for i in range(n.value)]

    def run_loop(self, args: list[Buffer], iters: int) -> float:
        """Wall ms of `iters` back-to-back executions run by the plugin's own
        loop (pjrtx_executable_run), synchronized on both sides."""
        L = self.client.p.lib
        arr = (c_void_p * max(1, len(args)))(*[b.handle for b in args])
        ms = c_double(0.0)
        self.client.p.hip_check(L.pjrtx_executable_run(self.handle, arr, len(args), iters, ctypes.byref(ms)))
        return ms.value

    def run_loop_pjrt(self, args: list[Buffer], iters: int) -> float:
        """Wall ms of `iters` executions, each a PJRT_LoadedExecutable_Execute
        through the plugin's C API table with its event and output buffers
        destroyed after it (pjrtx_executable_run_pjrt), synchronized on both
        sides."""
        L = self.client.p.lib
        arr = (c_void_p * max(1, len(args)))(*[b.handle for b in args])
        ms = c_double(0.0)
        self.client.p.hip_check(L.pjrtx_executable_run_pjrt(self.handle, arr, len(args), iters, ctypes.byref(ms)))
        return ms.value

    def execute_noalloc(self, arg_ptrs: list[int], out_ptrs: list[int], device: int = 0) -> int:
        """pjrtx_executable_execute_noalloc on raw device addresses (from
        DeviceArray); queued on the device stream. Returns the bytes of the
        fixed no-allocation block the call used."""
        L = self.client.p.lib
        a = (c_void_p * max(1, len(arg_ptrs)))(*arg_ptrs)
        o = (c_void_p * max(1, len(out_ptrs)))(*out_ptrs)
        used = c_size_t(0)
        self.client.p.hip_check(L.pjrtx_executable_execute_noalloc(self.handle, device, a, len(arg_ptrs), o,
                                                                   len(out_ptrs), ctypes.byref(used)))
        return used.value

    def step_names(self) -> list[str]:
        L = self.client.p.lib
        need = c_size_t(0)
        self.client.p.hip_check(L.pjrtx_executable_step_names(self.handle, None, 0, ctypes.byref(need)))
        buf = ctypes.create_string_buffer(need.value)
        self.client.p.hip_check(L.pjrtx_executable_step_names(self.handle, buf, need.value, ctypes.byref(need)))
        return [s for s in buf.value.decode().split("\n") if s]

    def graph_stats(self) -> dict:
        out = (c_int64 * 2)()
        self.client.p.hip_check(self.client.p.lib.pjrtx_executable_graph_stats(self.handle, out))
        return dict(captures=out[0], replays=out[1])

    def stats(self) -> dict:
        out = (c_int64 * 4)()
        self.client.p.hip_check(self.client.p.lib.pjrtx_executable_stats(self.handle, out))
        return dict(executions=out[0], kernel_launches=out[1], library_calls=out[2], released_values=out[3])

    def __del__(self):
        try:
            p = self.client.p
            d = _mk(ExecutableDestroyArgs())
            d.executable = self._exe_view
            p.call("Executable_Destroy", d)
            a = _mk(LoadedDestroyArgs())
            a.executable = self.handle
            p.call("LoadedExecutable_Destroy", a)
        except Exception:
            pass


class Client:
    """A PJRT client of the pjrtx platform on the visible GPU(s)."""

    def __init__(self, backend: str = "rocm", plugin_: Plugin | None = None):
        self.p = plugin_ or plugin()
        opt_name = b"pjrtx_backend"
        opt_val = backend.encode()
        nv = NamedValue()
        nv.struct_size = ctypes.sizeof(NamedValue)
        nv.name = opt_name
        nv.name_size = len(opt_name)
        nv.type = 0
        nv.string_value = opt_val
        nv.value_size = len(opt_val)
        self._keep = (opt_name, opt_val, nv)
        a = _mk(ClientCreateArgs())
        a.create_options = ctypes.pointer(nv)
        a.num_options = 1
        self.p.call("Client_Create", a)
        self.handle = a.client
        d = _mk(ClientDevicesArgs())
        d.client = self.handle
        self.p.call("Client_Devices", d)
        self.devices = [d.devices[i] for i in range(d.num_devices)]

    def topology_serialized(self) -> str:
        """PJRT_Client_TopologyDescription, then PJRT_TopologyDescription_Serialize
        (the bytes copied, the serialized topology freed by its deleter)."""
        t = _mk(ClientTopologyDescriptionArgs())
        t.client = self.handle
        self.p.call("Client_TopologyDescription", t)
        a = _mk(TopologySerializeArgs())
        a.topology = t.topology
        self.p.call("TopologyDescription_Serialize", a)
        out = ctypes.string_at(a.serialized_bytes, a.serialized_bytes_size).decode()
        a.serialized_topology_deleter(a.serialized_topology)
        return out

    @property
    def platform_name(self) -> str:
        a = _mk(ClientPlatformNameArgs())
        a.client = self.handle
        self.p.call("Client_PlatformName", a)
        return ctypes.string_at(a.platform_name, a.platform_name_size).decode()

    def buffer(self, array: np.ndarray, dtype: str | None = None) -> Buffer:
        arr = np.ascontiguousarray(array)
        if np.ndim(array) == 0:
            arr = arr.reshape(())  # ascontiguousarray promotes scalars to 1-d
        name = np_dtype_name(arr, dtype)
        if name == "pred":
            arr = arr.astype(np.uint8)
        dims = (c_int64 * max(1, arr.ndim))(*arr.shape)
        a = _mk(BufferFromHostArgs())
        a.client = self.handle
        a.data = arr.ctypes.data if arr.nbytes else None
        a.type = DTYPES[name]
        a.dims = dims
        a.num_dims = arr.ndim
        a.byte_strides = None
        a.num_byte_strides = 0
        a.host_buffer_semantics = 0
        a.device = self.devices[0]
        self.p.call("Client_BufferFromHostBuffer", a)
        if a.done_with_host_buffer:
            d = _mk(EventDestroyArgs())
            d.event = a.done_with_host_buffer
            self.p.call("Event_Destroy", d)
        return Buffer(self, a.buffer)

    def compile(self, text: str, compile_options: bytes = b"") -> Executable:
        code = text.encode()
        cbuf = ctypes.create_string_buffer(code, len(code))
        prog = _mk(Program())
        prog.code = ctypes.cast(cbuf, c_void_p)
        prog.code_size = len(code)
        prog.format = b"mlir"
        prog.format_size = 4
        a = _mk(ClientCompileArgs())
        a.client = self.handle
        a.program = ctypes.pointer(prog)
        a.compile_options = compile_options
        a.compile_options_size = len(compile_options)
        self.p.call("Client_Compile", a)
        return Executable(self, a.executable, text)

    def async_transfer(self, specs: list[tuple[tuple, str]]) -> AsyncTransfer:
        return AsyncTransfer(self, specs)

    def bytes_in_use(self) -> int:
        a = _mk(DeviceMemoryStatsArgs())
        a.device = self.devices[0]
        self.p.call("Device_MemoryStats", a)
        return a.bytes_in_use

    def close(self) -> None:
        if self.handle:
            a = _mk(ClientDestroyArgs())
            a.client = self.handle
            self.p.call("Client_Destroy", a)
            self.handle = None


class AsyncTransfer:
    """PJRT_Client_CreateBuffersForAsyncHostToDevice and the transfer
    manager's calls: device buffers of the given (shape, dtype) filled by
    `transfer` chunks in any order."""

    def __init__(self, client: "Client", specs: list[tuple[tuple, str]]):
        self.client = client
        self._dims = [(c_int64 * max(1, len(shape)))(*shape) for shape, _ in specs]
        arr = (ShapeSpec * max(1, len(specs)))()
        for i, (shape, dt) in enumerate(specs):
            _mk(arr[i])
            arr[i].dims = self._dims[i]
            arr[i].num_dims = len(shape)
            arr[i].element_type = DTYPES[dt]
        a = _mk(AsyncCreateArgs())
        a.client = client.handle
        a.shape_specs = arr
        a.num_shape_specs = len(specs)
        client.p.call("Client_CreateBuffersForAsyncHostToDevice", a)
        self.handle = a.transfer_manager

    def count(self) -> int:
        a = _mk(AsyncCountArgs())
        a.transfer_manager = self.handle
        self.client.p.call("AsyncHostToDeviceTransferManager_BufferCount", a)
        return a.buffer_count

    def size(self, i: int) -> int:
        a = _mk(AsyncSizeArgs())
        a.transfer_manager = self.handle
        a.buffer_index = i
        self.client.p.call("AsyncHostToDeviceTransferManager_BufferSize", a)
        return a.buffer_size

    def buffer(self, i: int) -> Buffer:
        a = _mk(AsyncRetrieveArgs())
        a.transfer_manager = self.handle
        a.buffer_index = i
        self.client.p.call("AsyncHostToDeviceTransferManager_RetrieveBuffer", a)
        return Buffer(self.client, a.buffer_out)

    def transfer(self, i: int, data: bytes | np.ndarray, offset: int, last: bool) -> None:
        """Copies `data` to bytes [offset, offset + len) of buffer i and
        waits until the host copy may be reused."""
        raw = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, bytes) else data).view(np.uint8)
        a = _mk(AsyncTransferDataArgs())
        a.transfer_manager = self.handle
        a.buffer_index = i
        a.data = raw.ctypes.data if raw.size else None
        a.offset = offset
        a.transfer_size = raw.size
        a.is_last_transfer = last
        self.client.p.call("AsyncHostToDeviceTransferManager_TransferData", a)
        if a.done_with_h2d_transfer:
            w = _mk(EventAwaitArgs())
            w.event = a.done_with_h2d_transfer
            self.client.p.call("Event_Await", w)
            d = _mk(EventDestroyArgs())
            d.event = a.done_with_h2d_transfer
            self.client.p.call("Event_Destroy", d)

    def set_error(self, i: int, code: int, message: str) -> None:
        msg = message.encode()
        a = _mk(AsyncSetErrorArgs())
        a.transfer_manager = self.handle
        a.buffer_index = i
        a.error_code = code
        a.error_message = msg
        a.error_message_size = len(msg)
        self.client.p.call("AsyncHostToDeviceTransferManager_SetBufferError", a)

    def close(self) -> None:
        if self.handle:
            a = _mk(AsyncManagerArgs())
            a.transfer_manager = self.handle
            self.client.p.call("AsyncHostToDeviceTransferManager_Destroy", a)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceArray:
    """Raw device memory from pjrtx_hip_malloc (caller-owned, for the
    allocation-free execute): `ptr` is the device address."""

    def __init__(self, plugin_: Plugin, nbytes: int, device: int = 0):
        self.p, self.nbytes, self.device = plugin_, int(nbytes), device
        ptr = c_void_p(0)
        self.p.hip_check(self.p.lib.pjrtx_hip_malloc(device, max(1, self.nbytes), ctypes.byref(ptr)))
        self.ptr = ptr.value

    @classmethod
    def from_numpy(cls, plugin_: Plugin, a: np.ndarray, device: int = 0) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(plugin_, a.nbytes, device)
        if a.nbytes:
            d.p.hip_check(d.p.lib.pjrtx_hip_copy_h2d(device, d.ptr, a.ctypes.data, a.nbytes))
        return d

    def to_numpy(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes == self.nbytes
        if out.nbytes:
            self.p.hip_check(self.p.lib.pjrtx_hip_copy_d2h(self.device, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            self.p.hip_check(self.p.lib.pjrtx_hip_free(self.device, self.ptr))
            self.ptr = None


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits (round to nearest even), as uint16."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
