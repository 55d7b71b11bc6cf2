/*
 * pjrt_c_api.h — this project's own restatement of the public PJRT C API
 * (OpenXLA, Apache-2.0): the type names, struct field order and function
 * pointer order of `PJRT_Api` that a PJRT plugin must present so that jaxlib's
 * PJRT C-API client can dlopen it and call `GetPjrtApi()`.
 *
 * The reference plugin takes these definitions from the XLA header pinned in
 * its build (reference: src/plugin/BUILD.bazel:63-91, third_party/xla/repo.bzl,
 * consumed as `c.PJRT_*` in src/plugin/api.zig:58-85). That header is not on
 * this machine, so the layout below is written from the published API; every
 * struct starts with `struct_size` + `extension_start`, and the plugin checks
 * `struct_size` of each Args struct it receives before reading a field, which
 * is how PJRT versions its ABI.
 *
 * Only the families the pjrtx hot path uses carry full Args definitions; the
 * other table slots keep their position with opaque Args types so that the
 * function-pointer order of PJRT_Api is preserved up to the last slot listed.
 */
#ifndef PJRTX_AMD_PJRT_C_API_H_
#define PJRTX_AMD_PJRT_C_API_H_

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PJRT_STRUCT_SIZE(struct_type, last_field) \
  (offsetof(struct_type, last_field) + sizeof(((struct_type*)0)->last_field))

#define PJRT_API_MAJOR 0
#define PJRT_API_MINOR 67

/* ------------------------------- Extensions ------------------------------ */

typedef enum {
  PJRT_Extension_Type_Gpu_Custom_Call = 0,
  PJRT_Extension_Type_Profiler,
  PJRT_Extension_Type_Custom_Partitioner,
  PJRT_Extension_Type_Stream,
  PJRT_Extension_Type_Layouts,
  PJRT_Extension_Type_FFI,
  PJRT_Extension_Type_MemoryDescriptions,
} PJRT_Extension_Type;

typedef struct PJRT_Extension_Base {
  size_t struct_size;
  PJRT_Extension_Type type;
  struct PJRT_Extension_Base* next;
} PJRT_Extension_Base;
#define PJRT_Extension_Base_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Extension_Base, next)

typedef struct PJRT_Api_Version {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  int major_version;
  int minor_version;
} PJRT_Api_Version;
#define PJRT_Api_Version_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Api_Version, minor_version)

/* ------------------------------ Opaque handles --------------------------- */

typedef struct PJRT_Error PJRT_Error;
typedef struct PJRT_Client PJRT_Client;
typedef struct PJRT_Device PJRT_Device;
typedef struct PJRT_DeviceDescription PJRT_DeviceDescription;
typedef struct PJRT_Memory PJRT_Memory;
typedef struct PJRT_Executable PJRT_Executable;
typedef struct PJRT_LoadedExecutable PJRT_LoadedExecutable;
typedef struct PJRT_Buffer PJRT_Buffer;
typedef struct PJRT_Event PJRT_Event;
typedef struct PJRT_TopologyDescription PJRT_TopologyDescription;
typedef struct PJRT_ExecuteContext PJRT_ExecuteContext;
typedef struct PJRT_CopyToDeviceStream PJRT_CopyToDeviceStream;
typedef struct PJRT_SerializedExecutable PJRT_SerializedExecutable;
typedef struct PJRT_AsyncHostToDeviceTransferManager PJRT_AsyncHostToDeviceTransferManager;

/* --------------------------------- Errors -------------------------------- */

typedef enum {
  PJRT_Error_Code_CANCELLED = 1,
  PJRT_Error_Code_UNKNOWN = 2,
  PJRT_Error_Code_INVALID_ARGUMENT = 3,
  PJRT_Error_Code_DEADLINE_EXCEEDED = 4,
  PJRT_Error_Code_NOT_FOUND = 5,
  PJRT_Error_Code_ALREADY_EXISTS = 6,
  PJRT_Error_Code_PERMISSION_DENIED = 7,
  PJRT_Error_Code_RESOURCE_EXHAUSTED = 8,
  PJRT_Error_Code_FAILED_PRECONDITION = 9,
  PJRT_Error_Code_ABORTED = 10,
  PJRT_Error_Code_OUT_OF_RANGE = 11,
  PJRT_Error_Code_UNIMPLEMENTED = 12,
  PJRT_Error_Code_INTERNAL = 13,
  PJRT_Error_Code_UNAVAILABLE = 14,
  PJRT_Error_Code_DATA_LOSS = 15,
  PJRT_Error_Code_UNAUTHENTICATED = 16,
} PJRT_Error_Code;

typedef struct PJRT_Error_Destroy_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Error* error;
} PJRT_Error_Destroy_Args;
#define PJRT_Error_Destroy_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Error_Destroy_Args, error)
typedef void PJRT_Error_Destroy(PJRT_Error_Destroy_Args* args);

typedef struct PJRT_Error_Message_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const PJRT_Error* error;
  const char* message; /* out, lifetime of `error` */
  size_t message_size; /* out */
} PJRT_Error_Message_Args;
#define PJRT_Error_Message_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Error_Message_Args, message_size)
typedef void PJRT_Error_Message(PJRT_Error_Message_Args* args);

typedef struct PJRT_Error_GetCode_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const PJRT_Error* error;
  PJRT_Error_Code code; /* out */
} PJRT_Error_GetCode_Args;
#define PJRT_Error_GetCode_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Error_GetCode_Args, code)
typedef PJRT_Error* PJRT_Error_GetCode(PJRT_Error_GetCode_Args* args);

/* ------------------------------ Named values ----------------------------- */

typedef enum {
  PJRT_NamedValue_kString = 0,
  PJRT_NamedValue_kInt64,
  PJRT_NamedValue_kInt64List,
  PJRT_NamedValue_kFloat,
  PJRT_NamedValue_kBool,
} PJRT_NamedValue_Type;

typedef struct PJRT_NamedValue {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const char* name;
  size_t name_size;
  PJRT_NamedValue_Type type;
  union {
    const char* string_value;
    int64_t int64_value;
    const int64_t* int64_array_value;
    float float_value;
    bool bool_value;
  };
  size_t value_size; /* string length, list length, or 1 */
} PJRT_NamedValue;
#define PJRT_NamedValue_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_NamedValue, value_size)

/* --------------------------------- Plugin -------------------------------- */

typedef struct PJRT_Plugin_Initialize_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
} PJRT_Plugin_Initialize_Args;
#define PJRT_Plugin_Initialize_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Plugin_Initialize_Args, extension_start)
typedef PJRT_Error* PJRT_Plugin_Initialize(PJRT_Plugin_Initialize_Args* args);

typedef struct PJRT_Plugin_Attributes_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const PJRT_NamedValue* attributes; /* out */
  size_t num_attributes;             /* out */
} PJRT_Plugin_Attributes_Args;
#define PJRT_Plugin_Attributes_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Plugin_Attributes_Args, num_attributes)
typedef PJRT_Error* PJRT_Plugin_Attributes(PJRT_Plugin_Attributes_Args* args);

/* --------------------------------- Events -------------------------------- */

typedef struct PJRT_Event_Destroy_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Event* event;
} PJRT_Event_Destroy_Args;
#define PJRT_Event_Destroy_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Event_Destroy_Args, event)
typedef PJRT_Error* PJRT_Event_Destroy(PJRT_Event_Destroy_Args* args);

typedef struct PJRT_Event_IsReady_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Event* event;
  bool is_ready; /* out */
} PJRT_Event_IsReady_Args;
#define PJRT_Event_IsReady_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Event_IsReady_Args, is_ready)
typedef PJRT_Error* PJRT_Event_IsReady(PJRT_Event_IsReady_Args* args);

typedef struct PJRT_Event_Error_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Event* event;
} PJRT_Event_Error_Args;
#define PJRT_Event_Error_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Event_Error_Args, event)
typedef PJRT_Error* PJRT_Event_Error(PJRT_Event_Error_Args* args);

typedef struct PJRT_Event_Await_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Event* event;
} PJRT_Event_Await_Args;
#define PJRT_Event_Await_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Event_Await_Args, event)
typedef PJRT_Error* PJRT_Event_Await(PJRT_Event_Await_Args* args);

typedef void (*PJRT_Event_OnReadyCallback)(PJRT_Error* error, void* user_arg);

typedef struct PJRT_Event_OnReady_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Event* event;
  PJRT_Event_OnReadyCallback callback;
  void* user_arg;
} PJRT_Event_OnReady_Args;
#define PJRT_Event_OnReady_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Event_OnReady_Args, user_arg)
typedef PJRT_Error* PJRT_Event_OnReady(PJRT_Event_OnReady_Args* args);

/* --------------------------------- Client -------------------------------- */

typedef void (*PJRT_KeyValueGetCallback)(void* args);
typedef void (*PJRT_KeyValuePutCallback)(void* args);
typedef void (*PJRT_KeyValueTryGetCallback)(void* args);

typedef struct PJRT_Client_Create_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const PJRT_NamedValue* create_options;
  size_t num_options;
  PJRT_KeyValueGetCallback kv_get_callback;
  void* kv_get_user_arg;
  PJRT_KeyValuePutCallback kv_put_callback;
  void* kv_put_user_arg;
  PJRT_Client* client; /* out */
  PJRT_KeyValueTryGetCallback kv_try_get_callback;
  void* kv_try_get_user_arg;
} PJRT_Client_Create_Args;
#define PJRT_Client_Create_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_Create_Args, client)
typedef PJRT_Error* PJRT_Client_Create(PJRT_Client_Create_Args* args);

typedef struct PJRT_Client_Destroy_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
} PJRT_Client_Destroy_Args;
#define PJRT_Client_Destroy_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_Destroy_Args, client)
typedef PJRT_Error* PJRT_Client_Destroy(PJRT_Client_Destroy_Args* args);

typedef struct PJRT_Client_PlatformName_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  const char* platform_name; /* out */
  size_t platform_name_size; /* out */
} PJRT_Client_PlatformName_Args;
#define PJRT_Client_PlatformName_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_PlatformName_Args, platform_name_size)
typedef PJRT_Error* PJRT_Client_PlatformName(PJRT_Client_PlatformName_Args* args);

typedef struct PJRT_Client_ProcessIndex_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  int process_index; /* out */
} PJRT_Client_ProcessIndex_Args;
#define PJRT_Client_ProcessIndex_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_ProcessIndex_Args, process_index)
typedef PJRT_Error* PJRT_Client_ProcessIndex(PJRT_Client_ProcessIndex_Args* args);

typedef struct PJRT_Client_PlatformVersion_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  const char* platform_version; /* out */
  size_t platform_version_size; /* out */
} PJRT_Client_PlatformVersion_Args;
#define PJRT_Client_PlatformVersion_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_PlatformVersion_Args, platform_version_size)
typedef PJRT_Error* PJRT_Client_PlatformVersion(PJRT_Client_PlatformVersion_Args* args);

typedef struct PJRT_Client_TopologyDescription_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  PJRT_TopologyDescription* topology; /* out, owned by the client */
} PJRT_Client_TopologyDescription_Args;
#define PJRT_Client_TopologyDescription_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_TopologyDescription_Args, topology)
typedef PJRT_Error* PJRT_Client_TopologyDescription(PJRT_Client_TopologyDescription_Args* args);

typedef struct PJRT_Client_Devices_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  PJRT_Device* const* devices; /* out */
  size_t num_devices;          /* out */
} PJRT_Client_Devices_Args;
#define PJRT_Client_Devices_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_Devices_Args, num_devices)
typedef PJRT_Error* PJRT_Client_Devices(PJRT_Client_Devices_Args* args);

typedef struct PJRT_Client_AddressableDevices_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  PJRT_Device* const* addressable_devices; /* out */
  size_t num_addressable_devices;          /* out */
} PJRT_Client_AddressableDevices_Args;
#define PJRT_Client_AddressableDevices_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_AddressableDevices_Args, num_addressable_devices)
typedef PJRT_Error* PJRT_Client_AddressableDevices(PJRT_Client_AddressableDevices_Args* args);

typedef struct PJRT_Client_LookupDevice_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  int id;
  PJRT_Device* device; /* out */
} PJRT_Client_LookupDevice_Args;
#define PJRT_Client_LookupDevice_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_LookupDevice_Args, device)
typedef PJRT_Error* PJRT_Client_LookupDevice(PJRT_Client_LookupDevice_Args* args);

typedef struct PJRT_Client_LookupAddressableDevice_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  int local_hardware_id;
  PJRT_Device* addressable_device; /* out */
} PJRT_Client_LookupAddressableDevice_Args;
#define PJRT_Client_LookupAddressableDevice_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_LookupAddressableDevice_Args, addressable_device)
typedef PJRT_Error* PJRT_Client_LookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* args);

typedef struct PJRT_Client_AddressableMemories_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  PJRT_Memory* const* addressable_memories; /* out */
  size_t num_addressable_memories;          /* out */
} PJRT_Client_AddressableMemories_Args;
#define PJRT_Client_AddressableMemories_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_AddressableMemories_Args, num_addressable_memories)
typedef PJRT_Error* PJRT_Client_AddressableMemories(PJRT_Client_AddressableMemories_Args* args);

typedef struct PJRT_Program {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  char* code; /* MLIR text or bytecode when format is "mlir" */
  size_t code_size;
  const char* format;
  size_t format_size;
} PJRT_Program;
#define PJRT_Program_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Program, format_size)

typedef struct PJRT_Client_Compile_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  const PJRT_Program* program;
  const char* compile_options; /* serialized CompileOptionsProto */
  size_t compile_options_size;
  PJRT_LoadedExecutable* executable; /* out */
} PJRT_Client_Compile_Args;
#define PJRT_Client_Compile_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_Compile_Args, executable)
typedef PJRT_Error* PJRT_Client_Compile(PJRT_Client_Compile_Args* args);

typedef struct PJRT_Client_DefaultDeviceAssignment_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  int num_replicas;
  int num_partitions;
  size_t default_assignment_size; /* capacity of default_assignment */
  int* default_assignment;        /* out, [num_replicas * num_partitions] */
} PJRT_Client_DefaultDeviceAssignment_Args;
#define PJRT_Client_DefaultDeviceAssignment_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_DefaultDeviceAssignment_Args, default_assignment)
typedef PJRT_Error* PJRT_Client_DefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* args);

typedef enum {
  PJRT_Buffer_Type_INVALID = 0,
  PJRT_Buffer_Type_PRED,
  PJRT_Buffer_Type_S8,
  PJRT_Buffer_Type_S16,
  PJRT_Buffer_Type_S32,
  PJRT_Buffer_Type_S64,
  PJRT_Buffer_Type_U8,
  PJRT_Buffer_Type_U16,
  PJRT_Buffer_Type_U32,
  PJRT_Buffer_Type_U64,
  PJRT_Buffer_Type_F16,
  PJRT_Buffer_Type_F32,
  PJRT_Buffer_Type_F64,
  PJRT_Buffer_Type_BF16,
  PJRT_Buffer_Type_C64,
  PJRT_Buffer_Type_C128,
  PJRT_Buffer_Type_F8E5M2,
  PJRT_Buffer_Type_F8E4M3FN,
  PJRT_Buffer_Type_F8E4M3B11FNUZ,
  PJRT_Buffer_Type_F8E5M2FNUZ,
  PJRT_Buffer_Type_F8E4M3FNUZ,
  PJRT_Buffer_Type_S4,
  PJRT_Buffer_Type_U4,
  PJRT_Buffer_Type_TOKEN,
  PJRT_Buffer_Type_S2,
  PJRT_Buffer_Type_U2,
} PJRT_Buffer_Type;

typedef enum {
  PJRT_HostBufferSemantics_kImmutableOnlyDuringCall = 0,
  PJRT_HostBufferSemantics_kImmutableUntilTransferCompletes,
  PJRT_HostBufferSemantics_kImmutableZeroCopy,
  PJRT_HostBufferSemantics_kMutableZeroCopy,
} PJRT_HostBufferSemantics;

typedef enum {
  PJRT_Buffer_MemoryLayout_Type_Tiled = 0,
  PJRT_Buffer_MemoryLayout_Type_Strides,
} PJRT_Buffer_MemoryLayout_Type;

typedef struct PJRT_Buffer_MemoryLayout_Tiled {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const int64_t* minor_to_major;
  size_t minor_to_major_size;
  const int64_t* tile_dims;
  const size_t* tile_dim_sizes;
  size_t num_tiles;
} PJRT_Buffer_MemoryLayout_Tiled;

typedef struct PJRT_Buffer_MemoryLayout_Strides {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const int64_t* byte_strides;
  size_t num_byte_strides;
} PJRT_Buffer_MemoryLayout_Strides;

typedef struct PJRT_Buffer_MemoryLayout {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  union {
    PJRT_Buffer_MemoryLayout_Tiled tiled;
    PJRT_Buffer_MemoryLayout_Strides strides;
  };
  PJRT_Buffer_MemoryLayout_Type type;
} PJRT_Buffer_MemoryLayout;

typedef struct PJRT_Client_BufferFromHostBuffer_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  const void* data;
  PJRT_Buffer_Type type;
  const int64_t* dims;
  size_t num_dims;
  const int64_t* byte_strides; /* may be NULL: dense row-major */
  size_t num_byte_strides;
  PJRT_HostBufferSemantics host_buffer_semantics;
  PJRT_Device* device;
  PJRT_Memory* memory;
  PJRT_Buffer_MemoryLayout* device_layout;
  PJRT_Event* done_with_host_buffer; /* out */
  PJRT_Buffer* buffer;               /* out */
} PJRT_Client_BufferFromHostBuffer_Args;
#define PJRT_Client_BufferFromHostBuffer_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Client_BufferFromHostBuffer_Args, buffer)
typedef PJRT_Error* PJRT_Client_BufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* args);

/* --------------------------- Device description -------------------------- */

typedef struct PJRT_DeviceDescription_Id_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_DeviceDescription* device_description;
  int id; /* out */
} PJRT_DeviceDescription_Id_Args;
#define PJRT_DeviceDescription_Id_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_DeviceDescription_Id_Args, id)
typedef PJRT_Error* PJRT_DeviceDescription_Id(PJRT_DeviceDescription_Id_Args* args);

typedef struct PJRT_DeviceDescription_ProcessIndex_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_DeviceDescription* device_description;
  int process_index; /* out */
} PJRT_DeviceDescription_ProcessIndex_Args;
#define PJRT_DeviceDescription_ProcessIndex_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_DeviceDescription_ProcessIndex_Args, process_index)
typedef PJRT_Error* PJRT_DeviceDescription_ProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* args);

typedef struct PJRT_DeviceDescription_Attributes_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_DeviceDescription* device_description;
  size_t num_attributes;             /* out */
  const PJRT_NamedValue* attributes; /* out */
} PJRT_DeviceDescription_Attributes_Args;
#define PJRT_DeviceDescription_Attributes_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_DeviceDescription_Attributes_Args, attributes)
typedef PJRT_Error* PJRT_DeviceDescription_Attributes(PJRT_DeviceDescription_Attributes_Args* args);

typedef struct PJRT_DeviceDescription_Kind_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_DeviceDescription* device_description;
  const char* device_kind; /* out */
  size_t device_kind_size; /* out */
} PJRT_DeviceDescription_Kind_Args;
#define PJRT_DeviceDescription_Kind_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_DeviceDescription_Kind_Args, device_kind_size)
typedef PJRT_Error* PJRT_DeviceDescription_Kind(PJRT_DeviceDescription_Kind_Args* args);

typedef struct PJRT_DeviceDescription_DebugString_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_DeviceDescription* device_description;
  const char* debug_string; /* out */
  size_t debug_string_size; /* out */
} PJRT_DeviceDescription_DebugString_Args;
#define PJRT_DeviceDescription_DebugString_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_DeviceDescription_DebugString_Args, debug_string_size)
typedef PJRT_Error* PJRT_DeviceDescription_DebugString(PJRT_DeviceDescription_DebugString_Args* args);

typedef struct PJRT_DeviceDescription_ToString_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_DeviceDescription* device_description;
  const char* to_string; /* out */
  size_t to_string_size; /* out */
} PJRT_DeviceDescription_ToString_Args;
#define PJRT_DeviceDescription_ToString_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_DeviceDescription_ToString_Args, to_string_size)
typedef PJRT_Error* PJRT_DeviceDescription_ToString(PJRT_DeviceDescription_ToString_Args* args);

/* --------------------------------- Device -------------------------------- */

typedef struct PJRT_Device_GetDescription_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Device* device;
  PJRT_DeviceDescription* device_description; /* out */
} PJRT_Device_GetDescription_Args;
#define PJRT_Device_GetDescription_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Device_GetDescription_Args, device_description)
typedef PJRT_Error* PJRT_Device_GetDescription(PJRT_Device_GetDescription_Args* args);

typedef struct PJRT_Device_IsAddressable_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Device* device;
  bool is_addressable; /* out */
} PJRT_Device_IsAddressable_Args;
#define PJRT_Device_IsAddressable_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Device_IsAddressable_Args, is_addressable)
typedef PJRT_Error* PJRT_Device_IsAddressable(PJRT_Device_IsAddressable_Args* args);

typedef struct PJRT_Device_LocalHardwareId_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Device* device;
  int local_hardware_id; /* out */
} PJRT_Device_LocalHardwareId_Args;
#define PJRT_Device_LocalHardwareId_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Device_LocalHardwareId_Args, local_hardware_id)
typedef PJRT_Error* PJRT_Device_LocalHardwareId(PJRT_Device_LocalHardwareId_Args* args);

typedef struct PJRT_Device_AddressableMemories_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Device* device;
  PJRT_Memory* const* memories; /* out */
  size_t num_memories;          /* out */
} PJRT_Device_AddressableMemories_Args;
#define PJRT_Device_AddressableMemories_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Device_AddressableMemories_Args, num_memories)
typedef PJRT_Error* PJRT_Device_AddressableMemories(PJRT_Device_AddressableMemories_Args* args);

typedef struct PJRT_Device_DefaultMemory_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Device* device;
  PJRT_Memory* memory; /* out */
} PJRT_Device_DefaultMemory_Args;
#define PJRT_Device_DefaultMemory_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Device_DefaultMemory_Args, memory)
typedef PJRT_Error* PJRT_Device_DefaultMemory(PJRT_Device_DefaultMemory_Args* args);

typedef struct PJRT_Device_MemoryStats_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Device* device;
  int64_t bytes_in_use; /* out */
  int64_t peak_bytes_in_use;
  bool peak_bytes_in_use_is_set;
  int64_t num_allocs;
  bool num_allocs_is_set;
  int64_t largest_alloc_size;
  bool largest_alloc_size_is_set;
  int64_t bytes_limit;
  bool bytes_limit_is_set;
  int64_t bytes_reserved;
  bool bytes_reserved_is_set;
  int64_t peak_bytes_reserved;
  bool peak_bytes_reserved_is_set;
  int64_t bytes_reservable_limit;
  bool bytes_reservable_limit_is_set;
  int64_t largest_free_block_bytes;
  bool largest_free_block_bytes_is_set;
  int64_t pool_bytes;
  bool pool_bytes_is_set;
  int64_t peak_pool_bytes;
  bool peak_pool_bytes_is_set;
} PJRT_Device_MemoryStats_Args;
#define PJRT_Device_MemoryStats_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Device_MemoryStats_Args, peak_pool_bytes_is_set)
typedef PJRT_Error* PJRT_Device_MemoryStats(PJRT_Device_MemoryStats_Args* args);

/* --------------------------------- Memory -------------------------------- */

typedef struct PJRT_Memory_Id_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Memory* memory;
  int id; /* out */
} PJRT_Memory_Id_Args;
#define PJRT_Memory_Id_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Memory_Id_Args, id)
typedef PJRT_Error* PJRT_Memory_Id(PJRT_Memory_Id_Args* args);

typedef struct PJRT_Memory_Kind_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Memory* memory;
  const char* kind; /* out */
  size_t kind_size; /* out */
} PJRT_Memory_Kind_Args;
#define PJRT_Memory_Kind_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Memory_Kind_Args, kind_size)
typedef PJRT_Error* PJRT_Memory_Kind(PJRT_Memory_Kind_Args* args);

typedef struct PJRT_Memory_Kind_Id_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Memory* memory;
  int kind_id; /* out */
} PJRT_Memory_Kind_Id_Args;
#define PJRT_Memory_Kind_Id_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Memory_Kind_Id_Args, kind_id)
typedef PJRT_Error* PJRT_Memory_Kind_Id(PJRT_Memory_Kind_Id_Args* args);

typedef struct PJRT_Memory_DebugString_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Memory* memory;
  const char* debug_string; /* out */
  size_t debug_string_size; /* out */
} PJRT_Memory_DebugString_Args;
#define PJRT_Memory_DebugString_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Memory_DebugString_Args, debug_string_size)
typedef PJRT_Error* PJRT_Memory_DebugString(PJRT_Memory_DebugString_Args* args);

typedef struct PJRT_Memory_ToString_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Memory* memory;
  const char* to_string; /* out */
  size_t to_string_size; /* out */
} PJRT_Memory_ToString_Args;
#define PJRT_Memory_ToString_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Memory_ToString_Args, to_string_size)
typedef PJRT_Error* PJRT_Memory_ToString(PJRT_Memory_ToString_Args* args);

typedef struct PJRT_Memory_AddressableByDevices_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Memory* memory;
  PJRT_Device* const* devices; /* out */
  size_t num_devices;          /* out */
} PJRT_Memory_AddressableByDevices_Args;
#define PJRT_Memory_AddressableByDevices_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Memory_AddressableByDevices_Args, num_devices)
typedef PJRT_Error* PJRT_Memory_AddressableByDevices(PJRT_Memory_AddressableByDevices_Args* args);

/* ------------------------------- Executables ----------------------------- */

typedef struct PJRT_Executable_Destroy_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
} PJRT_Executable_Destroy_Args;
#define PJRT_Executable_Destroy_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_Destroy_Args, executable)
typedef PJRT_Error* PJRT_Executable_Destroy(PJRT_Executable_Destroy_Args* args);

typedef struct PJRT_Executable_Name_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  const char* executable_name; /* out */
  size_t executable_name_size; /* out */
} PJRT_Executable_Name_Args;
#define PJRT_Executable_Name_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_Name_Args, executable_name_size)
typedef PJRT_Error* PJRT_Executable_Name(PJRT_Executable_Name_Args* args);

typedef struct PJRT_Executable_NumReplicas_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  size_t num_replicas; /* out */
} PJRT_Executable_NumReplicas_Args;
#define PJRT_Executable_NumReplicas_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_NumReplicas_Args, num_replicas)
typedef PJRT_Error* PJRT_Executable_NumReplicas(PJRT_Executable_NumReplicas_Args* args);

typedef struct PJRT_Executable_NumPartitions_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  size_t num_partitions; /* out */
} PJRT_Executable_NumPartitions_Args;
#define PJRT_Executable_NumPartitions_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_NumPartitions_Args, num_partitions)
typedef PJRT_Error* PJRT_Executable_NumPartitions(PJRT_Executable_NumPartitions_Args* args);

typedef struct PJRT_Executable_NumOutputs_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  size_t num_outputs; /* out */
} PJRT_Executable_NumOutputs_Args;
#define PJRT_Executable_NumOutputs_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_NumOutputs_Args, num_outputs)
typedef PJRT_Error* PJRT_Executable_NumOutputs(PJRT_Executable_NumOutputs_Args* args);

typedef struct PJRT_Executable_SizeOfGeneratedCodeInBytes_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  int64_t size_in_bytes; /* out */
} PJRT_Executable_SizeOfGeneratedCodeInBytes_Args;
#define PJRT_Executable_SizeOfGeneratedCodeInBytes_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args, size_in_bytes)
typedef PJRT_Error* PJRT_Executable_SizeOfGeneratedCodeInBytes(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* args);

typedef struct PJRT_Executable_GetCostAnalysis_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  size_t num_properties;             /* out */
  const PJRT_NamedValue* properties; /* out */
} PJRT_Executable_GetCostAnalysis_Args;
#define PJRT_Executable_GetCostAnalysis_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_GetCostAnalysis_Args, properties)
typedef PJRT_Error* PJRT_Executable_GetCostAnalysis(PJRT_Executable_GetCostAnalysis_Args* args);

typedef struct PJRT_Executable_OutputMemoryKinds_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  size_t num_outputs;              /* out */
  const char* const* memory_kinds; /* out */
  const size_t* memory_kind_sizes; /* out */
} PJRT_Executable_OutputMemoryKinds_Args;
#define PJRT_Executable_OutputMemoryKinds_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_OutputMemoryKinds_Args, memory_kind_sizes)
typedef PJRT_Error* PJRT_Executable_OutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* args);

typedef struct PJRT_Executable_OptimizedProgram_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  PJRT_Program* program; /* in/out: code==NULL asks for code_size */
} PJRT_Executable_OptimizedProgram_Args;
#define PJRT_Executable_OptimizedProgram_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_OptimizedProgram_Args, program)
typedef PJRT_Error* PJRT_Executable_OptimizedProgram(PJRT_Executable_OptimizedProgram_Args* args);

typedef struct PJRT_Executable_Serialize_Args PJRT_Executable_Serialize_Args;
typedef PJRT_Error* PJRT_Executable_Serialize(PJRT_Executable_Serialize_Args* args);

typedef struct PJRT_Executable_OutputElementTypes_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  PJRT_Buffer_Type* output_types; /* out */
  size_t num_output_types;        /* out */
} PJRT_Executable_OutputElementTypes_Args;
#define PJRT_Executable_OutputElementTypes_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_OutputElementTypes_Args, num_output_types)
typedef PJRT_Error* PJRT_Executable_OutputElementTypes(PJRT_Executable_OutputElementTypes_Args* args);

typedef struct PJRT_Executable_OutputDimensions_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  size_t num_outputs;       /* out */
  const int64_t* dims;      /* out, concatenated */
  const size_t* dim_sizes;  /* out, rank of each output */
} PJRT_Executable_OutputDimensions_Args;
#define PJRT_Executable_OutputDimensions_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_OutputDimensions_Args, dim_sizes)
typedef PJRT_Error* PJRT_Executable_OutputDimensions(PJRT_Executable_OutputDimensions_Args* args);

typedef struct PJRT_Executable_Fingerprint_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Executable* executable;
  const char* executable_fingerprint; /* out */
  size_t executable_fingerprint_size; /* out */
} PJRT_Executable_Fingerprint_Args;
#define PJRT_Executable_Fingerprint_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Executable_Fingerprint_Args, executable_fingerprint_size)
typedef PJRT_Error* PJRT_Executable_Fingerprint(PJRT_Executable_Fingerprint_Args* args);

typedef struct PJRT_Executable_GetCompiledMemoryStats_Args PJRT_Executable_GetCompiledMemoryStats_Args;
typedef PJRT_Error* PJRT_Executable_GetCompiledMemoryStats(PJRT_Executable_GetCompiledMemoryStats_Args* args);

typedef struct PJRT_LoadedExecutable_Destroy_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_LoadedExecutable* executable;
} PJRT_LoadedExecutable_Destroy_Args;
#define PJRT_LoadedExecutable_Destroy_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_LoadedExecutable_Destroy_Args, executable)
typedef PJRT_Error* PJRT_LoadedExecutable_Destroy(PJRT_LoadedExecutable_Destroy_Args* args);

typedef struct PJRT_LoadedExecutable_GetExecutable_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_LoadedExecutable* loaded_executable;
  PJRT_Executable* executable; /* out, caller destroys */
} PJRT_LoadedExecutable_GetExecutable_Args;
#define PJRT_LoadedExecutable_GetExecutable_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_LoadedExecutable_GetExecutable_Args, executable)
typedef PJRT_Error* PJRT_LoadedExecutable_GetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* args);

typedef struct PJRT_LoadedExecutable_AddressableDevices_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_LoadedExecutable* executable;
  PJRT_Device* const* addressable_devices; /* out */
  size_t num_addressable_devices;          /* out */
} PJRT_LoadedExecutable_AddressableDevices_Args;
#define PJRT_LoadedExecutable_AddressableDevices_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_LoadedExecutable_AddressableDevices_Args, num_addressable_devices)
typedef PJRT_Error* PJRT_LoadedExecutable_AddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* args);

typedef struct PJRT_LoadedExecutable_Delete_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_LoadedExecutable* executable;
} PJRT_LoadedExecutable_Delete_Args;
#define PJRT_LoadedExecutable_Delete_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_LoadedExecutable_Delete_Args, executable)
typedef PJRT_Error* PJRT_LoadedExecutable_Delete(PJRT_LoadedExecutable_Delete_Args* args);

typedef struct PJRT_LoadedExecutable_IsDeleted_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_LoadedExecutable* executable;
  bool is_deleted; /* out */
} PJRT_LoadedExecutable_IsDeleted_Args;
#define PJRT_LoadedExecutable_IsDeleted_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_LoadedExecutable_IsDeleted_Args, is_deleted)
typedef PJRT_Error* PJRT_LoadedExecutable_IsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* args);

typedef struct PJRT_SendCallbackInfo PJRT_SendCallbackInfo;
typedef struct PJRT_RecvCallbackInfo PJRT_RecvCallbackInfo;

typedef struct PJRT_ExecuteOptions {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_SendCallbackInfo** send_callbacks;
  PJRT_RecvCallbackInfo** recv_callbacks;
  size_t num_send_ops;
  size_t num_recv_ops;
  int launch_id;
  const int64_t* non_donatable_input_indices;
  size_t num_non_donatable_input_indices;
  PJRT_ExecuteContext* context;
} PJRT_ExecuteOptions;
#define PJRT_ExecuteOptions_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_ExecuteOptions, context)

typedef struct PJRT_LoadedExecutable_Execute_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_LoadedExecutable* executable;
  PJRT_ExecuteOptions* options;
  PJRT_Buffer* const* const* argument_lists; /* [num_devices][num_args] */
  size_t num_devices;
  size_t num_args;
  PJRT_Buffer** const* output_lists;    /* [num_devices][num_outputs], filled */
  PJRT_Event** device_complete_events;  /* [num_devices] or NULL, filled */
  PJRT_Device* execute_device;
} PJRT_LoadedExecutable_Execute_Args;
#define PJRT_LoadedExecutable_Execute_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_LoadedExecutable_Execute_Args, execute_device)
typedef PJRT_Error* PJRT_LoadedExecutable_Execute(PJRT_LoadedExecutable_Execute_Args* args);

typedef struct PJRT_Executable_DeserializeAndLoad_Args PJRT_Executable_DeserializeAndLoad_Args;
typedef PJRT_Error* PJRT_Executable_DeserializeAndLoad(PJRT_Executable_DeserializeAndLoad_Args* args);

typedef struct PJRT_LoadedExecutable_Fingerprint_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_LoadedExecutable* executable;
  const char* executable_fingerprint; /* out */
  size_t executable_fingerprint_size; /* out */
} PJRT_LoadedExecutable_Fingerprint_Args;
#define PJRT_LoadedExecutable_Fingerprint_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_LoadedExecutable_Fingerprint_Args, executable_fingerprint_size)
typedef PJRT_Error* PJRT_LoadedExecutable_Fingerprint(PJRT_LoadedExecutable_Fingerprint_Args* args);

/* --------------------------------- Buffers ------------------------------- */

typedef struct PJRT_Buffer_Destroy_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
} PJRT_Buffer_Destroy_Args;
#define PJRT_Buffer_Destroy_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_Destroy_Args, buffer)
typedef PJRT_Error* PJRT_Buffer_Destroy(PJRT_Buffer_Destroy_Args* args);

typedef struct PJRT_Buffer_ElementType_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  PJRT_Buffer_Type type; /* out */
} PJRT_Buffer_ElementType_Args;
#define PJRT_Buffer_ElementType_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_ElementType_Args, type)
typedef PJRT_Error* PJRT_Buffer_ElementType(PJRT_Buffer_ElementType_Args* args);

typedef struct PJRT_Buffer_Dimensions_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  const int64_t* dims; /* out, lifetime of buffer */
  size_t num_dims;     /* out */
} PJRT_Buffer_Dimensions_Args;
#define PJRT_Buffer_Dimensions_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_Dimensions_Args, num_dims)
typedef PJRT_Error* PJRT_Buffer_Dimensions(PJRT_Buffer_Dimensions_Args* args);

typedef struct PJRT_Buffer_UnpaddedDimensions_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  const int64_t* unpadded_dims; /* out */
  size_t num_dims;              /* out */
} PJRT_Buffer_UnpaddedDimensions_Args;
#define PJRT_Buffer_UnpaddedDimensions_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_UnpaddedDimensions_Args, num_dims)
typedef PJRT_Error* PJRT_Buffer_UnpaddedDimensions(PJRT_Buffer_UnpaddedDimensions_Args* args);

typedef struct PJRT_Buffer_DynamicDimensionIndices_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  const size_t* dynamic_dim_indices; /* out */
  size_t num_dynamic_dims;           /* out */
} PJRT_Buffer_DynamicDimensionIndices_Args;
#define PJRT_Buffer_DynamicDimensionIndices_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_DynamicDimensionIndices_Args, num_dynamic_dims)
typedef PJRT_Error* PJRT_Buffer_DynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* args);

typedef struct PJRT_Buffer_GetMemoryLayout_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  PJRT_Buffer_MemoryLayout layout; /* out */
} PJRT_Buffer_GetMemoryLayout_Args;
#define PJRT_Buffer_GetMemoryLayout_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_GetMemoryLayout_Args, layout)
typedef PJRT_Error* PJRT_Buffer_GetMemoryLayout(PJRT_Buffer_GetMemoryLayout_Args* args);

typedef struct PJRT_Buffer_OnDeviceSizeInBytes_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  size_t on_device_size_in_bytes; /* out */
} PJRT_Buffer_OnDeviceSizeInBytes_Args;
#define PJRT_Buffer_OnDeviceSizeInBytes_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_OnDeviceSizeInBytes_Args, on_device_size_in_bytes)
typedef PJRT_Error* PJRT_Buffer_OnDeviceSizeInBytes(PJRT_Buffer_OnDeviceSizeInBytes_Args* args);

typedef struct PJRT_Buffer_Device_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  PJRT_Device* device; /* out */
} PJRT_Buffer_Device_Args;
#define PJRT_Buffer_Device_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_Device_Args, device)
typedef PJRT_Error* PJRT_Buffer_Device(PJRT_Buffer_Device_Args* args);

typedef struct PJRT_Buffer_Memory_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  PJRT_Memory* memory; /* out */
} PJRT_Buffer_Memory_Args;
#define PJRT_Buffer_Memory_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_Memory_Args, memory)
typedef PJRT_Error* PJRT_Buffer_Memory(PJRT_Buffer_Memory_Args* args);

typedef struct PJRT_Buffer_Delete_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
} PJRT_Buffer_Delete_Args;
#define PJRT_Buffer_Delete_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_Delete_Args, buffer)
typedef PJRT_Error* PJRT_Buffer_Delete(PJRT_Buffer_Delete_Args* args);

typedef struct PJRT_Buffer_IsDeleted_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  bool is_deleted; /* out */
} PJRT_Buffer_IsDeleted_Args;
#define PJRT_Buffer_IsDeleted_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_IsDeleted_Args, is_deleted)
typedef PJRT_Error* PJRT_Buffer_IsDeleted(PJRT_Buffer_IsDeleted_Args* args);

typedef struct PJRT_Buffer_CopyToDevice_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  PJRT_Device* dst_device;
  PJRT_Buffer* dst_buffer; /* out */
} PJRT_Buffer_CopyToDevice_Args;
#define PJRT_Buffer_CopyToDevice_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_CopyToDevice_Args, dst_buffer)
typedef PJRT_Error* PJRT_Buffer_CopyToDevice(PJRT_Buffer_CopyToDevice_Args* args);

typedef struct PJRT_Buffer_ToHostBuffer_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* src;
  PJRT_Buffer_MemoryLayout* host_layout;
  void* dst;       /* NULL: only dst_size is written */
  size_t dst_size; /* in/out */
  PJRT_Event* event; /* out */
} PJRT_Buffer_ToHostBuffer_Args;
#define PJRT_Buffer_ToHostBuffer_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_ToHostBuffer_Args, event)
typedef PJRT_Error* PJRT_Buffer_ToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* args);

typedef struct PJRT_Buffer_IsOnCpu_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  bool is_on_cpu; /* out */
} PJRT_Buffer_IsOnCpu_Args;
#define PJRT_Buffer_IsOnCpu_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_IsOnCpu_Args, is_on_cpu)
typedef PJRT_Error* PJRT_Buffer_IsOnCpu(PJRT_Buffer_IsOnCpu_Args* args);

typedef struct PJRT_Buffer_ReadyEvent_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  PJRT_Event* event; /* out, caller destroys */
} PJRT_Buffer_ReadyEvent_Args;
#define PJRT_Buffer_ReadyEvent_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_ReadyEvent_Args, event)
typedef PJRT_Error* PJRT_Buffer_ReadyEvent(PJRT_Buffer_ReadyEvent_Args* args);

typedef struct PJRT_Buffer_UnsafePointer_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  uintptr_t buffer_pointer; /* out */
} PJRT_Buffer_UnsafePointer_Args;
#define PJRT_Buffer_UnsafePointer_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_UnsafePointer_Args, buffer_pointer)
typedef PJRT_Error* PJRT_Buffer_UnsafePointer(PJRT_Buffer_UnsafePointer_Args* args);

typedef struct PJRT_Buffer_IncreaseExternalReferenceCount_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
} PJRT_Buffer_IncreaseExternalReferenceCount_Args;
typedef PJRT_Error* PJRT_Buffer_IncreaseExternalReferenceCount(PJRT_Buffer_IncreaseExternalReferenceCount_Args* args);

typedef struct PJRT_Buffer_DecreaseExternalReferenceCount_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
} PJRT_Buffer_DecreaseExternalReferenceCount_Args;
typedef PJRT_Error* PJRT_Buffer_DecreaseExternalReferenceCount(PJRT_Buffer_DecreaseExternalReferenceCount_Args* args);

typedef struct PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  void* device_memory_ptr; /* out */
} PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args;
#define PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args, device_memory_ptr)
typedef PJRT_Error* PJRT_Buffer_OpaqueDeviceMemoryDataPointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* args);

typedef struct PJRT_Buffer_CopyToMemory_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Buffer* buffer;
  PJRT_Memory* dst_memory;
  PJRT_Buffer* dst_buffer; /* out */
} PJRT_Buffer_CopyToMemory_Args;
#define PJRT_Buffer_CopyToMemory_Args_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Buffer_CopyToMemory_Args, dst_buffer)
typedef PJRT_Error* PJRT_Buffer_CopyToMemory(PJRT_Buffer_CopyToMemory_Args* args);

/* ------------------------- async host-to-device ------------------------- */
/* A transfer manager owns one device buffer per shape spec; the host fills  */
/* each with TransferData chunks (any order, any sizes); a buffer is ready   */
/* once the call flagged is_last_transfer has been made for it.              */

typedef struct PJRT_ShapeSpec {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const int64_t* dims;
  size_t num_dims;
  PJRT_Buffer_Type element_type;
} PJRT_ShapeSpec;
#define PJRT_ShapeSpec_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_ShapeSpec, element_type)

typedef struct PJRT_Client_CreateBuffersForAsyncHostToDevice_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Client* client;
  PJRT_ShapeSpec* shape_specs;
  size_t num_shape_specs;
  PJRT_Buffer_MemoryLayout** device_layouts; /* optional */
  size_t num_device_layouts;
  PJRT_Memory* memory;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager; /* out */
} PJRT_Client_CreateBuffersForAsyncHostToDevice_Args;
#define PJRT_Client_CreateBuffersForAsyncHostToDevice_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_Client_CreateBuffersForAsyncHostToDevice_Args, transfer_manager)
typedef PJRT_Error* PJRT_Client_CreateBuffersForAsyncHostToDevice(PJRT_Client_CreateBuffersForAsyncHostToDevice_Args* args);

typedef struct PJRT_AsyncHostToDeviceTransferManager_Destroy_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager;
} PJRT_AsyncHostToDeviceTransferManager_Destroy_Args;
#define PJRT_AsyncHostToDeviceTransferManager_Destroy_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_AsyncHostToDeviceTransferManager_Destroy_Args, transfer_manager)
typedef PJRT_Error* PJRT_AsyncHostToDeviceTransferManager_Destroy(PJRT_AsyncHostToDeviceTransferManager_Destroy_Args* args);

typedef struct PJRT_AsyncHostToDeviceTransferManager_TransferData_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager;
  int buffer_index;
  const void* data;
  int64_t offset;
  int64_t transfer_size;
  bool is_last_transfer;
  PJRT_Event* done_with_h2d_transfer; /* out */
} PJRT_AsyncHostToDeviceTransferManager_TransferData_Args;
#define PJRT_AsyncHostToDeviceTransferManager_TransferData_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_AsyncHostToDeviceTransferManager_TransferData_Args, done_with_h2d_transfer)
typedef PJRT_Error* PJRT_AsyncHostToDeviceTransferManager_TransferData(PJRT_AsyncHostToDeviceTransferManager_TransferData_Args* args);

typedef struct PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager;
  int buffer_index;
  PJRT_Buffer* buffer_out; /* out */
} PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer_Args;
#define PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer_Args, buffer_out)
typedef PJRT_Error* PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer(PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer_Args* args);

typedef struct PJRT_AsyncHostToDeviceTransferManager_Device_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager;
  PJRT_Device* device_out; /* out */
} PJRT_AsyncHostToDeviceTransferManager_Device_Args;
#define PJRT_AsyncHostToDeviceTransferManager_Device_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_AsyncHostToDeviceTransferManager_Device_Args, device_out)
typedef PJRT_Error* PJRT_AsyncHostToDeviceTransferManager_Device(PJRT_AsyncHostToDeviceTransferManager_Device_Args* args);

typedef struct PJRT_AsyncHostToDeviceTransferManager_BufferCount_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager;
  size_t buffer_count; /* out */
} PJRT_AsyncHostToDeviceTransferManager_BufferCount_Args;
#define PJRT_AsyncHostToDeviceTransferManager_BufferCount_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_AsyncHostToDeviceTransferManager_BufferCount_Args, buffer_count)
typedef PJRT_Error* PJRT_AsyncHostToDeviceTransferManager_BufferCount(PJRT_AsyncHostToDeviceTransferManager_BufferCount_Args* args);

typedef struct PJRT_AsyncHostToDeviceTransferManager_BufferSize_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager;
  int buffer_index;
  size_t buffer_size; /* out */
} PJRT_AsyncHostToDeviceTransferManager_BufferSize_Args;
#define PJRT_AsyncHostToDeviceTransferManager_BufferSize_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_AsyncHostToDeviceTransferManager_BufferSize_Args, buffer_size)
typedef PJRT_Error* PJRT_AsyncHostToDeviceTransferManager_BufferSize(PJRT_AsyncHostToDeviceTransferManager_BufferSize_Args* args);

typedef struct PJRT_AsyncHostToDeviceTransferManager_SetBufferError_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager;
  int buffer_index;
  PJRT_Error_Code error_code;
  const char* error_message;
  size_t error_message_size;
} PJRT_AsyncHostToDeviceTransferManager_SetBufferError_Args;
#define PJRT_AsyncHostToDeviceTransferManager_SetBufferError_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_AsyncHostToDeviceTransferManager_SetBufferError_Args, error_message_size)
typedef PJRT_Error* PJRT_AsyncHostToDeviceTransferManager_SetBufferError(PJRT_AsyncHostToDeviceTransferManager_SetBufferError_Args* args);

typedef struct PJRT_AsyncHostToDeviceTransferManager_AddMetadata_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_AsyncHostToDeviceTransferManager* transfer_manager;
  const PJRT_NamedValue* transfer_metadata;
  size_t num_metadata;
} PJRT_AsyncHostToDeviceTransferManager_AddMetadata_Args;
#define PJRT_AsyncHostToDeviceTransferManager_AddMetadata_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_AsyncHostToDeviceTransferManager_AddMetadata_Args, num_metadata)
typedef PJRT_Error* PJRT_AsyncHostToDeviceTransferManager_AddMetadata(PJRT_AsyncHostToDeviceTransferManager_AddMetadata_Args* args);

/* --------------------- Families outside the hot path --------------------- */
/* Slots keep their table position; the plugin answers UNIMPLEMENTED.       */

typedef struct PJRT_CopyToDeviceStream_Destroy_Args PJRT_CopyToDeviceStream_Destroy_Args;
typedef PJRT_Error* PJRT_CopyToDeviceStream_Destroy(PJRT_CopyToDeviceStream_Destroy_Args* args);
typedef struct PJRT_CopyToDeviceStream_AddChunk_Args PJRT_CopyToDeviceStream_AddChunk_Args;
typedef PJRT_Error* PJRT_CopyToDeviceStream_AddChunk(PJRT_CopyToDeviceStream_AddChunk_Args* args);
typedef struct PJRT_CopyToDeviceStream_TotalBytes_Args PJRT_CopyToDeviceStream_TotalBytes_Args;
typedef PJRT_Error* PJRT_CopyToDeviceStream_TotalBytes(PJRT_CopyToDeviceStream_TotalBytes_Args* args);
typedef struct PJRT_CopyToDeviceStream_GranuleSize_Args PJRT_CopyToDeviceStream_GranuleSize_Args;
typedef PJRT_Error* PJRT_CopyToDeviceStream_GranuleSize(PJRT_CopyToDeviceStream_GranuleSize_Args* args);
typedef struct PJRT_CopyToDeviceStream_CurrentBytes_Args PJRT_CopyToDeviceStream_CurrentBytes_Args;
typedef PJRT_Error* PJRT_CopyToDeviceStream_CurrentBytes(PJRT_CopyToDeviceStream_CurrentBytes_Args* args);

typedef struct PJRT_TopologyDescription_Create_Args PJRT_TopologyDescription_Create_Args;
typedef PJRT_Error* PJRT_TopologyDescription_Create(PJRT_TopologyDescription_Create_Args* args);
typedef struct PJRT_TopologyDescription_Destroy_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_TopologyDescription* topology;
} PJRT_TopologyDescription_Destroy_Args;
typedef PJRT_Error* PJRT_TopologyDescription_Destroy(PJRT_TopologyDescription_Destroy_Args* args);
typedef struct PJRT_TopologyDescription_PlatformVersion_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_TopologyDescription* topology;
  const char* platform_version; /* out */
  size_t platform_version_size; /* out */
} PJRT_TopologyDescription_PlatformVersion_Args;
typedef PJRT_Error* PJRT_TopologyDescription_PlatformVersion(PJRT_TopologyDescription_PlatformVersion_Args* args);
typedef struct PJRT_TopologyDescription_PlatformName_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_TopologyDescription* topology;
  const char* platform_name; /* out */
  size_t platform_name_size; /* out */
} PJRT_TopologyDescription_PlatformName_Args;
typedef PJRT_Error* PJRT_TopologyDescription_PlatformName(PJRT_TopologyDescription_PlatformName_Args* args);
typedef struct PJRT_TopologyDescription_GetDeviceDescriptions_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_TopologyDescription* topology;
  PJRT_DeviceDescription* const* descriptions; /* out */
  size_t num_descriptions;                     /* out */
} PJRT_TopologyDescription_GetDeviceDescriptions_Args;
typedef PJRT_Error* PJRT_TopologyDescription_GetDeviceDescriptions(PJRT_TopologyDescription_GetDeviceDescriptions_Args* args);
typedef struct PJRT_SerializedTopology PJRT_SerializedTopology;
typedef struct PJRT_TopologyDescription_Serialize_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_TopologyDescription* topology;
  const char* serialized_bytes;                   /* out; lives as long as serialized_topology */
  size_t serialized_bytes_size;                   /* out */
  PJRT_SerializedTopology* serialized_topology;   /* out */
  void (*serialized_topology_deleter)(PJRT_SerializedTopology* serialized_topology); /* out; call once */
} PJRT_TopologyDescription_Serialize_Args;
#define PJRT_TopologyDescription_Serialize_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_TopologyDescription_Serialize_Args, serialized_topology_deleter)
typedef PJRT_Error* PJRT_TopologyDescription_Serialize(PJRT_TopologyDescription_Serialize_Args* args);
typedef struct PJRT_TopologyDescription_Attributes_Args {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_TopologyDescription* topology;
  const PJRT_NamedValue* attributes; /* out */
  size_t num_attributes;             /* out */
} PJRT_TopologyDescription_Attributes_Args;
typedef PJRT_Error* PJRT_TopologyDescription_Attributes(PJRT_TopologyDescription_Attributes_Args* args);

typedef struct PJRT_Compile_Args PJRT_Compile_Args;
typedef PJRT_Error* PJRT_Compile(PJRT_Compile_Args* args);

typedef struct PJRT_Client_CreateViewOfDeviceBuffer_Args PJRT_Client_CreateViewOfDeviceBuffer_Args;
typedef PJRT_Error* PJRT_Client_CreateViewOfDeviceBuffer(PJRT_Client_CreateViewOfDeviceBuffer_Args* args);

typedef struct PJRT_ExecuteContext_Create_Args PJRT_ExecuteContext_Create_Args;
typedef PJRT_Error* PJRT_ExecuteContext_Create(PJRT_ExecuteContext_Create_Args* args);
typedef struct PJRT_ExecuteContext_Destroy_Args PJRT_ExecuteContext_Destroy_Args;
typedef PJRT_Error* PJRT_ExecuteContext_Destroy(PJRT_ExecuteContext_Destroy_Args* args);
typedef struct PJRT_Buffer_CopyRawToHost_Args PJRT_Buffer_CopyRawToHost_Args;
typedef PJRT_Error* PJRT_Buffer_CopyRawToHost(PJRT_Buffer_CopyRawToHost_Args* args);
typedef struct PJRT_Client_DmaMap_Args PJRT_Client_DmaMap_Args;
typedef PJRT_Error* PJRT_Client_DmaMap(PJRT_Client_DmaMap_Args* args);
typedef struct PJRT_Client_DmaUnmap_Args PJRT_Client_DmaUnmap_Args;
typedef PJRT_Error* PJRT_Client_DmaUnmap(PJRT_Client_DmaUnmap_Args* args);

/* --------------------------------- The API ------------------------------- */

#define _PJRT_API_STRUCT_FIELD(fn_type) fn_type* fn_type

typedef struct PJRT_Api {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;

  PJRT_Api_Version pjrt_api_version;

  _PJRT_API_STRUCT_FIELD(PJRT_Error_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_Error_Message);
  _PJRT_API_STRUCT_FIELD(PJRT_Error_GetCode);

  _PJRT_API_STRUCT_FIELD(PJRT_Plugin_Initialize);
  _PJRT_API_STRUCT_FIELD(PJRT_Plugin_Attributes);

  _PJRT_API_STRUCT_FIELD(PJRT_Event_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_Event_IsReady);
  _PJRT_API_STRUCT_FIELD(PJRT_Event_Error);
  _PJRT_API_STRUCT_FIELD(PJRT_Event_Await);
  _PJRT_API_STRUCT_FIELD(PJRT_Event_OnReady);

  _PJRT_API_STRUCT_FIELD(PJRT_Client_Create);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_PlatformName);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_ProcessIndex);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_PlatformVersion);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_Devices);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_AddressableDevices);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_LookupDevice);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_LookupAddressableDevice);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_AddressableMemories);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_Compile);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_DefaultDeviceAssignment);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_BufferFromHostBuffer);

  _PJRT_API_STRUCT_FIELD(PJRT_DeviceDescription_Id);
  _PJRT_API_STRUCT_FIELD(PJRT_DeviceDescription_ProcessIndex);
  _PJRT_API_STRUCT_FIELD(PJRT_DeviceDescription_Attributes);
  _PJRT_API_STRUCT_FIELD(PJRT_DeviceDescription_Kind);
  _PJRT_API_STRUCT_FIELD(PJRT_DeviceDescription_DebugString);
  _PJRT_API_STRUCT_FIELD(PJRT_DeviceDescription_ToString);

  _PJRT_API_STRUCT_FIELD(PJRT_Device_GetDescription);
  _PJRT_API_STRUCT_FIELD(PJRT_Device_IsAddressable);
  _PJRT_API_STRUCT_FIELD(PJRT_Device_LocalHardwareId);
  _PJRT_API_STRUCT_FIELD(PJRT_Device_AddressableMemories);
  _PJRT_API_STRUCT_FIELD(PJRT_Device_DefaultMemory);
  _PJRT_API_STRUCT_FIELD(PJRT_Device_MemoryStats);

  _PJRT_API_STRUCT_FIELD(PJRT_Memory_Id);
  _PJRT_API_STRUCT_FIELD(PJRT_Memory_Kind);
  _PJRT_API_STRUCT_FIELD(PJRT_Memory_DebugString);
  _PJRT_API_STRUCT_FIELD(PJRT_Memory_ToString);
  _PJRT_API_STRUCT_FIELD(PJRT_Memory_AddressableByDevices);

  _PJRT_API_STRUCT_FIELD(PJRT_Executable_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_Name);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_NumReplicas);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_NumPartitions);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_NumOutputs);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_SizeOfGeneratedCodeInBytes);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_GetCostAnalysis);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_OutputMemoryKinds);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_OptimizedProgram);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_Serialize);

  _PJRT_API_STRUCT_FIELD(PJRT_LoadedExecutable_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_LoadedExecutable_GetExecutable);
  _PJRT_API_STRUCT_FIELD(PJRT_LoadedExecutable_AddressableDevices);
  _PJRT_API_STRUCT_FIELD(PJRT_LoadedExecutable_Delete);
  _PJRT_API_STRUCT_FIELD(PJRT_LoadedExecutable_IsDeleted);
  _PJRT_API_STRUCT_FIELD(PJRT_LoadedExecutable_Execute);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_DeserializeAndLoad);
  _PJRT_API_STRUCT_FIELD(PJRT_LoadedExecutable_Fingerprint);

  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_ElementType);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_Dimensions);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_UnpaddedDimensions);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_DynamicDimensionIndices);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_GetMemoryLayout);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_OnDeviceSizeInBytes);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_Device);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_Memory);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_Delete);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_IsDeleted);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_CopyToDevice);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_ToHostBuffer);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_IsOnCpu);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_ReadyEvent);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_UnsafePointer);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_IncreaseExternalReferenceCount);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_DecreaseExternalReferenceCount);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_OpaqueDeviceMemoryDataPointer);

  _PJRT_API_STRUCT_FIELD(PJRT_CopyToDeviceStream_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_CopyToDeviceStream_AddChunk);
  _PJRT_API_STRUCT_FIELD(PJRT_CopyToDeviceStream_TotalBytes);
  _PJRT_API_STRUCT_FIELD(PJRT_CopyToDeviceStream_GranuleSize);
  _PJRT_API_STRUCT_FIELD(PJRT_CopyToDeviceStream_CurrentBytes);

  _PJRT_API_STRUCT_FIELD(PJRT_TopologyDescription_Create);
  _PJRT_API_STRUCT_FIELD(PJRT_TopologyDescription_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_TopologyDescription_PlatformName);
  _PJRT_API_STRUCT_FIELD(PJRT_TopologyDescription_PlatformVersion);
  _PJRT_API_STRUCT_FIELD(PJRT_TopologyDescription_GetDeviceDescriptions);
  _PJRT_API_STRUCT_FIELD(PJRT_TopologyDescription_Serialize);
  _PJRT_API_STRUCT_FIELD(PJRT_TopologyDescription_Attributes);

  _PJRT_API_STRUCT_FIELD(PJRT_Compile);

  /* Appended after the 0.x base layout, in this order. */
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_OutputElementTypes);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_OutputDimensions);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_CopyToMemory);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_CreateViewOfDeviceBuffer);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_Fingerprint);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_TopologyDescription);
  _PJRT_API_STRUCT_FIELD(PJRT_Executable_GetCompiledMemoryStats);
  _PJRT_API_STRUCT_FIELD(PJRT_Memory_Kind_Id);
  _PJRT_API_STRUCT_FIELD(PJRT_ExecuteContext_Create);
  _PJRT_API_STRUCT_FIELD(PJRT_ExecuteContext_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_Buffer_CopyRawToHost);
  _PJRT_API_STRUCT_FIELD(PJRT_AsyncHostToDeviceTransferManager_Destroy);
  _PJRT_API_STRUCT_FIELD(PJRT_AsyncHostToDeviceTransferManager_TransferData);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_CreateBuffersForAsyncHostToDevice);
  _PJRT_API_STRUCT_FIELD(PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer);
  _PJRT_API_STRUCT_FIELD(PJRT_AsyncHostToDeviceTransferManager_Device);
  _PJRT_API_STRUCT_FIELD(PJRT_AsyncHostToDeviceTransferManager_BufferCount);
  _PJRT_API_STRUCT_FIELD(PJRT_AsyncHostToDeviceTransferManager_BufferSize);
  _PJRT_API_STRUCT_FIELD(PJRT_AsyncHostToDeviceTransferManager_SetBufferError);
  _PJRT_API_STRUCT_FIELD(PJRT_AsyncHostToDeviceTransferManager_AddMetadata);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_DmaMap);
  _PJRT_API_STRUCT_FIELD(PJRT_Client_DmaUnmap);
} PJRT_Api;

#define PJRT_Api_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Api, PJRT_Client_DmaUnmap)

#undef _PJRT_API_STRUCT_FIELD

/* Entry point every PJRT plugin exports.
 * Replaces reference src/plugin/plugin.zig:11 (`export fn GetPjrtApi`). */
const PJRT_Api* GetPjrtApi(void);

/* ------------------------ GPU custom-call extension ---------------------- */
/* The first (and only) entry of PJRT_Api.extension_start's chain: registers a
 * custom-call target by handler (the public PJRT GPU extension layout; the
 * reference installs the same extension, src/plugin/custom_call.zig:143-156,
 * api.zig:66). api_version 0 (untyped) only; the handler_execute pointer
 * names a pjrtx built-in by address (PjRTx_CustomCall_* in pjrtx_hip.h). */
typedef struct PJRT_Gpu_Register_Custom_Call_Args {
  size_t struct_size;
  const char* function_name;
  size_t function_name_size;
  int api_version;
  void* handler_instantiate;
  void* handler_prepare;
  void* handler_initialize;
  void* handler_execute;
} PJRT_Gpu_Register_Custom_Call_Args;
#define PJRT_Gpu_Register_Custom_Call_Args_STRUCT_SIZE \
  PJRT_STRUCT_SIZE(PJRT_Gpu_Register_Custom_Call_Args, handler_execute)

typedef PJRT_Error* PJRT_Gpu_Register_Custom_Call(PJRT_Gpu_Register_Custom_Call_Args* args);

typedef struct PJRT_Gpu_Custom_Call {
  PJRT_Extension_Base base;
  PJRT_Gpu_Register_Custom_Call* custom_call;
} PJRT_Gpu_Custom_Call;
#define PJRT_Gpu_Custom_Call_STRUCT_SIZE PJRT_STRUCT_SIZE(PJRT_Gpu_Custom_Call, custom_call)

#ifdef __cplusplus
}
#endif

#endif /* PJRTX_AMD_PJRT_C_API_H_ */
