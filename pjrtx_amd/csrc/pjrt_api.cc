// PJRT C-API adapter: GetPjrtApi() and the PJRT_* families JAX calls on the
// compile / transfer / execute path.
//
// Replaces the reference's Zig adapter (reference: src/plugin/plugin.zig:11
// GetPjrtApi, src/plugin/api.zig:40-85 table install, client.zig:28-47,
// 89-105, 290-406, execute.zig:18-337, buffer.zig:17-258, events.zig:61-67,
// errors.zig:90-95, device_memory.zig:21-124, plugin_process.zig:87-133,
// trace.zig:80-120 PJRTX_TRACE lines). Sharding is pinned to one device.
#include <chrono>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/pjrt_c_api.h"
#include "custom_call.h"
#include "pjrt_handles.h"
#include "runtime.h"

using namespace pjrtx;

// ------------------------------------------------------------------ helpers

namespace {

PJRT_Error* make_error(Code c, const std::string& msg) { return new PJRT_Error{c, msg}; }

// Process-wide device objects (one per visible GPU, created on first client).
std::mutex g_dev_mu;
std::vector<std::unique_ptr<Device>> g_devices;

Device* device_for(int ordinal) {
  std::lock_guard<std::mutex> lk(g_dev_mu);
  if (g_devices.empty()) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
      (void)hipGetLastError();
      fail(Code::kFailedPrecondition, "pjrtx: no HIP device is visible (hipGetDeviceCount returned none)");
    }
    g_devices.resize(n);
  }
  PJRTX_CHECK(ordinal >= 0 && ordinal < static_cast<int>(g_devices.size()), Code::kInvalidArgument, "bad device ordinal");
  if (!g_devices[ordinal]) g_devices[ordinal] = std::make_unique<Device>(ordinal);
  return g_devices[ordinal].get();
}

int visible_devices() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

// PJRTX_TRACE=1: one line per API call, in the reference's format
// (reference: src/plugin/trace.zig:80-120).
bool trace_enabled() {
  static bool on = env_flag("PJRTX_TRACE");
  return on;
}

template <typename Fn>
PJRT_Error* guarded(const char* name, Fn&& fn) {
  const auto t0 = std::chrono::steady_clock::now();
  PJRT_Error* err = nullptr;
  try {
    fn();
  } catch (const Error& e) {
    err = make_error(e.code, e.what());
  } catch (const std::exception& e) {
    err = make_error(Code::kInternal, e.what());
  }
  if (trace_enabled()) {
    const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    std::fprintf(stderr, "pjrtx_trace event=pjrt_api_call name=%s failed=%d error_code=%d elapsed_us=%.0f\n", name,
                 err ? 1 : 0, err ? static_cast<int>(err->code) : 0, us);
  }
  return err;
}

#define PJRTX_ARGS_CHECK(args, TYPE, LAST)                                                          \
  PJRTX_CHECK((args) != nullptr && (args)->struct_size >= PJRT_STRUCT_SIZE(TYPE, LAST),            \
              Code::kInvalidArgument, #TYPE ": struct_size too small or args missing")

DType dtype_from_pjrt(PJRT_Buffer_Type t) {
  int v = static_cast<int>(t);
  PJRTX_CHECK(v >= 1 && v <= 13 && v != 14, Code::kUnimplemented,
              strformat("pjrtx: element type %d is not supported", v));
  return static_cast<DType>(v);
}

PJRT_Buffer_Type pjrt_from_dtype(DType t) { return static_cast<PJRT_Buffer_Type>(static_cast<int>(t)); }

PJRT_NamedValue named_string(const char* name, const std::string& value) {
  PJRT_NamedValue v{};
  v.struct_size = PJRT_NamedValue_STRUCT_SIZE;
  v.name = name;
  v.name_size = std::strlen(name);
  v.type = PJRT_NamedValue_kString;
  v.string_value = value.c_str();
  v.value_size = value.size();
  return v;
}

PJRT_NamedValue named_int(const char* name, int64_t value) {
  PJRT_NamedValue v{};
  v.struct_size = PJRT_NamedValue_STRUCT_SIZE;
  v.name = name;
  v.name_size = std::strlen(name);
  v.type = PJRT_NamedValue_kInt64;
  v.int64_value = value;
  v.value_size = 1;
  return v;
}

PJRT_NamedValue named_list(const char* name, const int64_t* values, size_t n) {
  PJRT_NamedValue v{};
  v.struct_size = PJRT_NamedValue_STRUCT_SIZE;
  v.name = name;
  v.name_size = std::strlen(name);
  v.type = PJRT_NamedValue_kInt64List;
  v.int64_array_value = values;
  v.value_size = n;
  return v;
}

// Plugin attributes (reference: src/plugin/plugin_process.zig:13-16,87-106).
const int64_t kStablehloCurrent[3] = {1, 16, 0};
const int64_t kStablehloMinimum[3] = {1, 0, 0};
const std::string kXlaVersion = "local";
const std::string kPlatformName = "pjrtx";

const std::vector<PJRT_NamedValue>& plugin_attributes() {
  static std::vector<PJRT_NamedValue>* attrs = [] {
    auto* v = new std::vector<PJRT_NamedValue>();
    v->push_back(named_string("xla_version", kXlaVersion));
    v->push_back(named_list("stablehlo_current_version", kStablehloCurrent, 3));
    v->push_back(named_list("stablehlo_minimum_version", kStablehloMinimum, 3));
    return v;
  }();
  return *attrs;
}

// Minimal CompileOptionsProto reader: replica / partition counts of
// ExecutableBuildOptionsProto (field 3; num_replicas = 4,
// num_partitions = 5), or the text form "replicas=1; partitions=1"
// (reference: src/runtime/compile_options.zig:1-80,176).
bool read_varint(const uint8_t*& p, const uint8_t* end, uint64_t* out) {
  uint64_t v = 0;
  int shift = 0;
  while (p < end && shift < 64) {
    uint8_t b = *p++;
    v |= static_cast<uint64_t>(b & 0x7f) << shift;
    if (!(b & 0x80)) {
      *out = v;
      return true;
    }
    shift += 7;
  }
  return false;
}

bool skip_field(const uint8_t*& p, const uint8_t* end, int wire) {
  uint64_t tmp;
  switch (wire) {
    case 0: return read_varint(p, end, &tmp);
    case 1: p += 8; return p <= end;
    case 2:
      if (!read_varint(p, end, &tmp)) return false;
      p += tmp;
      return p <= end;
    case 5: p += 4; return p <= end;
    default: return false;
  }
}

void parse_compile_options(const char* data, size_t size, int64_t* replicas, int64_t* partitions) {
  *replicas = 1;
  *partitions = 1;
  if (!data || !size) return;
  std::string s(data, size);
  if (s.find("replicas=") != std::string::npos || s.find("partitions=") != std::string::npos) {
    auto grab = [&](const char* key, int64_t* out) {
      size_t k = s.find(key);
      if (k != std::string::npos) *out = std::atoll(s.c_str() + k + std::strlen(key));
    };
    grab("replicas=", replicas);
    grab("partitions=", partitions);
    return;
  }
  const uint8_t* p = reinterpret_cast<const uint8_t*>(data);
  const uint8_t* end = p + size;
  while (p < end) {
    uint64_t key;
    if (!read_varint(p, end, &key)) return;
    const int field = static_cast<int>(key >> 3), wire = static_cast<int>(key & 7);
    if (field == 3 && wire == 2) {
      uint64_t len;
      if (!read_varint(p, end, &len) || p + len > end) return;
      const uint8_t* q = p;
      const uint8_t* qe = p + len;
      while (q < qe) {
        uint64_t k2;
        if (!read_varint(q, qe, &k2)) break;
        const int f2 = static_cast<int>(k2 >> 3), w2 = static_cast<int>(k2 & 7);
        if ((f2 == 4 || f2 == 5) && w2 == 0) {
          uint64_t v;
          if (!read_varint(q, qe, &v)) break;
          (f2 == 4 ? *replicas : *partitions) = static_cast<int64_t>(v);
        } else if (!skip_field(q, qe, w2)) {
          break;
        }
      }
      p += len;
    } else if (!skip_field(p, end, wire)) {
      return;
    }
  }
}

std::string fingerprint_of(const std::string& text) {
  uint64_t h1 = 1469598103934665603ull, h2 = 0x9e3779b97f4a7c15ull;
  for (unsigned char c : text) {
    h1 = (h1 ^ c) * 1099511628211ull;
    h2 = (h2 ^ c) * 0x100000001b3ull + 0x1234567ull;
  }
  return strformat("pjrtx-%016llx%016llx", static_cast<unsigned long long>(h1), static_cast<unsigned long long>(h2));
}

PJRT_Executable* make_executable_view(const std::shared_ptr<Executable>& exe) {
  auto* e = new PJRT_Executable();
  e->exe = exe;
  const Program& prog = exe->program();
  for (int r : prog.results) {
    const TensorType& t = prog.type(r);
    e->out_types.push_back(pjrt_from_dtype(t.dtype));
    e->out_ranks.push_back(t.dims.size());
    for (int64_t d : t.dims) e->out_dims.push_back(d);
    e->out_kinds.push_back("device");
    e->out_kind_sizes.push_back(6);
  }
  return e;
}

}  // namespace

// ------------------------------------------------------------------- errors

static void Error_Destroy(PJRT_Error_Destroy_Args* args) {
  if (args && args->error) delete args->error;
}

static void Error_Message(PJRT_Error_Message_Args* args) {
  if (!args || !args->error) return;
  args->message = args->error->message.c_str();
  args->message_size = args->error->message.size();
}

static PJRT_Error* Error_GetCode(PJRT_Error_GetCode_Args* args) {
  return guarded("PJRT_Error_GetCode", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Error_GetCode_Args, code);
    args->code = static_cast<PJRT_Error_Code>(static_cast<int>(args->error->code));
  });
}

// ------------------------------------------------------------------- plugin

static PJRT_Error* Plugin_Initialize(PJRT_Plugin_Initialize_Args* args) {
  return guarded("PJRT_Plugin_Initialize", [&] { (void)args; });
}

static PJRT_Error* Plugin_Attributes(PJRT_Plugin_Attributes_Args* args) {
  return guarded("PJRT_Plugin_Attributes", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Plugin_Attributes_Args, num_attributes);
    const auto& a = plugin_attributes();
    args->attributes = a.data();
    args->num_attributes = a.size();
  });
}

// -------------------------------------------------------------------- event

static PJRT_Error* Event_Destroy(PJRT_Event_Destroy_Args* args) {
  return guarded("PJRT_Event_Destroy", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Event_Destroy_Args, event);
    delete args->event;
  });
}

static PJRT_Error* Event_IsReady(PJRT_Event_IsReady_Args* args) {
  return guarded("PJRT_Event_IsReady", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Event_IsReady_Args, is_ready);
    args->is_ready = args->event->ev->is_ready();
  });
}

static PJRT_Error* Event_Error(PJRT_Event_Error_Args* args) {
  PJRT_Error* outer = nullptr;
  PJRT_Error* inner = guarded("PJRT_Event_Error", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Event_Error_Args, event);
    auto& ev = args->event->ev;
    ev->is_ready();
    if (ev->error_code() != Code::kOk) outer = make_error(ev->error_code(), ev->error_message());
  });
  return inner ? inner : outer;
}

static PJRT_Error* Event_Await(PJRT_Event_Await_Args* args) {
  PJRT_Error* outer = nullptr;
  PJRT_Error* inner = guarded("PJRT_Event_Await", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Event_Await_Args, event);
    auto& ev = args->event->ev;
    ev->await();
    if (ev->error_code() != Code::kOk) outer = make_error(ev->error_code(), ev->error_message());
  });
  return inner ? inner : outer;
}

static PJRT_Error* Event_OnReady(PJRT_Event_OnReady_Args* args) {
  return guarded("PJRT_Event_OnReady", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Event_OnReady_Args, user_arg);
    std::shared_ptr<Event> ev = args->event->ev;
    PJRT_Event_OnReadyCallback cb = args->callback;
    void* user = args->user_arg;
    ev->on_ready([ev, cb, user] {
      PJRT_Error* e = ev->error_code() == Code::kOk ? nullptr : make_error(ev->error_code(), ev->error_message());
      cb(e, user);
    });
  });
}

// ------------------------------------------------------------------- client

static PJRT_Error* Client_Create(PJRT_Client_Create_Args* args) {
  return guarded("PJRT_Client_Create", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_Create_Args, client);
    // Accepted options (reference: src/plugin/client.zig:89-105): only
    // `pjrtx_backend`, whose value must name this backend.
    for (size_t i = 0; i < args->num_options; ++i) {
      const PJRT_NamedValue& o = args->create_options[i];
      std::string name(o.name, o.name_size);
      if (name == "pjrtx_backend") {
        PJRTX_CHECK(o.type == PJRT_NamedValue_kString, Code::kInvalidArgument, "pjrtx_backend must be a string");
        std::string v(o.string_value, o.value_size);
        PJRTX_CHECK(v == "rocm" || v == "hip" || v == "mi355x" || v == "default", Code::kInvalidArgument,
                    "pjrtx_backend '" + v + "' is not available; this plugin provides 'rocm'");
        continue;
      }
      fail(Code::kInvalidArgument, "unknown client create option '" + name + "'");
    }
    const int n = visible_devices();
    PJRTX_CHECK(n > 0, Code::kFailedPrecondition, "pjrtx: no HIP device is visible");
    auto* c = new PJRT_Client();
    c->topology.client = c;
    c->platform_version = "pjrtx-rocm (HIP " + std::to_string(HIP_VERSION_MAJOR) + "." +
                          std::to_string(HIP_VERSION_MINOR) + ")";
    for (int i = 0; i < n; ++i) {
      Device* dev = device_for(i);
      auto d = std::make_unique<PJRT_Device>();
      d->dev = dev;
      d->client = c;
      d->desc.id = i;
      d->desc.kind = dev->name().empty() ? "AMD Instinct" : dev->name();
      d->desc.debug = strformat("pjrtx:%d(%s)", i, dev->arch().c_str());
      d->desc.to_string = strformat("PjrtxDevice(id=%d, arch=%s)", i, dev->arch().c_str());
      d->desc.attr_strings.push_back(dev->arch());
      d->desc.attrs.push_back(named_string("gfx_arch", d->desc.attr_strings.back()));
      d->desc.attrs.push_back(named_int("compute_units", dev->compute_units()));
      d->desc.attrs.push_back(named_int("local_hardware_id", i));
      auto m = std::make_unique<PJRT_Memory>();
      m->id = i;
      m->device = d.get();
      m->debug = strformat("pjrtx:device_memory:%d", i);
      m->to_string = strformat("MEMORY_SPACE(device, id=%d)", i);
      d->memory = m.get();
      c->devices.push_back(d.get());
      c->memories.push_back(m.get());
      c->device_storage.push_back(std::move(d));
      c->memory_storage.push_back(std::move(m));
    }
    args->client = c;
  });
}

static PJRT_Error* Client_Destroy(PJRT_Client_Destroy_Args* args) {
  return guarded("PJRT_Client_Destroy", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_Destroy_Args, client);
    delete args->client;
  });
}

static PJRT_Error* Client_PlatformName(PJRT_Client_PlatformName_Args* args) {
  return guarded("PJRT_Client_PlatformName", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_PlatformName_Args, platform_name_size);
    args->platform_name = kPlatformName.c_str();
    args->platform_name_size = kPlatformName.size();
  });
}

static PJRT_Error* Client_ProcessIndex(PJRT_Client_ProcessIndex_Args* args) {
  return guarded("PJRT_Client_ProcessIndex", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_ProcessIndex_Args, process_index);
    args->process_index = 0;
  });
}

static PJRT_Error* Client_PlatformVersion(PJRT_Client_PlatformVersion_Args* args) {
  return guarded("PJRT_Client_PlatformVersion", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_PlatformVersion_Args, platform_version_size);
    args->platform_version = args->client->platform_version.c_str();
    args->platform_version_size = args->client->platform_version.size();
  });
}

static PJRT_Error* Client_TopologyDescription(PJRT_Client_TopologyDescription_Args* args) {
  return guarded("PJRT_Client_TopologyDescription", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_TopologyDescription_Args, topology);
    args->topology = &args->client->topology;
  });
}

static PJRT_Error* Client_Devices(PJRT_Client_Devices_Args* args) {
  return guarded("PJRT_Client_Devices", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_Devices_Args, num_devices);
    args->devices = args->client->devices.data();
    args->num_devices = args->client->devices.size();
  });
}

static PJRT_Error* Client_AddressableDevices(PJRT_Client_AddressableDevices_Args* args) {
  return guarded("PJRT_Client_AddressableDevices", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_AddressableDevices_Args, num_addressable_devices);
    args->addressable_devices = args->client->devices.data();
    args->num_addressable_devices = args->client->devices.size();
  });
}

static PJRT_Error* Client_LookupDevice(PJRT_Client_LookupDevice_Args* args) {
  return guarded("PJRT_Client_LookupDevice", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_LookupDevice_Args, device);
    PJRTX_CHECK(args->id >= 0 && args->id < static_cast<int>(args->client->devices.size()), Code::kInvalidArgument,
                strformat("no device with id %d", args->id));
    args->device = args->client->devices[args->id];
  });
}

static PJRT_Error* Client_LookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* args) {
  return guarded("PJRT_Client_LookupAddressableDevice", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_LookupAddressableDevice_Args, addressable_device);
    const int id = args->local_hardware_id;
    PJRTX_CHECK(id >= 0 && id < static_cast<int>(args->client->devices.size()), Code::kInvalidArgument,
                strformat("no addressable device with local hardware id %d", id));
    args->addressable_device = args->client->devices[id];
  });
}

static PJRT_Error* Client_AddressableMemories(PJRT_Client_AddressableMemories_Args* args) {
  return guarded("PJRT_Client_AddressableMemories", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_AddressableMemories_Args, num_addressable_memories);
    args->addressable_memories = args->client->memories.data();
    args->num_addressable_memories = args->client->memories.size();
  });
}

static PJRT_Error* Client_Compile(PJRT_Client_Compile_Args* args) {
  return guarded("PJRT_Client_Compile", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_Compile_Args, executable);
    PJRTX_CHECK(args->program && args->program->code, Code::kInvalidArgument, "Compile: program is missing");
    std::string format(args->program->format, args->program->format_size);
    PJRTX_CHECK(format == "mlir", Code::kInvalidArgument, "Compile: program format must be 'mlir', got '" + format + "'");
    int64_t replicas = 1, partitions = 1;
    parse_compile_options(args->compile_options, args->compile_options_size, &replicas, &partitions);
    PJRTX_CHECK(replicas == 1 && partitions == 1, Code::kUnimplemented,
                strformat("pjrtx runs on one device: compile asked for %lld replicas x %lld partitions",
                          static_cast<long long>(replicas), static_cast<long long>(partitions)));
    std::string text(args->program->code, args->program->code_size);
    std::shared_ptr<const CompiledProgram> cp = compile_program_cached(text);
    PJRTX_CHECK(cp->prog.num_partitions == 1 && cp->prog.num_replicas == 1, Code::kUnimplemented,
                "pjrtx runs on one device: module asks for more than one partition or replica");
    std::string name = cp->prog.module_name.empty() ? "main" : cp->prog.module_name;
    auto exe = std::make_shared<Executable>(cp->prog, cp->plan, fingerprint_of(text), name);
    PJRT_Device* d0 = args->client->devices.at(0);
    exe->load(d0->dev);  // compile kernels and upload constants now
    auto* le = new PJRT_LoadedExecutable();
    le->exe = exe;
    le->client = args->client;
    le->devices = {d0};
    args->executable = le;
  });
}

static PJRT_Error* Client_DefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* args) {
  return guarded("PJRT_Client_DefaultDeviceAssignment", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_DefaultDeviceAssignment_Args, default_assignment);
    const int n = args->num_replicas * args->num_partitions;
    PJRTX_CHECK(n == 1, Code::kUnimplemented, "pjrtx runs on one device");
    PJRTX_CHECK(args->default_assignment_size >= 1, Code::kInvalidArgument, "assignment buffer too small");
    args->default_assignment[0] = 0;
  });
}

static PJRT_Error* Client_BufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* args) {
  return guarded("PJRT_Client_BufferFromHostBuffer", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_BufferFromHostBuffer_Args, buffer);
    PJRT_Device* d = args->device;
    if (!d && args->memory) d = args->memory->device;
    if (!d) d = args->client->devices.at(0);
    TensorType t;
    t.dtype = dtype_from_pjrt(args->type);
    t.dims.assign(args->dims, args->dims + args->num_dims);
    for (int64_t x : t.dims) PJRTX_CHECK(x >= 0, Code::kInvalidArgument, "negative dimension");
    const int64_t* strides = (args->byte_strides && args->num_byte_strides == args->num_dims) ? args->byte_strides : nullptr;
    PJRTX_CHECK(args->data || t.bytes() == 0, Code::kInvalidArgument, "BufferFromHostBuffer: data is null");
    BufferRef b = buffer_from_host(d->dev, t, args->data, strides);
    auto* pb = new PJRT_Buffer();
    pb->buf = b;
    pb->client = args->client;
    pb->device = d;
    args->buffer = pb;
    args->done_with_host_buffer = new PJRT_Event{Event::ready()};
  });
}

// ----------------------------------------------------- async host transfers
// (reference: src/plugin/async_h2d.zig:196-437, client.zig:420-440)

static PJRT_AsyncHostToDeviceTransferManager* manager_of(PJRT_AsyncHostToDeviceTransferManager* m) {
  PJRTX_CHECK(m != nullptr && m->t != nullptr, Code::kInvalidArgument, "transfer manager is null");
  return m;
}

static size_t transfer_index(PJRT_AsyncHostToDeviceTransferManager* m, int i) {
  PJRTX_CHECK(i >= 0 && static_cast<size_t>(i) < m->t->count(), Code::kInvalidArgument,
              "async transfer buffer index is out of range");
  return static_cast<size_t>(i);
}

static PJRT_Error* Client_CreateBuffersForAsyncHostToDevice(PJRT_Client_CreateBuffersForAsyncHostToDevice_Args* args) {
  return guarded("PJRT_Client_CreateBuffersForAsyncHostToDevice", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Client_CreateBuffersForAsyncHostToDevice_Args, transfer_manager);
    PJRTX_CHECK(args->shape_specs != nullptr || args->num_shape_specs == 0, Code::kInvalidArgument,
                "shape specs are null");
    for (size_t i = 0; i < args->num_device_layouts; ++i)
      PJRTX_CHECK(args->device_layouts == nullptr || args->device_layouts[i] == nullptr, Code::kUnimplemented,
                  "async transfers take the default (dense row-major) layout only");
    PJRT_Device* d = args->memory ? args->memory->device : args->client->devices.at(0);
    std::vector<TensorType> types;
    for (size_t i = 0; i < args->num_shape_specs; ++i) {
      const PJRT_ShapeSpec& sp = args->shape_specs[i];
      PJRTX_CHECK(sp.dims != nullptr || sp.num_dims == 0, Code::kInvalidArgument, "shape spec dimensions are null");
      TensorType t;
      t.dtype = dtype_from_pjrt(sp.element_type);
      t.dims.assign(sp.dims, sp.dims + sp.num_dims);
      for (int64_t x : t.dims) PJRTX_CHECK(x >= 0, Code::kInvalidArgument, "negative dimension");
      types.push_back(t);
    }
    auto* m = new PJRT_AsyncHostToDeviceTransferManager();
    m->t = std::make_unique<AsyncTransfer>(d->dev, types);
    m->client = args->client;
    m->device = d;
    args->transfer_manager = m;
  });
}

static PJRT_Error* Transfer_Destroy(PJRT_AsyncHostToDeviceTransferManager_Destroy_Args* args) {
  return guarded("PJRT_AsyncHostToDeviceTransferManager_Destroy", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_AsyncHostToDeviceTransferManager_Destroy_Args, transfer_manager);
    delete args->transfer_manager;  // retrieved buffers keep their memory
  });
}

static PJRT_Error* Transfer_TransferData(PJRT_AsyncHostToDeviceTransferManager_TransferData_Args* args) {
  return guarded("PJRT_AsyncHostToDeviceTransferManager_TransferData", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_AsyncHostToDeviceTransferManager_TransferData_Args, done_with_h2d_transfer);
    auto* m = manager_of(args->transfer_manager);
    const size_t i = transfer_index(m, args->buffer_index);
    auto done = m->t->write(i, args->offset, args->data, args->transfer_size, args->is_last_transfer);
    args->done_with_h2d_transfer = new PJRT_Event{done};
  });
}

static PJRT_Error* Transfer_RetrieveBuffer(PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer_Args* args) {
  return guarded("PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer_Args, buffer_out);
    auto* m = manager_of(args->transfer_manager);
    auto* pb = new PJRT_Buffer();
    pb->buf = m->t->buffer(transfer_index(m, args->buffer_index));
    pb->client = m->client;
    pb->device = m->device;
    args->buffer_out = pb;
  });
}

static PJRT_Error* Transfer_Device(PJRT_AsyncHostToDeviceTransferManager_Device_Args* args) {
  return guarded("PJRT_AsyncHostToDeviceTransferManager_Device", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_AsyncHostToDeviceTransferManager_Device_Args, device_out);
    args->device_out = manager_of(args->transfer_manager)->device;
  });
}

static PJRT_Error* Transfer_BufferCount(PJRT_AsyncHostToDeviceTransferManager_BufferCount_Args* args) {
  return guarded("PJRT_AsyncHostToDeviceTransferManager_BufferCount", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_AsyncHostToDeviceTransferManager_BufferCount_Args, buffer_count);
    args->buffer_count = manager_of(args->transfer_manager)->t->count();
  });
}

static PJRT_Error* Transfer_BufferSize(PJRT_AsyncHostToDeviceTransferManager_BufferSize_Args* args) {
  return guarded("PJRT_AsyncHostToDeviceTransferManager_BufferSize", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_AsyncHostToDeviceTransferManager_BufferSize_Args, buffer_size);
    auto* m = manager_of(args->transfer_manager);
    args->buffer_size = m->t->bytes(transfer_index(m, args->buffer_index));
  });
}

static PJRT_Error* Transfer_SetBufferError(PJRT_AsyncHostToDeviceTransferManager_SetBufferError_Args* args) {
  return guarded("PJRT_AsyncHostToDeviceTransferManager_SetBufferError", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_AsyncHostToDeviceTransferManager_SetBufferError_Args, error_message_size);
    auto* m = manager_of(args->transfer_manager);
    const std::string msg = args->error_message ? std::string(args->error_message, args->error_message_size)
                                                : std::string("async transfer buffer failed");
    m->t->fail(transfer_index(m, args->buffer_index), static_cast<Code>(args->error_code), msg);
  });
}

static PJRT_Error* Transfer_AddMetadata(PJRT_AsyncHostToDeviceTransferManager_AddMetadata_Args* args) {
  return guarded("PJRT_AsyncHostToDeviceTransferManager_AddMetadata", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_AsyncHostToDeviceTransferManager_AddMetadata_Args, num_metadata);
    manager_of(args->transfer_manager);  // metadata is informational here
  });
}

// ------------------------------------------------------- device description

static PJRT_Error* DeviceDescription_Id(PJRT_DeviceDescription_Id_Args* args) {
  return guarded("PJRT_DeviceDescription_Id", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_DeviceDescription_Id_Args, id);
    args->id = args->device_description->id;
  });
}

static PJRT_Error* DeviceDescription_ProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* args) {
  return guarded("PJRT_DeviceDescription_ProcessIndex", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_DeviceDescription_ProcessIndex_Args, process_index);
    args->process_index = 0;
  });
}

static PJRT_Error* DeviceDescription_Attributes(PJRT_DeviceDescription_Attributes_Args* args) {
  return guarded("PJRT_DeviceDescription_Attributes", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_DeviceDescription_Attributes_Args, attributes);
    args->attributes = args->device_description->attrs.data();
    args->num_attributes = args->device_description->attrs.size();
  });
}

static PJRT_Error* DeviceDescription_Kind(PJRT_DeviceDescription_Kind_Args* args) {
  return guarded("PJRT_DeviceDescription_Kind", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_DeviceDescription_Kind_Args, device_kind_size);
    args->device_kind = args->device_description->kind.c_str();
    args->device_kind_size = args->device_description->kind.size();
  });
}

static PJRT_Error* DeviceDescription_DebugString(PJRT_DeviceDescription_DebugString_Args* args) {
  return guarded("PJRT_DeviceDescription_DebugString", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_DeviceDescription_DebugString_Args, debug_string_size);
    args->debug_string = args->device_description->debug.c_str();
    args->debug_string_size = args->device_description->debug.size();
  });
}

static PJRT_Error* DeviceDescription_ToString(PJRT_DeviceDescription_ToString_Args* args) {
  return guarded("PJRT_DeviceDescription_ToString", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_DeviceDescription_ToString_Args, to_string_size);
    args->to_string = args->device_description->to_string.c_str();
    args->to_string_size = args->device_description->to_string.size();
  });
}

// ------------------------------------------------------------------- device

static PJRT_Error* Device_GetDescription(PJRT_Device_GetDescription_Args* args) {
  return guarded("PJRT_Device_GetDescription", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Device_GetDescription_Args, device_description);
    args->device_description = &args->device->desc;
  });
}

static PJRT_Error* Device_IsAddressable(PJRT_Device_IsAddressable_Args* args) {
  return guarded("PJRT_Device_IsAddressable", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Device_IsAddressable_Args, is_addressable);
    args->is_addressable = true;
  });
}

static PJRT_Error* Device_LocalHardwareId(PJRT_Device_LocalHardwareId_Args* args) {
  return guarded("PJRT_Device_LocalHardwareId", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Device_LocalHardwareId_Args, local_hardware_id);
    args->local_hardware_id = args->device->dev->ordinal();
  });
}

static PJRT_Error* Device_AddressableMemories(PJRT_Device_AddressableMemories_Args* args) {
  return guarded("PJRT_Device_AddressableMemories", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Device_AddressableMemories_Args, num_memories);
    args->memories = &args->device->memory;
    args->num_memories = 1;
  });
}

static PJRT_Error* Device_DefaultMemory(PJRT_Device_DefaultMemory_Args* args) {
  return guarded("PJRT_Device_DefaultMemory", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Device_DefaultMemory_Args, memory);
    args->memory = args->device->memory;
  });
}

static PJRT_Error* Device_MemoryStats(PJRT_Device_MemoryStats_Args* args) {
  return guarded("PJRT_Device_MemoryStats", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Device_MemoryStats_Args, bytes_in_use);
    Allocator& a = args->device->dev->allocator();
    args->bytes_in_use = a.bytes_in_use();
    if (args->struct_size >= PJRT_Device_MemoryStats_Args_STRUCT_SIZE) {
      args->peak_bytes_in_use = a.peak_bytes_in_use();
      args->peak_bytes_in_use_is_set = true;
      args->num_allocs = a.num_allocs();
      args->num_allocs_is_set = true;
      args->largest_alloc_size = a.largest_alloc();
      args->largest_alloc_size_is_set = true;
      args->bytes_limit = args->device->dev->total_memory();
      args->bytes_limit_is_set = true;
      args->bytes_reserved = a.bytes_reserved();
      args->bytes_reserved_is_set = true;
    }
  });
}

// ------------------------------------------------------------------- memory

static PJRT_Error* Memory_Id(PJRT_Memory_Id_Args* args) {
  return guarded("PJRT_Memory_Id", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Memory_Id_Args, id);
    args->id = args->memory->id;
  });
}

static PJRT_Error* Memory_Kind(PJRT_Memory_Kind_Args* args) {
  return guarded("PJRT_Memory_Kind", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Memory_Kind_Args, kind_size);
    args->kind = args->memory->kind.c_str();
    args->kind_size = args->memory->kind.size();
  });
}

static PJRT_Error* Memory_Kind_Id(PJRT_Memory_Kind_Id_Args* args) {
  return guarded("PJRT_Memory_Kind_Id", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Memory_Kind_Id_Args, kind_id);
    args->kind_id = 0;
  });
}

static PJRT_Error* Memory_DebugString(PJRT_Memory_DebugString_Args* args) {
  return guarded("PJRT_Memory_DebugString", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Memory_DebugString_Args, debug_string_size);
    args->debug_string = args->memory->debug.c_str();
    args->debug_string_size = args->memory->debug.size();
  });
}

static PJRT_Error* Memory_ToString(PJRT_Memory_ToString_Args* args) {
  return guarded("PJRT_Memory_ToString", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Memory_ToString_Args, to_string_size);
    args->to_string = args->memory->to_string.c_str();
    args->to_string_size = args->memory->to_string.size();
  });
}

static PJRT_Error* Memory_AddressableByDevices(PJRT_Memory_AddressableByDevices_Args* args) {
  return guarded("PJRT_Memory_AddressableByDevices", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Memory_AddressableByDevices_Args, num_devices);
    args->devices = &args->memory->device;
    args->num_devices = 1;
  });
}

// --------------------------------------------------------------- executable

static PJRT_Error* Executable_Destroy(PJRT_Executable_Destroy_Args* args) {
  return guarded("PJRT_Executable_Destroy", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_Destroy_Args, executable);
    delete args->executable;
  });
}

static PJRT_Error* Executable_Name(PJRT_Executable_Name_Args* args) {
  return guarded("PJRT_Executable_Name", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_Name_Args, executable_name_size);
    args->executable_name = args->executable->exe->name().c_str();
    args->executable_name_size = args->executable->exe->name().size();
  });
}

static PJRT_Error* Executable_NumReplicas(PJRT_Executable_NumReplicas_Args* args) {
  return guarded("PJRT_Executable_NumReplicas", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_NumReplicas_Args, num_replicas);
    args->num_replicas = 1;
  });
}

static PJRT_Error* Executable_NumPartitions(PJRT_Executable_NumPartitions_Args* args) {
  return guarded("PJRT_Executable_NumPartitions", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_NumPartitions_Args, num_partitions);
    args->num_partitions = 1;
  });
}

static PJRT_Error* Executable_NumOutputs(PJRT_Executable_NumOutputs_Args* args) {
  return guarded("PJRT_Executable_NumOutputs", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_NumOutputs_Args, num_outputs);
    args->num_outputs = args->executable->exe->program().results.size();
  });
}

static PJRT_Error* Executable_SizeOfGeneratedCodeInBytes(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* args) {
  return guarded("PJRT_Executable_SizeOfGeneratedCodeInBytes", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_SizeOfGeneratedCodeInBytes_Args, size_in_bytes);
    args->size_in_bytes = static_cast<int64_t>(args->executable->exe->code_size());
  });
}

static PJRT_Error* Executable_GetCostAnalysis(PJRT_Executable_GetCostAnalysis_Args* args) {
  return guarded("PJRT_Executable_GetCostAnalysis", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_GetCostAnalysis_Args, properties);
    args->num_properties = 0;
    args->properties = nullptr;
  });
}

static PJRT_Error* Executable_OutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* args) {
  return guarded("PJRT_Executable_OutputMemoryKinds", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_OutputMemoryKinds_Args, memory_kind_sizes);
    args->num_outputs = args->executable->out_kinds.size();
    args->memory_kinds = args->executable->out_kinds.data();
    args->memory_kind_sizes = args->executable->out_kind_sizes.data();
  });
}

static PJRT_Error* Executable_OptimizedProgram(PJRT_Executable_OptimizedProgram_Args* args) {
  return guarded("PJRT_Executable_OptimizedProgram", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_OptimizedProgram_Args, program);
    PJRT_Executable* e = args->executable;
    if (e->optimized_text.empty()) {
      e->optimized_text = e->exe->plan().describe(e->exe->program());
    }
    PJRT_Program* p = args->program;
    static const char kFormat[] = "pjrtx-plan-json";
    p->format = kFormat;
    p->format_size = sizeof(kFormat) - 1;
    if (!p->code) {
      p->code_size = e->optimized_text.size();
      return;
    }
    PJRTX_CHECK(p->code_size >= e->optimized_text.size(), Code::kInvalidArgument, "OptimizedProgram: buffer too small");
    std::memcpy(p->code, e->optimized_text.data(), e->optimized_text.size());
    p->code_size = e->optimized_text.size();
  });
}

static PJRT_Error* Executable_OutputElementTypes(PJRT_Executable_OutputElementTypes_Args* args) {
  return guarded("PJRT_Executable_OutputElementTypes", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_OutputElementTypes_Args, num_output_types);
    args->output_types = args->executable->out_types.data();
    args->num_output_types = args->executable->out_types.size();
  });
}

static PJRT_Error* Executable_OutputDimensions(PJRT_Executable_OutputDimensions_Args* args) {
  return guarded("PJRT_Executable_OutputDimensions", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_OutputDimensions_Args, dim_sizes);
    args->num_outputs = args->executable->out_ranks.size();
    args->dims = args->executable->out_dims.data();
    args->dim_sizes = args->executable->out_ranks.data();
  });
}

static PJRT_Error* Executable_Fingerprint(PJRT_Executable_Fingerprint_Args* args) {
  return guarded("PJRT_Executable_Fingerprint", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Executable_Fingerprint_Args, executable_fingerprint_size);
    args->executable_fingerprint = args->executable->exe->fingerprint().c_str();
    args->executable_fingerprint_size = args->executable->exe->fingerprint().size();
  });
}

// -------------------------------------------------------- loaded executable

static PJRT_Error* LoadedExecutable_Destroy(PJRT_LoadedExecutable_Destroy_Args* args) {
  return guarded("PJRT_LoadedExecutable_Destroy", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_LoadedExecutable_Destroy_Args, executable);
    delete args->executable;
  });
}

static PJRT_Error* LoadedExecutable_GetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* args) {
  return guarded("PJRT_LoadedExecutable_GetExecutable", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_LoadedExecutable_GetExecutable_Args, executable);
    args->executable = make_executable_view(args->loaded_executable->exe);
  });
}

static PJRT_Error* LoadedExecutable_AddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* args) {
  return guarded("PJRT_LoadedExecutable_AddressableDevices", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_LoadedExecutable_AddressableDevices_Args, num_addressable_devices);
    args->addressable_devices = args->executable->devices.data();
    args->num_addressable_devices = args->executable->devices.size();
  });
}

static PJRT_Error* LoadedExecutable_Delete(PJRT_LoadedExecutable_Delete_Args* args) {
  return guarded("PJRT_LoadedExecutable_Delete", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_LoadedExecutable_Delete_Args, executable);
    args->executable->deleted = true;  // idempotent; metadata kept until Destroy
  });
}

static PJRT_Error* LoadedExecutable_IsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* args) {
  return guarded("PJRT_LoadedExecutable_IsDeleted", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_LoadedExecutable_IsDeleted_Args, is_deleted);
    args->is_deleted = args->executable->deleted;
  });
}

static PJRT_Error* LoadedExecutable_Fingerprint(PJRT_LoadedExecutable_Fingerprint_Args* args) {
  return guarded("PJRT_LoadedExecutable_Fingerprint", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_LoadedExecutable_Fingerprint_Args, executable_fingerprint_size);
    args->executable_fingerprint = args->executable->exe->fingerprint().c_str();
    args->executable_fingerprint_size = args->executable->exe->fingerprint().size();
  });
}

// Execute (reference: src/plugin/execute.zig:137-337): validate, run on the
// single device, fill output_lists and the completion event. Outputs are
// nulled first and destroyed again if anything fails.
static PJRT_Error* LoadedExecutable_Execute(PJRT_LoadedExecutable_Execute_Args* args) {
  return guarded("PJRT_LoadedExecutable_Execute", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_LoadedExecutable_Execute_Args, execute_device);
    PJRT_LoadedExecutable* le = args->executable;
    PJRTX_CHECK(!le->deleted, Code::kFailedPrecondition, "Execute: executable was deleted");
    PJRTX_CHECK(args->num_devices == 1, Code::kInvalidArgument,
                strformat("Execute: pjrtx runs on one device, got num_devices=%zu", args->num_devices));
    PJRTX_CHECK(args->output_lists && args->output_lists[0], Code::kInvalidArgument, "Execute: output_lists is null");
    const Program& prog = le->exe->program();
    const size_t nout = prog.results.size();
    for (size_t i = 0; i < nout; ++i) args->output_lists[0][i] = nullptr;
    if (args->device_complete_events) args->device_complete_events[0] = nullptr;
    PJRTX_CHECK(args->num_args == prog.params.size(), Code::kInvalidArgument,
                strformat("Execute: expected %zu arguments, got %zu", prog.params.size(), args->num_args));
    PJRT_Device* d = args->execute_device ? args->execute_device : le->devices[0];
    std::vector<BufferRef> in;
    for (size_t i = 0; i < args->num_args; ++i) {
      PJRT_Buffer* b = args->argument_lists[0][i];
      PJRTX_CHECK(b != nullptr, Code::kInvalidArgument, strformat("Execute: argument %zu is null", i));
      PJRTX_CHECK(!b->buf->deleted, Code::kInvalidArgument, strformat("Execute: argument %zu was deleted or donated", i));
      in.push_back(b->buf);
    }
    // Donation (reference: execute.zig:40-70): an argument whose parameter
    // carries tf.aliasing_output / jax.buffer_donor is donated unless the
    // caller lists it as non-donatable or passes the same buffer twice.
    const std::vector<int>& alias = prog.param_alias;
    std::vector<bool> donate(in.size(), false);
    for (size_t i = 0; i < in.size(); ++i) donate[i] = i < alias.size() && alias[i] != -1;
    if (args->options && args->options->non_donatable_input_indices) {
      for (size_t k = 0; k < args->options->num_non_donatable_input_indices; ++k) {
        const int64_t idx = args->options->non_donatable_input_indices[k];
        if (idx >= 0 && static_cast<size_t>(idx) < donate.size()) donate[idx] = false;
      }
    }
    for (size_t i = 0; i < in.size(); ++i)
      for (size_t j = 0; j < in.size(); ++j)
        if (i != j && in[i].get() == in[j].get()) donate[i] = false;
    std::shared_ptr<Event> done;
    std::vector<BufferRef> outs = le->exe->execute(d->dev, in, &done, &donate);
    for (size_t i = 0; i < in.size(); ++i) {
      if (!donate[i]) continue;
      in[i]->deleted = true;  // the memory now belongs to the results
      in[i]->mem.reset();
    }
    for (size_t i = 0; i < nout; ++i) {
      auto* pb = new PJRT_Buffer();
      pb->buf = outs[i];
      pb->client = le->client;
      pb->device = d;
      args->output_lists[0][i] = pb;
    }
    if (args->device_complete_events) args->device_complete_events[0] = new PJRT_Event{done};
  });
}

// ------------------------------------------------------------------- buffer

static PJRT_Error* Buffer_Destroy(PJRT_Buffer_Destroy_Args* args) {
  return guarded("PJRT_Buffer_Destroy", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_Destroy_Args, buffer);
    delete args->buffer;
  });
}

static PJRT_Error* Buffer_ElementType(PJRT_Buffer_ElementType_Args* args) {
  return guarded("PJRT_Buffer_ElementType", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_ElementType_Args, type);
    args->type = pjrt_from_dtype(args->buffer->buf->type.dtype);
  });
}

static PJRT_Error* Buffer_Dimensions(PJRT_Buffer_Dimensions_Args* args) {
  return guarded("PJRT_Buffer_Dimensions", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_Dimensions_Args, num_dims);
    args->dims = args->buffer->buf->type.dims.data();
    args->num_dims = args->buffer->buf->type.dims.size();
  });
}

static PJRT_Error* Buffer_UnpaddedDimensions(PJRT_Buffer_UnpaddedDimensions_Args* args) {
  return guarded("PJRT_Buffer_UnpaddedDimensions", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_UnpaddedDimensions_Args, num_dims);
    args->unpadded_dims = args->buffer->buf->type.dims.data();
    args->num_dims = args->buffer->buf->type.dims.size();
  });
}

static PJRT_Error* Buffer_DynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* args) {
  return guarded("PJRT_Buffer_DynamicDimensionIndices", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_DynamicDimensionIndices_Args, num_dynamic_dims);
    args->dynamic_dim_indices = nullptr;
    args->num_dynamic_dims = 0;
  });
}

static PJRT_Error* Buffer_OnDeviceSizeInBytes(PJRT_Buffer_OnDeviceSizeInBytes_Args* args) {
  return guarded("PJRT_Buffer_OnDeviceSizeInBytes", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_OnDeviceSizeInBytes_Args, on_device_size_in_bytes);
    args->on_device_size_in_bytes = args->buffer->buf->type.bytes();
  });
}

static PJRT_Error* Buffer_Device(PJRT_Buffer_Device_Args* args) {
  return guarded("PJRT_Buffer_Device", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_Device_Args, device);
    args->device = args->buffer->device;
  });
}

static PJRT_Error* Buffer_Memory(PJRT_Buffer_Memory_Args* args) {
  return guarded("PJRT_Buffer_Memory", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_Memory_Args, memory);
    args->memory = args->buffer->device->memory;
  });
}

static PJRT_Error* Buffer_Delete(PJRT_Buffer_Delete_Args* args) {
  return guarded("PJRT_Buffer_Delete", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_Delete_Args, buffer);
    args->buffer->buf->deleted = true;
    args->buffer->buf->mem.reset();  // device memory returns to the cache
  });
}

static PJRT_Error* Buffer_IsDeleted(PJRT_Buffer_IsDeleted_Args* args) {
  return guarded("PJRT_Buffer_IsDeleted", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_IsDeleted_Args, is_deleted);
    args->is_deleted = args->buffer->buf->deleted;
  });
}

static PJRT_Error* Buffer_ToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* args) {
  return guarded("PJRT_Buffer_ToHostBuffer", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_ToHostBuffer_Args, event);
    const Buffer& b = *args->src->buf;
    PJRTX_CHECK(!b.deleted, Code::kFailedPrecondition, "ToHostBuffer: buffer was deleted");
    if (!args->dst) {
      args->dst_size = b.type.bytes();
      return;
    }
    buffer_to_host(b, args->dst, args->dst_size);
    args->event = new PJRT_Event{Event::ready()};
  });
}

static PJRT_Error* Buffer_IsOnCpu(PJRT_Buffer_IsOnCpu_Args* args) {
  return guarded("PJRT_Buffer_IsOnCpu", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_IsOnCpu_Args, is_on_cpu);
    args->is_on_cpu = false;
  });
}

static PJRT_Error* Buffer_ReadyEvent(PJRT_Buffer_ReadyEvent_Args* args) {
  return guarded("PJRT_Buffer_ReadyEvent", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_ReadyEvent_Args, event);
    auto ev = args->buffer->buf->ready;
    args->event = new PJRT_Event{ev ? ev : Event::ready()};
  });
}

static PJRT_Error* Buffer_UnsafePointer(PJRT_Buffer_UnsafePointer_Args* args) {
  return guarded("PJRT_Buffer_UnsafePointer", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_UnsafePointer_Args, buffer_pointer);
    const auto& m = args->buffer->buf->mem;
    args->buffer_pointer = reinterpret_cast<uintptr_t>(m ? m->ptr : nullptr);
  });
}

static PJRT_Error* Buffer_OpaqueDeviceMemoryDataPointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* args) {
  return guarded("PJRT_Buffer_OpaqueDeviceMemoryDataPointer", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args, device_memory_ptr);
    const auto& m = args->buffer->buf->mem;
    args->device_memory_ptr = m ? m->ptr : nullptr;
  });
}

static PJRT_Error* Buffer_IncreaseExternalReferenceCount(PJRT_Buffer_IncreaseExternalReferenceCount_Args* args) {
  return guarded("PJRT_Buffer_IncreaseExternalReferenceCount", [&] { (void)args; });
}

static PJRT_Error* Buffer_DecreaseExternalReferenceCount(PJRT_Buffer_DecreaseExternalReferenceCount_Args* args) {
  return guarded("PJRT_Buffer_DecreaseExternalReferenceCount", [&] { (void)args; });
}

static PJRT_Error* Buffer_CopyToDevice(PJRT_Buffer_CopyToDevice_Args* args) {
  return guarded("PJRT_Buffer_CopyToDevice", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_CopyToDevice_Args, dst_buffer);
    const Buffer& src = *args->buffer->buf;
    if (src.ready) src.ready->wait_resolved();  // an async transfer still filling it
    PJRT_Device* d = args->dst_device;
    auto b = std::make_shared<Buffer>();
    b->dev = d->dev;
    b->type = src.type;
    b->mem = d->dev->allocate(src.type.bytes());
    if (src.type.bytes()) {
      d->dev->make_current();
      hip_check(hipMemcpyAsync(b->mem->ptr, src.mem->ptr, src.type.bytes(), hipMemcpyDefault, src.dev->stream()),
                "hipMemcpyAsync(D2D)");
      hip_check(hipStreamSynchronize(src.dev->stream()), "hipStreamSynchronize");
    }
    b->ready = Event::ready();
    auto* pb = new PJRT_Buffer();
    pb->buf = b;
    pb->client = args->buffer->client;
    pb->device = d;
    args->dst_buffer = pb;
  });
}

static PJRT_Error* Buffer_CopyToMemory(PJRT_Buffer_CopyToMemory_Args* args) {
  return guarded("PJRT_Buffer_CopyToMemory", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_Buffer_CopyToMemory_Args, dst_buffer);
    PJRT_Buffer_CopyToDevice_Args c{};
    c.struct_size = PJRT_Buffer_CopyToDevice_Args_STRUCT_SIZE;
    c.buffer = args->buffer;
    c.dst_device = args->dst_memory->device;
    PJRT_Error* e = Buffer_CopyToDevice(&c);
    if (e) {
      Error err(e->code, e->message);
      delete e;
      throw err;
    }
    args->dst_buffer = c.dst_buffer;
  });
}

// ----------------------------------------------------------------- topology

static PJRT_Error* TopologyDescription_Destroy(PJRT_TopologyDescription_Destroy_Args* args) {
  return guarded("PJRT_TopologyDescription_Destroy", [&] { (void)args; /* owned by the client */ });
}

static PJRT_Error* TopologyDescription_PlatformName(PJRT_TopologyDescription_PlatformName_Args* args) {
  return guarded("PJRT_TopologyDescription_PlatformName", [&] {
    args->platform_name = kPlatformName.c_str();
    args->platform_name_size = kPlatformName.size();
  });
}

static PJRT_Error* TopologyDescription_PlatformVersion(PJRT_TopologyDescription_PlatformVersion_Args* args) {
  return guarded("PJRT_TopologyDescription_PlatformVersion", [&] {
    const std::string& v = args->topology->client->platform_version;
    args->platform_version = v.c_str();
    args->platform_version_size = v.size();
  });
}

static PJRT_Error* TopologyDescription_GetDeviceDescriptions(PJRT_TopologyDescription_GetDeviceDescriptions_Args* args) {
  return guarded("PJRT_TopologyDescription_GetDeviceDescriptions", [&] {
    static thread_local std::vector<PJRT_DeviceDescription*> descs;
    descs.clear();
    for (PJRT_Device* d : args->topology->client->devices) descs.push_back(&d->desc);
    args->descriptions = descs.data();
    args->num_descriptions = descs.size();
  });
}

// "platform=<name>;version=<version>;devices=<n>" and one
// ";device=<id>:<local hardware id>:<process index>:<kind>" per device
// (reference: topology.zig:85-108, the same fields in the same order).
static void SerializedTopology_Delete(PJRT_SerializedTopology* t) { delete t; }

static PJRT_Error* TopologyDescription_Serialize(PJRT_TopologyDescription_Serialize_Args* args) {
  return guarded("PJRT_TopologyDescription_Serialize", [&] {
    PJRTX_ARGS_CHECK(args, PJRT_TopologyDescription_Serialize_Args, serialized_topology_deleter);
    PJRTX_CHECK(args->topology != nullptr && args->topology->client != nullptr, Code::kInvalidArgument,
                "PJRT_TopologyDescription_Serialize: topology is null");
    const PJRT_Client* client = args->topology->client;
    auto t = std::make_unique<PJRT_SerializedTopology>();
    std::string& s = t->bytes;
    s = "platform=" + kPlatformName + ";version=" + client->platform_version +
        ";devices=" + std::to_string(client->devices.size());
    for (const PJRT_Device* d : client->devices)
      s += ";device=" + std::to_string(d->desc.id) + ":" + std::to_string(d->desc.id) + ":0:" + d->desc.kind;
    args->serialized_bytes = s.data();
    args->serialized_bytes_size = s.size();
    args->serialized_topology = t.release();
    args->serialized_topology_deleter = SerializedTopology_Delete;
  });
}

static PJRT_Error* TopologyDescription_Attributes(PJRT_TopologyDescription_Attributes_Args* args) {
  return guarded("PJRT_TopologyDescription_Attributes", [&] {
    args->attributes = nullptr;
    args->num_attributes = 0;
  });
}

// ---------------------------------------------------- unimplemented families

template <typename A>
static PJRT_Error* Unimplemented(A*) {
  return make_error(Code::kUnimplemented, "pjrtx: this PJRT function is not implemented by the ROCm backend");
}

// ------------------------------------------------------ custom-call targets
// The PJRT GPU custom-call extension and the PjRTx_* registration exports
// (reference: src/plugin/custom_call.zig:35-185). A handler registered
// through the extension is recognised by its address: one of the three
// marker functions below; any other handler is UNIMPLEMENTED (this plugin
// runs no host or device code of the caller's).

extern "C" {
__attribute__((visibility("default"))) void PjRTx_CustomCall_Identity(void) {}
__attribute__((visibility("default"))) void PjRTx_CustomCall_UnarySqrt(void) {}
__attribute__((visibility("default"))) void PjRTx_CustomCall_BinaryAdd(void) {}
}

static std::string name_of(const char* p, size_t n, const char* what) {
  PJRTX_CHECK(p != nullptr, Code::kInvalidArgument, std::string("custom call ") + what + " is null");
  return std::string(p, n);
}

static PJRT_Error* Gpu_Register_Custom_Call(PJRT_Gpu_Register_Custom_Call_Args* args) {
  return guarded("PJRT_Gpu_Register_Custom_Call", [&] {
    PJRTX_CHECK(args != nullptr, Code::kInvalidArgument, "custom call registration args are null");
    PJRTX_CHECK(args->struct_size >= PJRT_Gpu_Register_Custom_Call_Args_STRUCT_SIZE, Code::kInvalidArgument,
                "custom call registration args struct is too small");
    const std::string target = name_of(args->function_name, args->function_name_size, "target");
    PJRTX_CHECK(args->api_version == 0, Code::kUnimplemented,
                "pjrtx custom calls support the PJRT GPU untyped API version 0 only");
    PJRTX_CHECK(args->handler_execute != nullptr, Code::kInvalidArgument, "custom call handler_execute is null");
    const void* h = args->handler_execute;
    if (h == reinterpret_cast<const void*>(&PjRTx_CustomCall_Identity)) {
      register_custom_call_identity(target);
    } else if (h == reinterpret_cast<const void*>(&PjRTx_CustomCall_UnarySqrt)) {
      register_custom_call_unary(target, "sqrt");
    } else if (h == reinterpret_cast<const void*>(&PjRTx_CustomCall_BinaryAdd)) {
      register_custom_call_binary(target, "add");
    } else {
      fail(Code::kUnimplemented, "custom call handler is not a pjrtx handler (PjRTx_CustomCall_*)");
    }
  });
}

static PJRT_Gpu_Custom_Call g_gpu_custom_call = {
    {PJRT_Gpu_Custom_Call_STRUCT_SIZE, PJRT_Extension_Type_Gpu_Custom_Call, nullptr}, Gpu_Register_Custom_Call};

extern "C" {
__attribute__((visibility("default"))) PJRT_Error* PjRTx_RegisterCustomCallIdentity(const char* function_name,
                                                                                   size_t function_name_size) {
  return guarded("PjRTx_RegisterCustomCallIdentity",
                 [&] { register_custom_call_identity(name_of(function_name, function_name_size, "target")); });
}

__attribute__((visibility("default"))) PJRT_Error* PjRTx_RegisterCustomCallUnary(const char* function_name,
                                                                                size_t function_name_size,
                                                                                const char* op_name,
                                                                                size_t op_name_size) {
  return guarded("PjRTx_RegisterCustomCallUnary", [&] {
    register_custom_call_unary(name_of(function_name, function_name_size, "target"),
                               name_of(op_name, op_name_size, "op name"));
  });
}

__attribute__((visibility("default"))) PJRT_Error* PjRTx_RegisterCustomCallBinary(const char* function_name,
                                                                                 size_t function_name_size,
                                                                                 const char* op_name,
                                                                                 size_t op_name_size) {
  return guarded("PjRTx_RegisterCustomCallBinary", [&] {
    register_custom_call_binary(name_of(function_name, function_name_size, "target"),
                                name_of(op_name, op_name_size, "op name"));
  });
}

__attribute__((visibility("default"))) void PjRTx_UnregisterCustomCall(const char* function_name,
                                                                      size_t function_name_size) {
  if (function_name != nullptr) unregister_custom_call(std::string(function_name, function_name_size));
}
}

// ----------------------------------------------------------------- the table

extern "C" __attribute__((visibility("default"))) const PJRT_Api* GetPjrtApi(void) {
  static PJRT_Api api = [] {
    PJRT_Api a;
    std::memset(&a, 0, sizeof(a));
    a.struct_size = PJRT_Api_STRUCT_SIZE;
    a.extension_start = &g_gpu_custom_call.base;
    a.pjrt_api_version.struct_size = PJRT_Api_Version_STRUCT_SIZE;
    a.pjrt_api_version.extension_start = nullptr;
    a.pjrt_api_version.major_version = PJRT_API_MAJOR;
    a.pjrt_api_version.minor_version = PJRT_API_MINOR;

    a.PJRT_Error_Destroy = Error_Destroy;
    a.PJRT_Error_Message = Error_Message;
    a.PJRT_Error_GetCode = Error_GetCode;
    a.PJRT_Plugin_Initialize = Plugin_Initialize;
    a.PJRT_Plugin_Attributes = Plugin_Attributes;
    a.PJRT_Event_Destroy = Event_Destroy;
    a.PJRT_Event_IsReady = Event_IsReady;
    a.PJRT_Event_Error = Event_Error;
    a.PJRT_Event_Await = Event_Await;
    a.PJRT_Event_OnReady = Event_OnReady;
    a.PJRT_Client_Create = Client_Create;
    a.PJRT_Client_Destroy = Client_Destroy;
    a.PJRT_Client_PlatformName = Client_PlatformName;
    a.PJRT_Client_ProcessIndex = Client_ProcessIndex;
    a.PJRT_Client_PlatformVersion = Client_PlatformVersion;
    a.PJRT_Client_Devices = Client_Devices;
    a.PJRT_Client_AddressableDevices = Client_AddressableDevices;
    a.PJRT_Client_LookupDevice = Client_LookupDevice;
    a.PJRT_Client_LookupAddressableDevice = Client_LookupAddressableDevice;
    a.PJRT_Client_AddressableMemories = Client_AddressableMemories;
    a.PJRT_Client_Compile = Client_Compile;
    a.PJRT_Client_DefaultDeviceAssignment = Client_DefaultDeviceAssignment;
    a.PJRT_Client_BufferFromHostBuffer = Client_BufferFromHostBuffer;
    a.PJRT_DeviceDescription_Id = DeviceDescription_Id;
    a.PJRT_DeviceDescription_ProcessIndex = DeviceDescription_ProcessIndex;
    a.PJRT_DeviceDescription_Attributes = DeviceDescription_Attributes;
    a.PJRT_DeviceDescription_Kind = DeviceDescription_Kind;
    a.PJRT_DeviceDescription_DebugString = DeviceDescription_DebugString;
    a.PJRT_DeviceDescription_ToString = DeviceDescription_ToString;
    a.PJRT_Device_GetDescription = Device_GetDescription;
    a.PJRT_Device_IsAddressable = Device_IsAddressable;
    a.PJRT_Device_LocalHardwareId = Device_LocalHardwareId;
    a.PJRT_Device_AddressableMemories = Device_AddressableMemories;
    a.PJRT_Device_DefaultMemory = Device_DefaultMemory;
    a.PJRT_Device_MemoryStats = Device_MemoryStats;
    a.PJRT_Memory_Id = Memory_Id;
    a.PJRT_Memory_Kind = Memory_Kind;
    a.PJRT_Memory_DebugString = Memory_DebugString;
    a.PJRT_Memory_ToString = Memory_ToString;
    a.PJRT_Memory_AddressableByDevices = Memory_AddressableByDevices;
    a.PJRT_Executable_Destroy = Executable_Destroy;
    a.PJRT_Executable_Name = Executable_Name;
    a.PJRT_Executable_NumReplicas = Executable_NumReplicas;
    a.PJRT_Executable_NumPartitions = Executable_NumPartitions;
    a.PJRT_Executable_NumOutputs = Executable_NumOutputs;
    a.PJRT_Executable_SizeOfGeneratedCodeInBytes = Executable_SizeOfGeneratedCodeInBytes;
    a.PJRT_Executable_GetCostAnalysis = Executable_GetCostAnalysis;
    a.PJRT_Executable_OutputMemoryKinds = Executable_OutputMemoryKinds;
    a.PJRT_Executable_OptimizedProgram = Executable_OptimizedProgram;
    a.PJRT_Executable_Serialize = Unimplemented<PJRT_Executable_Serialize_Args>;
    a.PJRT_LoadedExecutable_Destroy = LoadedExecutable_Destroy;
    a.PJRT_LoadedExecutable_GetExecutable = LoadedExecutable_GetExecutable;
    a.PJRT_LoadedExecutable_AddressableDevices = LoadedExecutable_AddressableDevices;
    a.PJRT_LoadedExecutable_Delete = LoadedExecutable_Delete;
    a.PJRT_LoadedExecutable_IsDeleted = LoadedExecutable_IsDeleted;
    a.PJRT_LoadedExecutable_Execute = LoadedExecutable_Execute;
    a.PJRT_Executable_DeserializeAndLoad = Unimplemented<PJRT_Executable_DeserializeAndLoad_Args>;
    a.PJRT_LoadedExecutable_Fingerprint = LoadedExecutable_Fingerprint;
    a.PJRT_Buffer_Destroy = Buffer_Destroy;
    a.PJRT_Buffer_ElementType = Buffer_ElementType;
    a.PJRT_Buffer_Dimensions = Buffer_Dimensions;
    a.PJRT_Buffer_UnpaddedDimensions = Buffer_UnpaddedDimensions;
    a.PJRT_Buffer_DynamicDimensionIndices = Buffer_DynamicDimensionIndices;
    a.PJRT_Buffer_GetMemoryLayout = Unimplemented<PJRT_Buffer_GetMemoryLayout_Args>;
    a.PJRT_Buffer_OnDeviceSizeInBytes = Buffer_OnDeviceSizeInBytes;
    a.PJRT_Buffer_Device = Buffer_Device;
    a.PJRT_Buffer_Memory = Buffer_Memory;
    a.PJRT_Buffer_Delete = Buffer_Delete;
    a.PJRT_Buffer_IsDeleted = Buffer_IsDeleted;
    a.PJRT_Buffer_CopyToDevice = Buffer_CopyToDevice;
    a.PJRT_Buffer_ToHostBuffer = Buffer_ToHostBuffer;
    a.PJRT_Buffer_IsOnCpu = Buffer_IsOnCpu;
    a.PJRT_Buffer_ReadyEvent = Buffer_ReadyEvent;
    a.PJRT_Buffer_UnsafePointer = Buffer_UnsafePointer;
    a.PJRT_Buffer_IncreaseExternalReferenceCount = Buffer_IncreaseExternalReferenceCount;
    a.PJRT_Buffer_DecreaseExternalReferenceCount = Buffer_DecreaseExternalReferenceCount;
    a.PJRT_Buffer_OpaqueDeviceMemoryDataPointer = Buffer_OpaqueDeviceMemoryDataPointer;
    a.PJRT_CopyToDeviceStream_Destroy = Unimplemented<PJRT_CopyToDeviceStream_Destroy_Args>;
    a.PJRT_CopyToDeviceStream_AddChunk = Unimplemented<PJRT_CopyToDeviceStream_AddChunk_Args>;
    a.PJRT_CopyToDeviceStream_TotalBytes = Unimplemented<PJRT_CopyToDeviceStream_TotalBytes_Args>;
    a.PJRT_CopyToDeviceStream_GranuleSize = Unimplemented<PJRT_CopyToDeviceStream_GranuleSize_Args>;
    a.PJRT_CopyToDeviceStream_CurrentBytes = Unimplemented<PJRT_CopyToDeviceStream_CurrentBytes_Args>;
    a.PJRT_TopologyDescription_Create = Unimplemented<PJRT_TopologyDescription_Create_Args>;
    a.PJRT_TopologyDescription_Destroy = TopologyDescription_Destroy;
    a.PJRT_TopologyDescription_PlatformName = TopologyDescription_PlatformName;
    a.PJRT_TopologyDescription_PlatformVersion = TopologyDescription_PlatformVersion;
    a.PJRT_TopologyDescription_GetDeviceDescriptions = TopologyDescription_GetDeviceDescriptions;
    a.PJRT_TopologyDescription_Serialize = TopologyDescription_Serialize;
    a.PJRT_TopologyDescription_Attributes = TopologyDescription_Attributes;
    a.PJRT_Compile = Unimplemented<PJRT_Compile_Args>;
    a.PJRT_Executable_OutputElementTypes = Executable_OutputElementTypes;
    a.PJRT_Executable_OutputDimensions = Executable_OutputDimensions;
    a.PJRT_Buffer_CopyToMemory = Buffer_CopyToMemory;
    a.PJRT_Client_CreateViewOfDeviceBuffer = Unimplemented<PJRT_Client_CreateViewOfDeviceBuffer_Args>;
    a.PJRT_Executable_Fingerprint = Executable_Fingerprint;
    a.PJRT_Client_TopologyDescription = Client_TopologyDescription;
    a.PJRT_Executable_GetCompiledMemoryStats = Unimplemented<PJRT_Executable_GetCompiledMemoryStats_Args>;
    a.PJRT_Memory_Kind_Id = Memory_Kind_Id;
    a.PJRT_ExecuteContext_Create = Unimplemented<PJRT_ExecuteContext_Create_Args>;
    a.PJRT_ExecuteContext_Destroy = Unimplemented<PJRT_ExecuteContext_Destroy_Args>;
    a.PJRT_Buffer_CopyRawToHost = Unimplemented<PJRT_Buffer_CopyRawToHost_Args>;
    a.PJRT_AsyncHostToDeviceTransferManager_Destroy = Transfer_Destroy;
    a.PJRT_AsyncHostToDeviceTransferManager_TransferData = Transfer_TransferData;
    a.PJRT_Client_CreateBuffersForAsyncHostToDevice = Client_CreateBuffersForAsyncHostToDevice;
    a.PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer = Transfer_RetrieveBuffer;
    a.PJRT_AsyncHostToDeviceTransferManager_Device = Transfer_Device;
    a.PJRT_AsyncHostToDeviceTransferManager_BufferCount = Transfer_BufferCount;
    a.PJRT_AsyncHostToDeviceTransferManager_BufferSize = Transfer_BufferSize;
    a.PJRT_AsyncHostToDeviceTransferManager_SetBufferError = Transfer_SetBufferError;
    a.PJRT_AsyncHostToDeviceTransferManager_AddMetadata = Transfer_AddMetadata;
    a.PJRT_Client_DmaMap = Unimplemented<PJRT_Client_DmaMap_Args>;
    a.PJRT_Client_DmaUnmap = Unimplemented<PJRT_Client_DmaUnmap_Args>;
    return a;
  }();
  return &api;
}
