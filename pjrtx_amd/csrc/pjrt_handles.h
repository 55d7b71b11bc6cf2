// Definitions of the opaque PJRT handle types (PJRT_Client, PJRT_Buffer,
// ...) shared by the PJRT adapter and the pjrtx_hip C ABI.
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "../../include/pjrt_c_api.h"
#include "runtime.h"

struct PJRT_Error {
  pjrtx::Code code;
  std::string message;
};

struct PJRT_Event {
  std::shared_ptr<pjrtx::Event> ev;
};

struct PJRT_Memory;

struct PJRT_DeviceDescription {
  int id = 0;
  std::string kind, debug, to_string;
  std::vector<PJRT_NamedValue> attrs;
  std::vector<std::string> attr_strings;
  int64_t ordinal_attr = 0;
};

struct PJRT_Device {
  pjrtx::Device* dev = nullptr;
  PJRT_DeviceDescription desc;
  PJRT_Memory* memory = nullptr;
  PJRT_Client* client = nullptr;
};

struct PJRT_Memory {
  int id = 0;
  std::string kind = "device";
  std::string debug, to_string;
  PJRT_Device* device = nullptr;
};

struct PJRT_TopologyDescription {
  PJRT_Client* client = nullptr;
};

// PJRT_TopologyDescription_Serialize's result, freed by its deleter.
struct PJRT_SerializedTopology {
  std::string bytes;
};

struct PJRT_Client {
  std::vector<std::unique_ptr<PJRT_Device>> device_storage;
  std::vector<std::unique_ptr<PJRT_Memory>> memory_storage;
  std::vector<PJRT_Device*> devices;
  std::vector<PJRT_Memory*> memories;
  PJRT_TopologyDescription topology;
  std::string platform_version;
};

struct PJRT_Buffer {
  pjrtx::BufferRef buf;
  PJRT_Client* client = nullptr;
  PJRT_Device* device = nullptr;
};

struct PJRT_Executable {
  std::shared_ptr<pjrtx::Executable> exe;
  std::vector<PJRT_Buffer_Type> out_types;
  std::vector<int64_t> out_dims;
  std::vector<size_t> out_ranks;
  std::vector<const char*> out_kinds;
  std::vector<size_t> out_kind_sizes;
  std::string optimized_text;
};

struct PJRT_LoadedExecutable {
  std::shared_ptr<pjrtx::Executable> exe;
  PJRT_Client* client = nullptr;
  std::vector<PJRT_Device*> devices;
  bool deleted = false;
};

struct PJRT_AsyncHostToDeviceTransferManager {
  std::unique_ptr<pjrtx::AsyncTransfer> t;
  PJRT_Client* client = nullptr;
  PJRT_Device* device = nullptr;
};
