// Shared value types of the pjrtx_amd plugin: element types, shapes and a
// status type that carries a PJRT error code.
//
// Dense row-major layout only, as the reference planner assumes
// (reference: src/compiler/tensor.zig:4-52, row-major at :36-39).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace pjrtx {

// Element types. Values equal PJRT_Buffer_Type so conversion is a cast.
enum class DType : int {
  kInvalid = 0,
  kPred = 1,
  kS8 = 2,
  kS16 = 3,
  kS32 = 4,
  kS64 = 5,
  kU8 = 6,
  kU16 = 7,
  kU32 = 8,
  kU64 = 9,
  kF16 = 10,
  kF32 = 11,
  kF64 = 12,
  kBF16 = 13,
};

size_t dtype_size(DType t);
bool dtype_is_float(DType t);
bool dtype_is_signed_int(DType t);
bool dtype_is_unsigned_int(DType t);  // includes pred
const char* dtype_name(DType t);      // "f32", "bf16", "i32", "ui32", "i1" ...
DType dtype_from_mlir(const std::string& s);  // "f32" "bf16" "i32" "ui8" "i1"

// C type used for a value of this dtype inside generated kernels.
// Floating types narrower than f32 compute in float and round after each op.
const char* dtype_compute_ctype(DType t);
// C type used for a stored element in memory.
const char* dtype_storage_ctype(DType t);

using Dims = std::vector<int64_t>;

int64_t num_elements(const Dims& d);
std::string dims_str(const Dims& d);

struct TensorType {
  DType dtype = DType::kInvalid;
  Dims dims;
  int64_t elements() const { return num_elements(dims); }
  size_t bytes() const { return static_cast<size_t>(elements()) * dtype_size(dtype); }
  int rank() const { return static_cast<int>(dims.size()); }
  bool operator==(const TensorType& o) const { return dtype == o.dtype && dims == o.dims; }
  bool operator!=(const TensorType& o) const { return !(*this == o); }
  std::string str() const;  // tensor<4x8xf32>
};

// Error codes follow PJRT_Error_Code numbering.
enum class Code : int {
  kOk = 0,
  kCancelled = 1,
  kInvalidArgument = 3,
  kNotFound = 5,
  kResourceExhausted = 8,
  kFailedPrecondition = 9,
  kUnimplemented = 12,
  kInternal = 13,
};

// Exception type used inside the plugin; converted to PJRT_Error at the
// C-API boundary so no exception crosses `extern "C"`.
struct Error : std::runtime_error {
  Code code;
  Error(Code c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

[[noreturn]] void fail(Code c, const std::string& msg);
#define PJRTX_CHECK(cond, code, msg)                 \
  do {                                               \
    if (!(cond)) ::pjrtx::fail((code), (msg));       \
  } while (0)

std::string strformat(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Environment switches, parsed the way the reference parses its PJRTX_* vars
// (reference: src/backend/mlx_metal/profiling_env.zig:79-83).
bool env_flag(const char* name);
int64_t env_int(const char* name, int64_t dflt);

}  // namespace pjrtx
