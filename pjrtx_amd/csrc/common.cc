#include "common.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace pjrtx {

size_t dtype_size(DType t) {
  switch (t) {
    case DType::kPred:
    case DType::kS8:
    case DType::kU8:
      return 1;
    case DType::kS16:
    case DType::kU16:
    case DType::kF16:
    case DType::kBF16:
      return 2;
    case DType::kS32:
    case DType::kU32:
    case DType::kF32:
      return 4;
    case DType::kS64:
    case DType::kU64:
    case DType::kF64:
      return 8;
    default:
      return 0;
  }
}

bool dtype_is_float(DType t) {
  return t == DType::kF16 || t == DType::kBF16 || t == DType::kF32 || t == DType::kF64;
}
bool dtype_is_signed_int(DType t) {
  return t == DType::kS8 || t == DType::kS16 || t == DType::kS32 || t == DType::kS64;
}
bool dtype_is_unsigned_int(DType t) {
  return t == DType::kPred || t == DType::kU8 || t == DType::kU16 || t == DType::kU32 ||
         t == DType::kU64;
}

const char* dtype_name(DType t) {
  switch (t) {
    case DType::kPred: return "i1";
    case DType::kS8: return "i8";
    case DType::kS16: return "i16";
    case DType::kS32: return "i32";
    case DType::kS64: return "i64";
    case DType::kU8: return "ui8";
    case DType::kU16: return "ui16";
    case DType::kU32: return "ui32";
    case DType::kU64: return "ui64";
    case DType::kF16: return "f16";
    case DType::kF32: return "f32";
    case DType::kF64: return "f64";
    case DType::kBF16: return "bf16";
    default: return "invalid";
  }
}

DType dtype_from_mlir(const std::string& s) {
  if (s == "f32") return DType::kF32;
  if (s == "bf16") return DType::kBF16;
  if (s == "f16") return DType::kF16;
  if (s == "f64") return DType::kF64;
  if (s == "i1") return DType::kPred;
  if (s == "i8") return DType::kS8;
  if (s == "i16") return DType::kS16;
  if (s == "i32") return DType::kS32;
  if (s == "i64") return DType::kS64;
  if (s == "ui8") return DType::kU8;
  if (s == "ui16") return DType::kU16;
  if (s == "ui32") return DType::kU32;
  if (s == "ui64") return DType::kU64;
  return DType::kInvalid;
}

const char* dtype_compute_ctype(DType t) {
  switch (t) {
    case DType::kPred: return "bool";
    case DType::kS8: return "int8_t";
    case DType::kS16: return "int16_t";
    case DType::kS32: return "int32_t";
    case DType::kS64: return "int64_t";
    case DType::kU8: return "uint8_t";
    case DType::kU16: return "uint16_t";
    case DType::kU32: return "uint32_t";
    case DType::kU64: return "uint64_t";
    case DType::kF16:
    case DType::kBF16:
    case DType::kF32: return "float";
    case DType::kF64: return "double";
    default: return "void";
  }
}

const char* dtype_storage_ctype(DType t) {
  switch (t) {
    case DType::kPred: return "uint8_t";
    case DType::kF16: return "uint16_t";
    case DType::kBF16: return "uint16_t";
    default: return dtype_compute_ctype(t);
  }
}

int64_t num_elements(const Dims& d) {
  int64_t n = 1;
  for (int64_t x : d) n *= x;
  return n;
}

std::string dims_str(const Dims& d) {
  std::string s = "[";
  for (size_t i = 0; i < d.size(); ++i) {
    if (i) s += ",";
    s += std::to_string(d[i]);
  }
  return s + "]";
}

std::string TensorType::str() const {
  std::string s = "tensor<";
  for (int64_t x : dims) s += std::to_string(x) + "x";
  return s + dtype_name(dtype) + ">";
}

void fail(Code c, const std::string& msg) { throw Error(c, msg); }

std::string strformat(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  char buf[1024];
  int n = vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  if (n < static_cast<int>(sizeof(buf))) return std::string(buf, n < 0 ? 0 : n);
  std::string out(n + 1, '\0');
  va_start(ap, fmt);
  vsnprintf(out.data(), out.size(), fmt, ap);
  va_end(ap);
  out.resize(n);
  return out;
}

bool env_flag(const char* name) {
  const char* v = std::getenv(name);
  if (!v || !*v) return false;
  return !(std::strcmp(v, "0") == 0 || std::strcmp(v, "false") == 0);
}

int64_t env_int(const char* name, int64_t dflt) {
  const char* v = std::getenv(name);
  if (!v || !*v) return dflt;
  char* end = nullptr;
  long long x = std::strtoll(v, &end, 10);
  return (end && *end == '\0') ? x : dflt;
}

}  // namespace pjrtx
