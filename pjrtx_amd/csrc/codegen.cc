// Kernel source generation for fusion groups.
//
// Each loop / reduce step becomes one `extern "C" __global__` function built
// from the hand-written skeletons below plus the group's expression DAG,
// evaluated per element at an index that view ops (broadcast_in_dim,
// reshape, transpose, slice, reverse, iota) remap arithmetically instead of
// materializing. Counterpart of the reference's MSL fusion writer
// (reference: executable_metal_graph_fusion_request_record.zig:11-211,
// executable_metal_graph_fusion_expression.zig:56-152 broadcast/slice index
// maps, executable_metal_graph_fusion_request_writer.zig:7-55).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <set>
#include <sstream>

#include "planner.h"

namespace pjrtx {
namespace {

std::string hex_u32(uint32_t v) { return strformat("0x%08xu", v); }

// C literal for the element `i` of a constant op, in compute type.
std::string literal_expr(const Program& prog, const Op& op, size_t i) {
  const TensorType& t = prog.type(op.results[0]);
  const size_t esz = dtype_size(t.dtype);
  const size_t idx = op.splat ? 0 : i;
  const uint8_t* p = op.literal.data() + idx * esz;
  switch (t.dtype) {
    case DType::kF32: {
      uint32_t u;
      std::memcpy(&u, p, 4);
      return "__builtin_bit_cast(float, " + hex_u32(u) + ")";
    }
    case DType::kBF16: {
      uint16_t b;
      std::memcpy(&b, p, 2);
      return "__builtin_bit_cast(float, " + hex_u32(static_cast<uint32_t>(b) << 16) + ")";
    }
    case DType::kF16: {
      uint16_t h;
      std::memcpy(&h, p, 2);
      float f = f16_bits_to_f32(h);
      uint32_t u;
      std::memcpy(&u, &f, 4);
      return "__builtin_bit_cast(float, " + hex_u32(u) + ")";
    }
    case DType::kF64: {
      uint64_t u;
      std::memcpy(&u, p, 8);
      return strformat("__builtin_bit_cast(double, 0x%016llxull)", static_cast<unsigned long long>(u));
    }
    case DType::kPred: return p[0] ? "true" : "false";
    case DType::kS8: return strformat("((int8_t)%d)", static_cast<int>(*reinterpret_cast<const int8_t*>(p)));
    case DType::kU8: return strformat("((uint8_t)%u)", static_cast<unsigned>(p[0]));
    case DType::kS16: { int16_t v; std::memcpy(&v, p, 2); return strformat("((int16_t)%d)", v); }
    case DType::kU16: { uint16_t v; std::memcpy(&v, p, 2); return strformat("((uint16_t)%u)", v); }
    case DType::kS32: { int32_t v; std::memcpy(&v, p, 4); return strformat("((int32_t)%d)", v); }
    case DType::kU32: { uint32_t v; std::memcpy(&v, p, 4); return strformat("((uint32_t)%uu)", v); }
    case DType::kS64: { int64_t v; std::memcpy(&v, p, 8); return strformat("((int64_t)%lldll)", static_cast<long long>(v)); }
    case DType::kU64: { uint64_t v; std::memcpy(&v, p, 8); return strformat("((uint64_t)%lluull)", static_cast<unsigned long long>(v)); }
    default: fail(Code::kUnimplemented, "literal of unsupported type");
  }
}

std::string load_expr(DType t, const std::string& ptr, const std::string& idx) {
  switch (t) {
    case DType::kBF16: return "bf16_to_f32(" + ptr + "[" + idx + "])";
    case DType::kF16: return "f16_to_f32(" + ptr + "[" + idx + "])";
    case DType::kPred: return "(" + ptr + "[" + idx + "] != 0)";
    default: return ptr + "[" + idx + "]";
  }
}

std::string from_storage(DType t, const std::string& s) {
  switch (t) {
    case DType::kBF16: return "bf16_to_f32(" + s + ")";
    case DType::kF16: return "f16_to_f32(" + s + ")";
    case DType::kPred: return "(" + s + " != 0)";
    default: return s;
  }
}

std::string to_storage(DType t, const std::string& c) {
  switch (t) {
    case DType::kBF16: return "f32_to_bf16(" + c + ")";
    case DType::kF16: return "f32_to_f16(" + c + ")";
    case DType::kPred: return "(uint8_t)(" + c + ")";
    default: return c;
  }
}

// Rounds a float computation to the narrow float type of its result.
std::string round_to(DType t, const std::string& e) {
  if (t == DType::kBF16) return "round_bf16(" + e + ")";
  if (t == DType::kF16) return "round_f16(" + e + ")";
  return e;
}

const char* unsigned_of(DType t) {
  switch (t) {
    case DType::kS8: case DType::kU8: return "uint8_t";
    case DType::kS16: case DType::kU16: return "uint16_t";
    case DType::kS32: case DType::kU32: return "uint32_t";
    default: return "uint64_t";
  }
}

// An index into a value of a given shape: a linear expression, per-dim
// expressions, or both. `identity` marks the kernel's own root position,
// where vector-preloaded inputs can be used.
struct Idx {
  std::string key;
  Dims shape;
  std::string lin;
  std::vector<std::string> multi;
  bool identity = false;
};

class Writer {
 public:
  Writer(const Program& prog, const std::map<int, std::string>& ptr_of, const std::string& idx_t)
      : prog_(prog), ptr_of_(ptr_of), idx_t_(idx_t) {}

  std::ostringstream body;              // per-element statements
  std::map<int, std::string> preload;   // value -> preload array name (root identity)
  // Values that are per-row scalars of a row-fused kernel: any index into
  // them is the current row (the planner checks this), so they read as the
  // named variable.
  std::map<int, std::string> row_scalar;
  // Values held in LDS by the enclosing kernel (a GEMV's results in its
  // epilogue): the function maps a linear index into the value to the
  // expression that reads it.
  std::map<int, std::function<std::string(const std::string&)>> lds_value;

  int add_index(Idx idx) {
    idxs_.push_back(std::move(idx));
    return static_cast<int>(idxs_.size()) - 1;
  }
  void seed(int v, int idx, const std::string& var) { memo_[memo_key(v, idx)] = var; }

  std::string lin_of(int id) {
    Idx& I = idxs_[id];
    if (!I.lin.empty()) return I.lin;
    if (I.shape.empty()) return I.lin = "0";
    std::string e;
    int64_t stride = 1;
    for (int d = static_cast<int>(I.shape.size()) - 1; d >= 0; --d) {
      if (I.shape[d] != 1) {
        std::string term = stride == 1 ? "(" + I.multi[d] + ")" : "(" + I.multi[d] + ")*" + std::to_string(stride) + "u";
        e = e.empty() ? term : term + " + " + e;
      }
      stride *= I.shape[d];
    }
    if (e.empty()) e = "0";
    std::string var = tmp();
    body << "const " << idx_t_ << " " << var << " = " << e << ";\n";
    return idxs_[id].lin = var;
  }

  const std::vector<std::string>& multi_of(int id) {
    Idx& I = idxs_[id];
    if (!I.multi.empty() || I.shape.empty()) return I.multi;
    const std::string lin = lin_of(id);
    std::vector<std::string> m(I.shape.size());
    std::string rest = lin;
    for (int d = static_cast<int>(I.shape.size()) - 1; d >= 0; --d) {
      const int64_t D = I.shape[d];
      if (D == 1) {
        m[d] = "0";
        continue;
      }
      if (d == 0) {
        m[d] = rest;
        break;
      }
      std::string dv = tmp(), q = tmp();
      body << "const " << idx_t_ << " " << dv << " = " << rest << " % " << D << "u;\n";
      body << "const " << idx_t_ << " " << q << " = " << rest << " / " << D << "u;\n";
      m[d] = dv;
      rest = q;
    }
    idxs_[id].multi = m;
    return idxs_[id].multi;
  }

  // Returns an expression (usually a variable) holding value v at index `id`.
  std::string value(int v, int id);

 private:
  const Program& prog_;
  const std::map<int, std::string>& ptr_of_;
  std::string idx_t_;
  std::vector<Idx> idxs_;
  std::map<std::string, std::string> memo_;
  int tmp_ = 0;

  std::string tmp() { return "t" + std::to_string(tmp_++); }
  std::string memo_key(int v, int id) { return std::to_string(v) + "@" + idxs_[id].key; }
  std::string define(DType t, const std::string& e) {
    std::string var = tmp();
    body << "const " << dtype_compute_ctype(t) << " " << var << " = " << e << ";\n";
    return var;
  }
  int scalar_index() {
    Idx s;
    s.key = "S";
    s.lin = "0";
    return add_index(s);
  }
  std::string emit_op(const Op& op, int v, int id);
};

std::string Writer::value(int v, int id) {
  auto rsv = row_scalar.find(v);
  if (rsv != row_scalar.end()) return rsv->second;
  const std::string key = memo_key(v, id);
  auto m = memo_.find(key);
  if (m != memo_.end()) return m->second;
  std::string out;
  auto lv = lds_value.find(v);
  if (lv != lds_value.end()) {
    out = define(prog_.type(v).dtype, lv->second(lin_of(id)));
    memo_[key] = out;
    return out;
  }
  auto p = ptr_of_.find(v);
  const DType t = prog_.type(v).dtype;
  if (p != ptr_of_.end()) {
    auto pre = preload.find(v);
    if (idxs_[id].identity && pre != preload.end()) {
      out = define(t, from_storage(t, pre->second + "[j]"));
    } else {
      out = define(t, load_expr(t, p->second, lin_of(id)));
    }
  } else {
    // Find the producing op.
    int oi = -1;
    for (size_t i = 0; i < prog_.ops.size() && oi < 0; ++i)
      for (int r : prog_.ops[i].results)
        if (r == v) oi = static_cast<int>(i);
    PJRTX_CHECK(oi >= 0, Code::kInternal, "fusion value without producer or input");
    out = emit_op(prog_.ops[oi], v, id);
  }
  memo_[key] = out;
  return out;
}

std::string Writer::emit_op(const Op& op, int v, int id) {
  const TensorType& rt = prog_.type(v);
  const DType R = rt.dtype;
  auto operand_at_same = [&](int k) {
    const int u = op.operands[k];
    // Rank-0 operands of elementwise ops (select predicate, clamp bounds).
    if (prog_.type(u).rank() == 0 && rt.rank() > 0) return value(u, scalar_index());
    return value(u, id);
  };
  switch (op.kind) {
    case OpKind::kConstant: {
      if (op.splat || rt.elements() == 1) return literal_expr(prog_, op, 0);
      fail(Code::kInternal, "non-splat constant inside a fusion");
    }
    case OpKind::kIota: {
      const auto& m = multi_of(id);
      const std::string e = rt.rank() == 0 ? "0" : m[op.dim];
      if (dtype_is_float(R)) return define(R, round_to(R, "(float)(" + e + ")"));
      return define(R, std::string("(") + dtype_compute_ctype(R) + ")(" + e + ")");
    }
    case OpKind::kReshape: {
      Idx I;
      I.key = idxs_[id].key + "|r" + dims_str(prog_.type(op.operands[0]).dims);
      I.shape = prog_.type(op.operands[0]).dims;
      I.lin = lin_of(id);
      I.identity = idxs_[id].identity;
      return value(op.operands[0], add_index(I));
    }
    case OpKind::kBroadcastInDim: {
      const Dims& od = prog_.type(op.operands[0]).dims;
      Idx I;
      I.key = "b" + std::to_string(v) + "(" + idxs_[id].key + ")";
      I.shape = od;
      if (od.empty()) {
        I.lin = "0";
      } else {
        const auto& m = multi_of(id);
        for (size_t k = 0; k < od.size(); ++k)
          I.multi.push_back((od[k] == 1 && rt.dims[op.dims[k]] != 1) ? std::string("0") : m[op.dims[k]]);
      }
      return value(op.operands[0], add_index(I));
    }
    case OpKind::kTranspose: {
      const Dims& od = prog_.type(op.operands[0]).dims;
      const auto& m = multi_of(id);
      Idx I;
      I.key = "t" + std::to_string(v) + "(" + idxs_[id].key + ")";
      I.shape = od;
      I.multi.resize(od.size());
      for (size_t k = 0; k < op.dims.size(); ++k) I.multi[op.dims[k]] = m[k];
      return value(op.operands[0], add_index(I));
    }
    case OpKind::kSlice: {
      const Dims& od = prog_.type(op.operands[0]).dims;
      const auto& m = multi_of(id);
      Idx I;
      I.key = "s" + std::to_string(v) + "(" + idxs_[id].key + ")";
      I.shape = od;
      for (size_t k = 0; k < od.size(); ++k) {
        std::string e = m[k];
        const int64_t st = op.strides.empty() ? 1 : op.strides[k];
        if (st != 1) e = "(" + e + ")*" + std::to_string(st) + "u";
        if (op.start[k] != 0) e = "(" + e + " + " + std::to_string(op.start[k]) + "u)";
        I.multi.push_back(e);
      }
      return value(op.operands[0], add_index(I));
    }
    case OpKind::kReverse: {
      const Dims& od = prog_.type(op.operands[0]).dims;
      const auto& m = multi_of(id);
      Idx I;
      I.key = "v" + std::to_string(v) + "(" + idxs_[id].key + ")";
      I.shape = od;
      I.multi = m;
      for (int64_t d : op.dims) I.multi[d] = "(" + std::to_string(od[d] - 1) + "u - " + m[d] + ")";
      return value(op.operands[0], add_index(I));
    }
    case OpKind::kConcatenate: {
      // Each operand is read at the coordinate clamped into its own extent
      // (always in bounds); the result is chosen by the range the output
      // coordinate falls in. `m` is copied: add_index below may reallocate.
      const std::vector<std::string> m = multi_of(id);
      const int64_t cd = op.dim;
      const std::string c = m[cd];
      // Copies of one value (RoPE's [cos, cos] table): the coordinate is
      // wrapped into the operand and the operand evaluated once, instead of
      // once per copy and a select.
      bool copies = op.operands.size() > 1 && prog_.type(op.operands[0]).dims[cd] > 0;
      for (int o : op.operands) copies &= o == op.operands[0];
      if (copies) {
        const int64_t sz = prog_.type(op.operands[0]).dims[cd];
        const int64_t n = static_cast<int64_t>(op.operands.size());
        std::string e = "(" + c + " - " + std::to_string((n - 1) * sz) + "u)";
        for (int64_t k = n - 2; k >= 0; --k)
          e = "(" + c + " < " + std::to_string((k + 1) * sz) + "u ? " + c + " - " + std::to_string(k * sz) + "u : " + e + ")";
        Idx I;
        I.key = "cc" + std::to_string(v) + "(" + idxs_[id].key + ")";
        I.shape = prog_.type(op.operands[0]).dims;
        I.multi = m;
        I.multi[cd] = e;
        return define(R, value(op.operands[0], add_index(I)));
      }
      std::vector<std::string> vals;
      std::vector<int64_t> ends;
      int64_t off = 0;
      for (size_t k = 0; k < op.operands.size(); ++k) {
        const Dims& od = prog_.type(op.operands[k]).dims;
        const int64_t sz = od[cd];
        if (sz == 0) continue;
        const std::string lo = std::to_string(off) + "u", hi = std::to_string(sz - 1) + "u";
        std::string e;
        if (off == 0) {
          e = "(" + c + " < " + hi + " ? " + c + " : " + hi + ")";
        } else {
          e = "(" + c + " < " + lo + " ? 0u : (" + c + " - " + lo + " < " + hi + " ? " + c + " - " + lo + " : " + hi +
              "))";
        }
        Idx I;
        I.key = "c" + std::to_string(v) + "_" + std::to_string(k) + "(" + idxs_[id].key + ")";
        I.shape = od;
        I.multi = m;
        I.multi[cd] = e;
        vals.push_back(value(op.operands[k], add_index(I)));
        off += sz;
        ends.push_back(off);
      }
      PJRTX_CHECK(!vals.empty(), Code::kInternal, "concatenate with no elements inside a fusion");
      std::string e = vals.back();
      for (int k = static_cast<int>(vals.size()) - 2; k >= 0; --k)
        e = "(" + c + " < " + std::to_string(ends[k]) + "u ? " + vals[k] + " : " + e + ")";
      return define(R, e);
    }
    default:
      break;
  }
  PJRTX_CHECK(op_is_elementwise(op.kind), Code::kUnimplemented,
              std::string("cannot fuse op ") + op.name);
  std::vector<std::string> a;
  for (size_t k = 0; k < op.operands.size(); ++k) a.push_back(operand_at_same(static_cast<int>(k)));
  const DType A = prog_.type(op.operands[0]).dtype;
  const bool fa = dtype_is_float(A);
  const bool dbl = A == DType::kF64;
  const char* ct = dtype_compute_ctype(R);
  const char* act = dtype_compute_ctype(A);
  auto fl = [&](const std::string& e) { return define(R, round_to(R, e)); };
  auto fn1 = [&](const char* f32fn, const char* f64fn) {
    return fl(std::string(dbl ? f64fn : f32fn) + "(" + a[0] + ")");
  };
  switch (op.kind) {
    case OpKind::kAdd:
      if (R == DType::kPred) return define(R, a[0] + " || " + a[1]);
      return fa ? fl(a[0] + " + " + a[1]) : define(R, std::string("(") + ct + ")(" + a[0] + " + " + a[1] + ")");
    case OpKind::kSubtract:
      return fa ? fl(a[0] + " - " + a[1]) : define(R, std::string("(") + ct + ")(" + a[0] + " - " + a[1] + ")");
    case OpKind::kMultiply:
      if (R == DType::kPred) return define(R, a[0] + " && " + a[1]);
      return fa ? fl(a[0] + " * " + a[1]) : define(R, std::string("(") + ct + ")(" + a[0] + " * " + a[1] + ")");
    case OpKind::kDivide:
      if (fa) return fl(a[0] + " / " + a[1]);
      return define(R, std::string(dtype_is_signed_int(R) ? "div_s<" : "div_u<") + ct + ">(" + a[0] + ", " + a[1] + ")");
    case OpKind::kRemainder:
      if (fa) return fl(std::string(dbl ? "fmod(" : "fmodf(") + a[0] + ", " + a[1] + ")");
      return define(R, std::string(dtype_is_signed_int(R) ? "rem_s<" : "rem_u<") + ct + ">(" + a[0] + ", " + a[1] + ")");
    case OpKind::kPower:
      if (fa) return fl(std::string(dbl ? "pow(" : "powf(") + a[0] + ", " + a[1] + ")");
      return define(R, std::string("ipow<") + ct + ">(" + a[0] + ", " + a[1] + ")");
    case OpKind::kMaximum:
      if (fa) return fl(std::string(dbl ? "max_d(" : "max_f(") + a[0] + ", " + a[1] + ")");
      if (R == DType::kPred) return define(R, a[0] + " || " + a[1]);
      return define(R, std::string("max_i<") + ct + ">(" + a[0] + ", " + a[1] + ")");
    case OpKind::kMinimum:
      if (fa) return fl(std::string(dbl ? "min_d(" : "min_f(") + a[0] + ", " + a[1] + ")");
      if (R == DType::kPred) return define(R, a[0] + " && " + a[1]);
      return define(R, std::string("min_i<") + ct + ">(" + a[0] + ", " + a[1] + ")");
    case OpKind::kAnd:
      return define(R, R == DType::kPred ? a[0] + " && " + a[1] : std::string("(") + ct + ")(" + a[0] + " & " + a[1] + ")");
    case OpKind::kOr:
      return define(R, R == DType::kPred ? a[0] + " || " + a[1] : std::string("(") + ct + ")(" + a[0] + " | " + a[1] + ")");
    case OpKind::kXor:
      return define(R, R == DType::kPred ? a[0] + " != " + a[1] : std::string("(") + ct + ")(" + a[0] + " ^ " + a[1] + ")");
    case OpKind::kNot:
      return define(R, R == DType::kPred ? "!" + a[0] : std::string("(") + ct + ")(~" + a[0] + ")");
    case OpKind::kShiftLeft:
      return define(R, std::string("shl<") + ct + ", " + unsigned_of(R) + ">(" + a[0] + ", " + a[1] + ")");
    case OpKind::kShiftRightLogical:
      return define(R, std::string("shr_logical<") + ct + ", " + unsigned_of(R) + ">(" + a[0] + ", " + a[1] + ")");
    case OpKind::kShiftRightArithmetic:
      return define(R, std::string("shr_arith<") + ct + ", " + unsigned_of(R) + ">(" + a[0] + ", " + a[1] + ")");
    case OpKind::kAtan2: return fl(std::string(dbl ? "atan2(" : "atan2f(") + a[0] + ", " + a[1] + ")");
    case OpKind::kCompare: {
      static const char* ops[] = {"==", "!=", "<", "<=", ">", ">="};
      const char* o = ops[static_cast<int>(op.cmp_dir)];
      if (op.cmp_type == CmpType::kTotalOrder && fa)
        return define(R, "total_order_key(" + a[0] + ") " + o + " total_order_key(" + a[1] + ")");
      (void)act;
      return define(R, a[0] + " " + o + " " + a[1]);
    }
    case OpKind::kSelect: return define(R, a[0] + " ? " + a[1] + " : " + a[2]);
    case OpKind::kClamp: {
      // clamp(min, x, max)
      const DType X = prog_.type(op.operands[1]).dtype;
      if (dtype_is_float(X)) {
        const bool d = X == DType::kF64;
        return fl(std::string(d ? "min_d(max_d(" : "min_f(max_f(") + a[1] + ", " + a[0] + "), " + a[2] + ")");
      }
      return define(R, std::string("min_i<") + ct + ">(max_i<" + ct + ">(" + a[1] + ", " + a[0] + "), " + a[2] + ")");
    }
    case OpKind::kAbs:
      if (fa) return fn1("fabsf", "fabs");
      return define(R, std::string("(") + ct + ")(" + a[0] + " < 0 ? -" + a[0] + " : " + a[0] + ")");
    case OpKind::kNegate:
      return fa ? fl("-" + a[0]) : define(R, std::string("(") + ct + ")(-" + a[0] + ")");
    case OpKind::kExp: return R == DType::kF32 || dbl ? fn1("expf", "exp") : fn1("__expf", "exp");
    case OpKind::kExpm1: return fn1("expm1f", "expm1");
    case OpKind::kLog: return fn1("logf", "log");
    case OpKind::kLog1p: return fn1("log1pf", "log1p");
    case OpKind::kLogistic:
      return dbl ? fl("1.0 / (1.0 + exp(-" + a[0] + "))") : fl("1.0f / (1.0f + expf(-" + a[0] + "))");
    case OpKind::kSqrt: return fn1("sqrtf", "sqrt");
    case OpKind::kRsqrt: return dbl ? fl("1.0 / sqrt(" + a[0] + ")") : fl("1.0f / sqrtf(" + a[0] + ")");
    case OpKind::kCbrt: return fn1("cbrtf", "cbrt");
    case OpKind::kTanh: return fn1("tanhf", "tanh");
    case OpKind::kSine: return fn1("sinf", "sin");
    case OpKind::kCosine: return fn1("cosf", "cos");
    case OpKind::kTan: return fn1("tanf", "tan");
    case OpKind::kFloor: return fa ? fn1("floorf", "floor") : define(R, a[0]);
    case OpKind::kCeil: return fa ? fn1("ceilf", "ceil") : define(R, a[0]);
    case OpKind::kRoundAfz: return fn1("roundf", "round");
    case OpKind::kRoundEven: return fn1("rintf", "rint");
    case OpKind::kSign:
      if (fa) return fl(std::string(dbl ? "sign_d(" : "sign_f(") + a[0] + ")");
      return define(R, std::string("sign_i<") + ct + ">(" + a[0] + ")");
    case OpKind::kIsFinite: return define(R, "__builtin_isfinite(" + a[0] + ")");
    case OpKind::kPopcnt:
      // zero-extended through the unsigned type of the operand's width
      return define(R, std::string("(") + ct + ")" + (dtype_size(A) == 8 ? "__popcll((uint64_t)(" : "__popc((uint32_t)(") +
                           std::string(unsigned_of(A)) + ")" + a[0] + ")");
    case OpKind::kClz: {
      const size_t bits = dtype_size(A) * 8;
      if (bits == 64) return define(R, std::string("(") + ct + ")__clzll((int64_t)" + a[0] + ")");
      return define(R, std::string("(") + ct + ")(__clz((int32_t)(uint32_t)(" + unsigned_of(A) + ")" + a[0] + ") - " +
                           std::to_string(32 - bits) + ")");
    }
    case OpKind::kReducePrecision: {
      PJRTX_CHECK(op.exponent_bits >= 1 && op.mantissa_bits >= 0, Code::kInvalidArgument,
                  "reduce_precision: exponent_bits must be >= 1 and mantissa_bits >= 0");
      const char* fn = R == DType::kF32 ? "rp_f32" : R == DType::kF64 ? "rp_f64" : R == DType::kBF16 ? "rp_bf16"
                     : R == DType::kF16 ? "rp_f16" : nullptr;
      PJRTX_CHECK(fn != nullptr, Code::kUnimplemented, "reduce_precision: element type must be a float");
      return define(R, std::string(fn) + "(" + a[0] + ", " + std::to_string(op.exponent_bits) + ", " +
                           std::to_string(op.mantissa_bits) + ")");
    }
    case OpKind::kConvert: {
      const std::string x = a[0];
      if (R == DType::kPred) return define(R, x + " != 0");
      if (dtype_is_float(R)) {
        if (R == DType::kF64) return define(R, "(double)" + x);
        return fl("(float)" + x);
      }
      if (fa) {
        const std::string xf = dbl ? "(float)" + x : x;
        switch (R) {
          case DType::kS32: return define(R, "f2i32(" + xf + ")");
          case DType::kU32: return define(R, "f2u32(" + xf + ")");
          case DType::kS64: return define(R, "f2i64(" + xf + ")");
          case DType::kS8: return define(R, "f2i<int8_t>(" + xf + ", -128.0f, 127.0f)");
          case DType::kU8: return define(R, "f2i<uint8_t>(" + xf + ", 0.0f, 255.0f)");
          case DType::kS16: return define(R, "f2i<int16_t>(" + xf + ", -32768.0f, 32767.0f)");
          case DType::kU16: return define(R, "f2i<uint16_t>(" + xf + ", 0.0f, 65535.0f)");
          default: return define(R, std::string("(") + ct + ")(" + xf + ")");
        }
      }
      return define(R, std::string("(") + ct + ")(" + x + ")");
    }
    case OpKind::kBitcastConvert: {
      PJRTX_CHECK(dtype_size(A) == dtype_size(R), Code::kUnimplemented, "bitcast_convert between widths");
      const std::string s = to_storage(A, a[0]);
      return define(R, from_storage(R, std::string("__builtin_bit_cast(") + dtype_storage_ctype(R) + ", (" +
                                           dtype_storage_ctype(A) + ")(" + s + "))"));
    }
    default:
      fail(Code::kUnimplemented, std::string("cannot fuse op ") + op.name);
  }
}

// ----------------------------------------------------------------------------

struct Accum {
  ReducerKind kind;
  DType vt;            // value dtype (result 0)
  DType it;            // index dtype (argmax result 1)
  std::string acc_t;   // accumulator C type
  std::string v, i;    // accumulator variable names (i for argmax)
};

std::string acc_ctype(ReducerKind k, DType t) {
  if (k == ReducerKind::kAnd || k == ReducerKind::kOr) return "uint32_t";
  if (t == DType::kF64) return "double";
  if (dtype_is_float(t)) return "float";
  if (t == DType::kPred) return "uint32_t";
  return dtype_compute_ctype(t);
}

std::string identity_of(ReducerKind k, DType t, const std::string& ct) {
  const bool f = dtype_is_float(t);
  switch (k) {
    case ReducerKind::kSum: return "(" + ct + ")0";
    case ReducerKind::kProd: return "(" + ct + ")1";
    case ReducerKind::kAnd: return "1u";
    case ReducerKind::kOr: return "0u";
    case ReducerKind::kMax:
    case ReducerKind::kArgMax:
      if (f) return t == DType::kF64 ? "-__builtin_inf()" : "-__builtin_inff()";
      return dtype_is_signed_int(t) ? "(" + ct + ")((" + ct + ")1 << (sizeof(" + ct + ")*8-1))" : "(" + ct + ")0";
    case ReducerKind::kMin:
    case ReducerKind::kArgMin:
      if (f) return t == DType::kF64 ? "__builtin_inf()" : "__builtin_inff()";
      return dtype_is_signed_int(t) ? "(" + ct + ")(~((" + ct + ")1 << (sizeof(" + ct + ")*8-1)))" : "(" + ct + ")~(" + ct + ")0";
  }
  return "0";
}

// a = combine(a, b) for single-value reducers.
std::string combine_stmt(ReducerKind k, DType t, const std::string& a, const std::string& b) {
  const bool f = dtype_is_float(t);
  const bool d = t == DType::kF64;
  switch (k) {
    case ReducerKind::kSum: return a + " += " + b + ";";
    case ReducerKind::kProd: return a + " *= " + b + ";";
    case ReducerKind::kAnd: return a + " = " + a + " & (uint32_t)(" + b + ");";
    case ReducerKind::kOr: return a + " = " + a + " | (uint32_t)(" + b + ");";
    case ReducerKind::kMax:
      return a + " = " + (f ? (d ? "max_d(" : "max_r(") : "max_i(") + a + ", " + b + ");";
    case ReducerKind::kMin:
      return a + " = " + (f ? (d ? "min_d(" : "min_r(") : "min_i(") + a + ", " + b + ");";
    default: return "";
  }
}

std::string arg_better(ReducerKind k) { return k == ReducerKind::kArgMax ? "argmax_better" : "argmin_better"; }

// DPP exchange steps that fold lanes [0, width) into each of those lanes:
// xor 1 and xor 2 within quads, then the mirror within 8 lanes, then the
// mirror within the 16-lane row.
int dpp_steps_for(int width) { return width <= 2 ? 1 : width <= 4 ? 2 : width <= 8 ? 3 : 4; }

// Wavefront all-reduce of `v` (type `ty`) with the fold `comb(a, b)` (a
// statement updating a): four DPP exchange steps within rows of 16 lanes,
// then the four row values read from lanes 0, 16, 32, 48 and folded in a
// fixed tree. Every lane ends with the same value; the order is fixed, so
// the result is deterministic. With `width` <= 16 only lanes [0, width)
// carry values (the others hold the fold's identity): the first
// dpp_steps_for(width) steps leave the fold of those lanes in each of them,
// the same value the full form gives (identities change no result), and the
// later steps are not emitted.
std::string wave_allreduce(const std::string& ty, const std::string& v,
                           const std::function<std::string(const std::string&, const std::string&)>& comb, int width = 64) {
  static const char* const kSteps[4] = {"kDppXor1", "kDppXor2", "kDppHalfMirror", "kDppMirror"};
  const int steps = width <= 16 ? dpp_steps_for(width) : 4;
  std::ostringstream o;
  o << "{ " << ty << " o_;\n";
  for (int k = 0; k < steps; ++k) o << "o_ = dpp_move<" << kSteps[k] << ">(" << v << "); " << comb(v, "o_") << "\n";
  if (width > 16) {
    o << ty << " w1_ = lane_value(" << v << ", 16), w2_ = lane_value(" << v << ", 32), w3_ = lane_value(" << v << ", 48);\n";
    o << v << " = lane_value(" << v << ", 0);\n";
    o << comb(v, "w1_") << " " << comb("w2_", "w3_") << " " << comb(v, "w2_") << "\n";
  }
  o << "}\n";
  return o.str();
}

// The same for an argmax/argmin (value, index) pair under its comparator.
std::string wave_allreduce_arg(ReducerKind k, const std::string& ity, const std::string& v, const std::string& i,
                               int width = 64) {
  static const char* const kSteps[4] = {"kDppXor1", "kDppXor2", "kDppHalfMirror", "kDppMirror"};
  const int steps = width <= 16 ? dpp_steps_for(width) : 4;
  const std::string better = arg_better(k);
  std::ostringstream o;
  auto take = [&](const std::string& av, const std::string& ai, const std::string& bv, const std::string& bi) {
    return "if (" + better + "(" + bv + ", " + bi + ", " + av + ", " + ai + ")) { " + av + " = " + bv + "; " + ai + " = " + bi +
           "; }";
  };
  o << "{ float ov_; " << ity << " oi_;\n";
  for (int s = 0; s < steps; ++s)
    o << "ov_ = dpp_move<" << kSteps[s] << ">(" << v << "); oi_ = dpp_move<" << kSteps[s] << ">(" << i << "); "
      << take(v, i, "ov_", "oi_") << "\n";
  if (width > 16) {
    o << "float w1v_ = lane_value(" << v << ", 16), w2v_ = lane_value(" << v << ", 32), w3v_ = lane_value(" << v << ", 48);\n";
    o << ity << " w1i_ = lane_value(" << i << ", 16), w2i_ = lane_value(" << i << ", 32), w3i_ = lane_value(" << i << ", 48);\n";
    o << v << " = lane_value(" << v << ", 0); " << i << " = lane_value(" << i << ", 0);\n";
    o << take(v, i, "w1v_", "w1i_") << " " << take("w2v_", "w2i_", "w3v_", "w3i_") << " " << take(v, i, "w2v_", "w2i_") << "\n";
  }
  o << "}\n";
  return o.str();
}

class KernelGen {
 public:
  KernelGen(const Program& prog, std::ostringstream& out, int64_t nt_min_bytes = 0)
      : prog_(prog), out_(out), nt_min_bytes_(nt_min_bytes) {}
  void loop(Step& s);
  void reduce(Step& s);
  void row_fused(Step& s);
  void gemv(Step& s);

 private:
  const Program& prog_;
  std::ostringstream& out_;
  int64_t nt_min_bytes_ = 0;
  // "ldv<storage type, vec[, true]>": the vector load of input v, in its
  // non-temporal form when `stream` is set and v is at least nt_min_bytes_.
  // Reductions set it: their large inputs stream in once while little is
  // written (C1's 2 x 67 MB rows: 21.8 -> 20.7 us). Kernels that write as
  // much as they read do not (a 134 MB copy: 38.1 us with plain loads, 41.0
  // with non-temporal ones).
  std::string ldv_of(int v, int vec, bool stream = false) const {
    const bool nt = stream && nt_min_bytes_ > 0 && prog_.type(v).bytes() >= nt_min_bytes_;
    return std::string("ldv<") + dtype_storage_ctype(prog_.type(v).dtype) + ", " + std::to_string(vec) + (nt ? ", true>" : ">");
  }

  std::string idx_type(const Step& s) {
    int64_t m = 0;
    for (int v : s.inputs) m = std::max(m, prog_.type(v).elements());
    for (int v : s.outputs) m = std::max(m, prog_.type(v).elements());
    if (s.kind == StepKind::kReduce || s.kind == StepKind::kRowFused)
      m = std::max(m, num_elements(s.reduce_operand_shape));
    if (s.kind == StepKind::kLoop) m = std::max(m, num_elements(s.loop_shape));
    return m < (int64_t(1) << 31) ? "uint32_t" : "uint64_t";
  }
  void signature(const Step& s, std::map<int, std::string>* ptr_of, bool with_scratch, const char* suffix = "");
  struct RowTarget {
    std::string lds;  // LDS float array receiving the row (empty: the kernel's outputs)
    std::string row;  // row index expression when `lds` is set
    // Emitted right after the row's inputs are requested, before they are
    // used (a GEMV issues its weight loads there, so that waiting for the
    // row's inputs does not wait for the weights).
    std::function<void()> after_preload;
    // Inputs already staged in LDS by the caller (value -> array of its
    // storage elements): read from there, never from global memory.
    std::map<int, std::string> lds_inputs;
  };
  void row_body(Step& s, std::map<int, std::string>& ptr_of, const RowTarget& t);
  void gemv_epilogue(Step& s, const std::map<int, std::string>& ptr_of, const std::string& seg);
};

void KernelGen::signature(const Step& s, std::map<int, std::string>* ptr_of, bool with_scratch, const char* suffix) {
  // The separate combine kernel always runs 256 threads.
  const int bounds = suffix && *suffix ? 256 : std::max(256, static_cast<int>(s.block));
  out_ << "extern \"C\" __global__ void __launch_bounds__(" << bounds << ") " << s.name << suffix << "(";
  int k = 0;
  for (int v : s.inputs) {
    const DType t = prog_.type(v).dtype;
    out_ << (k ? ", " : "") << "const " << dtype_storage_ctype(t) << "* __restrict__ in" << k;
    (*ptr_of)[v] = "in" + std::to_string(k);
    ++k;
  }
  int o = 0;
  for (int v : s.outputs) {
    const DType t = prog_.type(v).dtype;
    out_ << (k + o ? ", " : "") << dtype_storage_ctype(t) << "* __restrict__ out" << o;
    ++o;
  }
  if (with_scratch) out_ << ", unsigned char* __restrict__ scratch";
  if (with_scratch && s.fused_combine) out_ << ", const uint32_t fused_mode";
  out_ << ") {\n";
}

void KernelGen::loop(Step& s) {
  std::map<int, std::string> ptr_of;
  signature(s, &ptr_of, false);
  const std::string it = idx_type(s);
  const int64_t n = num_elements(s.loop_shape);
  const int vec = s.vec;
  out_ << "typedef " << it << " idx_t;\n";
  out_ << "const idx_t n = " << n << "u;\n";
  out_ << "const idx_t base = ((idx_t)blockIdx.x * 256u + threadIdx.x) * " << vec << "u;\n";
  out_ << "if (base >= n) return;\n";
  out_ << "const bool full = base + " << vec << "u <= n;\n";
  Writer w(prog_, ptr_of, it);
  // Inputs with the root's element count are read at the root linear index
  // through a reshape chain at most: preload them as vectors.
  for (int v : s.inputs) {
    if (prog_.type(v).elements() != n) continue;
    const DType t = prog_.type(v).dtype;
    std::string name = "pre_" + ptr_of[v];
    out_ << dtype_storage_ctype(t) << " " << name << "[" << vec << "];\n";
    out_ << ldv_of(v, vec) << "(" << name << ", " << ptr_of[v] << ", base, n, full);\n";
    w.preload[v] = name;
  }
  for (size_t o = 0; o < s.outputs.size(); ++o) {
    out_ << dtype_storage_ctype(prog_.type(s.outputs[o]).dtype) << " res" << o << "[" << vec << "];\n";
  }
  Idx root;
  root.key = "R";
  root.shape = s.loop_shape;
  root.lin = "lin";
  root.identity = true;
  const int rid = w.add_index(root);
  w.multi_of(rid);  // unused digits are dropped by the compiler
  std::vector<std::string> vals;
  for (size_t o = 0; o < s.outputs.size(); ++o) {
    auto ww = s.window_out.find(static_cast<int>(o));
    vals.push_back(w.value(ww == s.window_out.end() ? s.outputs[o] : ww->second.update, rid));
  }
  // Window outputs (fused in-place dynamic_update_slice): clamped starts,
  // read once per thread.
  for (auto& [o, ww] : s.window_out) {
    const Dims& od = prog_.type(ww.operand).dims;
    for (size_t d = 0; d < ww.starts.size(); ++d) {
      const int sv = ww.starts[d];
      std::string e;
      auto pi = ptr_of.find(sv);
      if (pi != ptr_of.end()) {
        e = "(int64_t)" + pi->second + "[0]";
      } else {
        const Op* c = nullptr;
        for (const Op& op : prog_.ops)
          if (!op.results.empty() && op.results[0] == sv) c = &op;
        PJRTX_CHECK(c && c->kind == OpKind::kConstant, Code::kInternal, "window start is neither an input nor a constant");
        e = "(int64_t)(" + literal_expr(prog_, *c, 0) + ")";
      }
      const int64_t hi = od[d] - s.loop_shape[d];
      out_ << "int64_t ws" << o << "_" << d << " = " << e << ";\n";
      out_ << "ws" << o << "_" << d << " = ws" << o << "_" << d << " < 0 ? 0 : (ws" << o << "_" << d << " > " << hi
           << " ? " << hi << " : ws" << o << "_" << d << ");\n";
    }
  }
  out_ << "#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) {\n";
  out_ << "const idx_t lin = full ? base + j : ((base + j < n) ? base + j : n - 1u);\n";
  out_ << w.body.str();
  for (size_t o = 0; o < s.outputs.size(); ++o)
    out_ << "res" << o << "[j] = " << to_storage(prog_.type(s.outputs[o]).dtype, vals[o]) << ";\n";
  out_ << "}\n";
  for (size_t o = 0; o < s.outputs.size(); ++o) {
    const DType t = prog_.type(s.outputs[o]).dtype;
    auto ww = s.window_out.find(static_cast<int>(o));
    if (ww == s.window_out.end()) {
      out_ << "stv<" << dtype_storage_ctype(t) << ", " << vec << ">(out" << o << ", base, res" << o << ", n, full);\n";
      continue;
    }
    // The thread's vec elements lie in one innermost row of the window
    // (the window spans that dim, a multiple of vec): one store at the
    // window position of `base`.
    const Dims& od = prog_.type(ww->second.operand).dims;
    out_ << "{ uint32_t rem = base, dst = 0;\n";
    int64_t stride = 1;
    for (int d = static_cast<int>(od.size()) - 1; d >= 0; --d) {
      out_ << "{ const uint32_t c = rem % " << s.loop_shape[d] << "u; rem /= " << s.loop_shape[d] << "u; dst += (c + (uint32_t)ws"
           << o << "_" << d << ") * " << stride << "u; }\n";
      stride *= od[d];
    }
    out_ << "stv<" << dtype_storage_ctype(t) << ", " << vec << ">(out" << o << ", dst, res" << o << ", dst + (n - base), full); }\n";
  }
  out_ << "}\n\n";
}

void KernelGen::reduce(Step& s) {
  std::map<int, std::string> ptr_of;
  const bool split = s.row_schedule && s.splits > 1;
  signature(s, &ptr_of, split);
  const std::string it = idx_type(s);
  out_ << "typedef " << it << " idx_t;\n";
  const Dims& shape = s.reduce_operand_shape;
  const int rank = static_cast<int>(shape.size());
  auto is_red = [&](int d) {
    return std::binary_search(s.reduce_dims.begin(), s.reduce_dims.end(), static_cast<int64_t>(d));
  };
  Dims kept_dims, red_dims;
  for (int d = 0; d < rank; ++d) (is_red(d) ? red_dims : kept_dims).push_back(shape[d]);

  // Accumulators.
  std::vector<Accum> accs;
  for (size_t r = 0; r < s.reduces.size(); ++r) {
    const ReduceSpec& rs = s.reduces[r];
    Accum a;
    a.kind = rs.kind;
    a.vt = prog_.type(rs.results[0]).dtype;
    a.it = rs.results.size() > 1 ? prog_.type(rs.results[1]).dtype : DType::kInvalid;
    a.acc_t = acc_ctype(rs.kind, a.vt);
    a.v = "acc" + std::to_string(r);
    a.i = "aci" + std::to_string(r);
    accs.push_back(a);
  }
  // Argmax index accumulators are 32-bit when every index fits.
  const bool narrow_index = num_elements(shape) < (int64_t(1) << 31);
  const std::string ait = narrow_index ? "int32_t" : "int64_t";
  const std::string aimax = narrow_index ? "0x7fffffff" : "0x7fffffffffffffffll";

  Writer w(prog_, ptr_of, it);
  // Root index over the reduce operand shape.
  Idx root;
  root.key = "R";
  root.shape = shape;
  root.lin = "lin";
  root.identity = s.row_schedule;
  root.multi.resize(rank);
  const int vec = s.vec;

  std::ostringstream head;  // before the element loop
  bool epilogue_then_combine = false;  // fused combine: also emit the `_combine` fallback kernel
  std::string combine_fallback_body;
  if (s.row_schedule) {
    if (s.fused_combine && s.rows % 8 == 0) {
      // Workgroup b runs on XCD b % 8 and rows % 8 == 0: with row = b % rows
      // every split of a row lands on the same XCD (one L2).
      head << "const idx_t row = (idx_t)blockIdx.x % " << s.rows << "u;\n";
      head << "const idx_t split = (idx_t)blockIdx.x / " << s.rows << "u;\n";
    } else if (s.fused_combine) {
      // Padded grid: row (b % 8) + 8 * ((b / 8) / splits) keeps a row's
      // splits on XCD b % 8; workgroups past the last row exit.
      head << "const idx_t row = (idx_t)(blockIdx.x & 7u) + 8u * ((idx_t)(blockIdx.x >> 3) / " << s.splits << "u);\n";
      head << "const idx_t split = (idx_t)(blockIdx.x >> 3) % " << s.splits << "u;\n";
      head << "if (row >= " << s.rows << "u) return;\n";
    } else {
      head << "const idx_t row = (idx_t)blockIdx.x / " << s.splits << "u;\n";
      head << "const idx_t split = (idx_t)blockIdx.x - row * " << s.splits << "u;\n";
    }
    head << "const idx_t c0 = split * " << s.chunk << "u;\n";
    head << "const idx_t c1 = (c0 + " << s.chunk << "u < " << s.row_len << "u) ? c0 + " << s.chunk << "u : "
         << s.row_len << "u;\n";
    // kept digits from row, reduced digits from col
    std::string rest = "row";
    for (int d = rank - 1, k = static_cast<int>(kept_dims.size()) - 1; d >= 0; --d) {
      if (is_red(d)) continue;
      if (k == 0) {
        root.multi[d] = rest;
      } else {
        head << "const idx_t kd" << d << " = " << rest << " % " << shape[d] << "u;\n";
        head << "const idx_t kq" << d << " = " << rest << " / " << shape[d] << "u;\n";
        root.multi[d] = "kd" + std::to_string(d);
        rest = "kq" + std::to_string(d);
      }
      --k;
    }
  } else {
    head << "const idx_t row = (idx_t)blockIdx.x * 256u + threadIdx.x;\n";
    head << "if (row >= " << s.rows << "u) return;\n";
    std::string rest = "row";
    for (int d = rank - 1, k = static_cast<int>(kept_dims.size()) - 1; d >= 0; --d) {
      if (is_red(d)) continue;
      if (k == 0) {
        root.multi[d] = rest;
      } else {
        head << "const idx_t kd" << d << " = " << rest << " % " << shape[d] << "u;\n";
        head << "const idx_t kq" << d << " = " << rest << " / " << shape[d] << "u;\n";
        root.multi[d] = "kd" + std::to_string(d);
        rest = "kq" + std::to_string(d);
      }
      --k;
    }
  }
  // Reduced digits from `col` (emitted inside the element loop).
  std::ostringstream col_digits;
  {
    std::string rest = "col";
    for (int d = rank - 1, k = static_cast<int>(red_dims.size()) - 1; d >= 0; --d) {
      if (!is_red(d)) continue;
      if (k == 0) {
        root.multi[d] = rest;
      } else {
        col_digits << "const idx_t rd" << d << " = " << rest << " % " << shape[d] << "u;\n";
        col_digits << "const idx_t rq" << d << " = " << rest << " / " << shape[d] << "u;\n";
        root.multi[d] = "rd" + std::to_string(d);
        rest = "rq" + std::to_string(d);
      }
      --k;
    }
  }
  if (kept_dims.empty()) {
    // nothing: all dims reduced
  }
  const int rid = w.add_index(root);
  // Values of every reduce operand at the root.
  std::vector<std::vector<std::string>> xs(s.reduces.size());
  // Preloads (row schedule only): `unroll` sub-chunks of `vec` elements per
  // thread are all requested before any is consumed, so that each thread has
  // several 16-byte loads in flight. The element body reads P_<input>[j],
  // bound to the current sub-chunk's registers.
  std::ostringstream pre_decl, pre_load;
  const int unroll = std::max<int>(1, s.unroll);
  if (s.row_schedule) {
    const int64_t n_all = num_elements(shape);
    for (int v : s.inputs) {
      if (prog_.type(v).elements() != n_all) continue;
      const DType t = prog_.type(v).dtype;
      const std::string st = dtype_storage_ctype(t);
      const std::string name = "pre_" + ptr_of[v];
      pre_decl << st << " " << name << "[" << unroll << "][" << vec << "];\n";
      // row_len and chunk are multiples of vec, so a sub-chunk lies wholly
      // inside or wholly outside [c0, c1): whole 16-byte loads only.
      pre_load << ldv_of(v, vec, true) << "(" << name << "[u], " << ptr_of[v] << ", row * " << s.row_len
               << "u + cu, 0u, true);\n";
      w.preload[v] = "P_" + ptr_of[v];
    }
    if (s.row_len % vec != 0 || s.chunk % vec != 0)
      fail(Code::kInternal, "reduce kernel: row length and chunk must be multiples of the vector width");
  }
  // f32 sums of f16 values (JAX's f16 sum: convert f16->f32, add) fold each
  // element with one mixed-precision FMA on the f16 value (add_f16v), or, in
  // the row schedule's vectorised loop, each pair of elements with one packed
  // convert and one dot2 (add2_f16v).
  std::vector<bool> f16_sum(s.reduces.size(), false);
  std::vector<std::string> f16_pre(s.reduces.size());
  for (size_t r = 0; r < s.reduces.size(); ++r) {
    const ReduceSpec& rs = s.reduces[r];
    for (int v : rs.inputs) {
      // max/min of a float->float convert: a rounding is monotone, so the
      // running max/min is kept on the unconverted value and rounded once in
      // the final step (which rounds to the result type anyway).
      const bool mm = rs.kind == ReducerKind::kMax || rs.kind == ReducerKind::kMin;
      const bool sum32 = rs.kind == ReducerKind::kSum && rs.inputs.size() == 1 && prog_.type(v).dtype == DType::kF32;
      int src = v;
      for (const Op& op : prog_.ops) {
        if (op.results.empty() || op.results[0] != v || op.kind != OpKind::kConvert) continue;
        const DType from = prog_.type(op.operands[0]).dtype, to = prog_.type(v).dtype;
        const bool f32ish = [](DType t) { return t == DType::kF32 || t == DType::kF16 || t == DType::kBF16; }(from);
        if (mm && f32ish && (to == DType::kF32 || to == DType::kF16 || to == DType::kBF16)) src = op.operands[0];
        if (sum32 && from == DType::kF16) {
          src = op.operands[0];
          f16_sum[r] = true;
        }
      }
      xs[r].push_back(w.value(src, rid));
      // The f16 value's own source when it is a convert from f32 or bf16:
      // add2_f16v rounds that value to f16 itself (one packed convert for two
      // elements), which is the same rounding (bf16 widens to f32 exactly).
      if (f16_sum[r])
        for (const Op& op : prog_.ops)
          if (!op.results.empty() && op.results[0] == src && op.kind == OpKind::kConvert &&
              (prog_.type(op.operands[0]).dtype == DType::kF32 || prog_.type(op.operands[0]).dtype == DType::kBF16))
            f16_pre[r] = "(float)(" + w.value(op.operands[0], rid) + ")";
    }
  }
  std::string elem_body = w.body.str();

  out_ << head.str();
  for (auto& a : accs) {
    out_ << a.acc_t << " " << a.v << " = " << identity_of(a.kind, a.vt, a.acc_t) << ";\n";
    if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin)
      out_ << ait << " " << a.i << " = " << aimax << ";\n";
  }
  // In-thread update. A thread visits its elements by increasing column, so
  // when the index operand is the column the in-order forms (argmax_take,
  // max_seq, min_seq) give the same result as the full pair comparator with
  // fewer instructions; any other index operand folds with the comparator.
  // An index operand that is an iota along the one reduced dimension is the
  // column itself (the deferred scan below recomputes it instead of keeping
  // it).
  std::vector<bool> idx_is_col(s.reduces.size(), false);
  for (size_t r = 0; r < s.reduces.size(); ++r) {
    const ReduceSpec& rs = s.reduces[r];
    if (rs.inputs.size() != 2 || red_dims.size() != 1) continue;
    for (const Op& op : prog_.ops)
      if (!op.results.empty() && op.results[0] == rs.inputs[1] && op.kind == OpKind::kIota && is_red(static_cast<int>(op.dim)) &&
          prog_.type(rs.inputs[1]).dims == shape && !dtype_is_float(prog_.type(rs.inputs[1]).dtype))
        idx_is_col[r] = true;
  }
  auto is_arg = [](const Accum& a) { return a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin; };
  // Float-valued argmax/argmin: the two-phase and deferred folds apply.
  auto fast_arg = [&](size_t r) { return is_arg(accs[r]) && accs[r].acc_t == "float"; };
  // Whole vec-element sub-chunks of the row schedule fold an argmax in two
  // phases: the sub-chunk's max (IEEE maximum, NaN propagating; two new
  // values per instruction), then the first element equal to it (or the
  // first NaN) found by a backward scan, merged into the running pair with
  // the in-order rule. Same winner and value bits as the element-wise fold.
  auto two_phase_decl = [&](std::ostream& o) {
    for (size_t r = 0; r < accs.size(); ++r)
      if (fast_arg(r) && idx_is_col[r])
        o << "float xa" << r << "[" << vec << "]; " << ait << " ia" << r << "[" << vec << "]; float mc" << r << " = "
          << (accs[r].kind == ReducerKind::kArgMax ? "-__builtin_inff()" : "__builtin_inff()") << ";\n";
  };
  auto two_phase_finish = [&](std::ostream& o) {
    for (size_t r = 0; r < accs.size(); ++r) {
      const Accum& a = accs[r];
      if (!fast_arg(r) || !idx_is_col[r]) continue;
      const char* take = a.kind == ReducerKind::kArgMax ? "argmax_take" : "argmin_take";
      const std::string R = std::to_string(r);
      o << "{ float sv = mc" << R << "; " << ait << " si = 0;\n";
      o << "if (__any(mc" << R << " != mc" << R << ")) {\n";
      o << "const bool mn = mc" << R << " != mc" << R << ";\n";
      o << "#pragma unroll\nfor (int j = " << vec - 1 << "; j >= 0; --j) { const bool hit = mn ? (xa" << R << "[j] != xa"
        << R << "[j]) : (xa" << R << "[j] == mc" << R << "); sv = hit ? xa" << R << "[j] : sv; si = hit ? ia" << R
        << "[j] : si; }\n";
      o << "} else {\n";
      o << "#pragma unroll\nfor (int j = " << vec - 1 << "; j >= 0; --j) { const bool hit = xa" << R << "[j] == mc" << R
        << "; sv = hit ? xa" << R << "[j] : sv; si = hit ? ia" << R << "[j] : si; }\n";
      o << "}\n";
      o << "const bool bt = " << take << "(sv, " << a.v << "); " << a.v << " = bt ? sv : " << a.v << "; " << a.i
        << " = bt ? si : " << a.i << "; }\n";
    }
  };
  // Single-pass row schedule (each thread's share fits one unrolled pass)
  // defers the argmax index entirely: the pass keeps the values in registers
  // and folds only the IEEE maximum of each vec-element sub-chunk (shared
  // with a max over the same values). Each wavefront then finds its own
  // winner with no barrier: its maximum m (NaN if any lane saw one); with
  // the column as index, the first sub-chunk u (in column order: u, then
  // lane) whose maximum is m, found by one ballot per u, then that lane's
  // first element equal to m (or first NaN). Any other index operand scans
  // every element for the lowest index among those equal to m, then takes
  // the wavefront's lowest (all of them tie on value). The winner is the
  // comparator's (NaN first, then the larger value, ties to the lower index)
  // with that element's value bits; the wavefront winners meet in the block
  // step.
  auto ident = [&](size_t r) {
    return accs[r].kind == ReducerKind::kArgMax || accs[r].kind == ReducerKind::kMax ? std::string("-__builtin_inff()")
                                                                                      : std::string("__builtin_inff()");
  };
  // A float max/min over the same values as a deferred argmax/argmin folds
  // that argmax's sub-chunk maxima instead of every element.
  std::vector<int> shares(accs.size(), -1);
  for (size_t r = 0; r < accs.size(); ++r) {
    const Accum& a = accs[r];
    if (a.acc_t != "float" || (a.kind != ReducerKind::kMax && a.kind != ReducerKind::kMin)) continue;
    for (size_t r2 = 0; r2 < accs.size(); ++r2)
      if (fast_arg(r2) && xs[r2][0] == xs[r][0] &&
          (accs[r2].kind == ReducerKind::kArgMax) == (a.kind == ReducerKind::kMax)) {
        shares[r] = static_cast<int>(r2);
        break;
      }
  }
  auto deferred_decl = [&](std::ostream& o) {
    for (size_t r = 0; r < accs.size(); ++r) {
      if (!fast_arg(r)) continue;
      o << "float xa" << r << "[" << unroll << "][" << vec << "]; float mu" << r << "[" << unroll << "]; ";
      if (!idx_is_col[r]) o << ait << " ia" << r << "[" << unroll << "][" << vec << "]; ";
      o << "\n";
    }
  };
  std::vector<bool> wave_done(accs.size(), false);
  auto deferred_finish = [&](std::ostream& o, int full_u) {
    for (size_t r = 0; r < accs.size(); ++r) {
      const Accum& a = accs[r];
      if (!fast_arg(r)) continue;
      wave_done[r] = true;
      const std::string R = std::to_string(r);
      const char* mx = a.kind == ReducerKind::kArgMax ? "max_r" : "min_r";
      const std::string span = std::to_string(s.block * vec) + "u";
      o << "{ float bm = mu" << R << "[0];\n";
      o << "#pragma unroll\nfor (int u = 1; u < " << unroll << "; ++u) bm = " << mx << "(bm, mu" << R << "[u]);\n";
      o << wave_allreduce("float", "bm", [&](const std::string& x, const std::string& y) {
        return x + " = " + mx + "(" + x + ", " + y + ");";
      });
      o << "const bool bn = bm != bm;\n";
      // A max (min) over the same values as this argmax (argmin) folds the
      // same sub-chunk maxima (minima) in the same total order (IEEE
      // maximum/minimum): its wavefront result is bm.
      for (size_t r2 = 0; r2 < accs.size(); ++r2)
        if (shares[r2] == static_cast<int>(r)) {
          o << accs[r2].v << " = bm;\n";
          wave_done[r2] = true;
        }
      o << "const idx_t c = c0 + threadIdx.x * " << vec << "u;\n";
      if (idx_is_col[r]) {
        // bm is the same in every lane, so the NaN and the ordinary case are
        // separate uniform branches: each ballot is then one compare.
        o << "int fu = -1; unsigned long long fm = 0ull;\n";
        for (int nan_case = 0; nan_case < 2; ++nan_case) {
          o << (nan_case ? "} else {\n" : "if (!bn) {\n");
          o << "#pragma unroll\nfor (int u = " << unroll - 1 << "; u >= 0; --u) {\n";
          o << "const bool ok = u < " << full_u << " || c + (idx_t)u * " << span << " < c1;\n";
          o << "const unsigned long long m = __ballot(ok && "
            << (nan_case ? "mu" + R + "[u] != mu" + R + "[u]" : "mu" + R + "[u] == bm") << ");\n";
          o << "if (m) { fu = u; fm = m; }\n}\n";
        }
        o << "}\n";
        o << a.v << " = bm; " << a.i << " = " << aimax << ";\n";
        // Lane L's first hit in sub-chunk fu: one ballot per element (all
        // independent), then bit L of each, picked in scalar code. The value
        // bits are bm's except for a zero maximum (the sign of the first
        // zero) or a NaN (its payload): those read lane L's elements.
        o << "if (fm) {\n";
        o << "const int L = __ffsll(fm) - 1;\n";
        o << "int sj = " << vec - 1 << "; int svb = __builtin_bit_cast(int, bm);\n";
        o << "#pragma unroll\nfor (int u = 0; u < " << unroll << "; ++u) {\n";
        o << "if (u == fu) {\n";
        o << "unsigned long long hj[" << vec << "];\n";
        for (int nan_case = 0; nan_case < 2; ++nan_case) {
          o << (nan_case ? "} else {\n" : "if (!bn) {\n");
          o << "#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) { const float x = xa" << R << "[u][j]; hj[j] = __ballot("
            << (nan_case ? "x != x" : "x == bm") << "); }\n";
        }
        o << "}\n";
        o << "#pragma unroll\nfor (int j = " << vec - 2 << "; j >= 0; --j) if ((hj[j] >> L) & 1ull) sj = j;\n";
        o << "if (bn || bm == 0.f) {\n";
        o << "#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) { const int b = __builtin_amdgcn_readlane(__builtin_bit_cast(int, xa"
          << R << "[u][j]), L); svb = j == sj ? b : svb; }\n";
        o << "}\n}\n}\n";
        o << a.v << " = __builtin_bit_cast(float, svb);\n";
        o << a.i << " = (" << ait << ")(c0 + ((threadIdx.x & ~63u) + (idx_t)L) * " << vec << "u + (idx_t)fu * " << span
          << " + (idx_t)sj);\n";
        o << "}\n}\n";
      } else {
        o << "float sv = bm; " << ait << " si = " << aimax << ";\n";
        o << "#pragma unroll\nfor (int u = 0; u < " << unroll << "; ++u) {\n";
        o << "const bool ok = u < " << full_u << " || c + (idx_t)u * " << span << " < c1;\n";
        o << "#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) {\n";
        o << "const float x = xa" << R << "[u][j]; const " << ait << " ix = ia" << R << "[u][j];\n";
        o << "const bool hit = ok && (bn ? x != x : x == bm) && ix < si;\n";
        o << "sv = hit ? x : sv; si = hit ? ix : si;\n}\n}\n";
        o << ait << " wi = si;\n";
        o << wave_allreduce(ait, "wi", [](const std::string& x, const std::string& y) {
          return x + " = " + y + " < " + x + " ? " + y + " : " + x + ";";
        });
        o << a.v << " = wave_value_at(sv, si == wi); " << a.i << " = wi; }\n";
      }
    }
  };
  // mode 0: element-wise fold; 1: per-sub-chunk two-phase argmax; 2: deferred argmax.
  // pairs: the caller's unrolled loop over j = 0..vec-1 (vec even) lets an
  // f16 sum hold element j's value when j is even and add the pair at the
  // odd j (add2_f16v).
  auto combine_elem = [&](std::ostream& o, int mode, bool pairs = false) {
    for (size_t r = 0; r < accs.size(); ++r) {
      const Accum& a = accs[r];
      const char* mx = a.kind == ReducerKind::kArgMax ? "max_r(" : "min_r(";
      if (mode == 1 && fast_arg(r) && idx_is_col[r]) {
        o << "xa" << r << "[j] = (float)" << xs[r][0] << "; ia" << r << "[j] = (" << ait << ")" << xs[r][1] << "; mc" << r
          << " = " << mx << "mc" << r << ", xa" << r << "[j]);\n";
      } else if (mode == 2 && fast_arg(r)) {
        o << "xa" << r << "[u][j] = (float)" << xs[r][0] << "; ";
        if (!idx_is_col[r]) o << "ia" << r << "[u][j] = (" << ait << ")" << xs[r][1] << "; ";
        o << "mu" << r << "[u] = " << mx << "mu" << r << "[u], xa" << r << "[u][j]);\n";
      } else if (mode == 2 && shares[r] >= 0) {
        // folded from the sub-chunk maximum after the element loop
      } else if ((a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin) && idx_is_col[r]) {
        const char* take = a.kind == ReducerKind::kArgMax ? "argmax_take" : "argmin_take";
        o << "{ const float xv = (float)" << xs[r][0] << "; const bool bt = " << take << "(xv, " << a.v << "); " << a.v
          << " = bt ? xv : " << a.v << "; " << a.i << " = bt ? (" << ait << ")" << xs[r][1] << " : " << a.i << "; }\n";
      } else if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin) {
        o << "{ const float xv = (float)" << xs[r][0] << "; const " << ait << " xi = (" << ait << ")" << xs[r][1]
          << "; if (" << arg_better(a.kind) << "(xv, xi, " << a.v << ", " << a.i << ")) { " << a.v << " = xv; " << a.i
          << " = xi; } }\n";
      } else if ((a.kind == ReducerKind::kMax || a.kind == ReducerKind::kMin) && a.acc_t == "float") {
        o << a.v << " = " << (a.kind == ReducerKind::kMax ? "max_seq(" : "min_seq(") << a.v << ", (float)(" << xs[r][0]
          << "));\n";
      } else if (f16_sum[r] && a.acc_t == "float" && pairs) {
        const std::string x = f16_pre[r].empty() ? xs[r][0] : f16_pre[r];
        o << "if (j & 1) " << a.v << " = add2_f16v(" << a.v << ", f16p" << r << ", " << x << "); else f16p" << r << " = " << x
          << ";\n";
      } else if (f16_sum[r] && a.acc_t == "float") {
        o << a.v << " = add_f16v(" << a.v << ", " << xs[r][0] << ");\n";
      } else {
        o << combine_stmt(a.kind, a.vt, a.v, "(" + a.acc_t + ")(" + xs[r][0] + ")") << "\n";
      }
    }
  };
  if (s.row_schedule) {
    const int64_t span = static_cast<int64_t>(s.block) * vec;
    const int nwaves = static_cast<int>(s.block) / 64;
    bool any_fast = false, any_two_phase = false;
    for (size_t r = 0; r < accs.size(); ++r) {
      any_fast = any_fast || fast_arg(r);
      any_two_phase = any_two_phase || (fast_arg(r) && idx_is_col[r]);
    }
    // chunk <= span * unroll: the loop below would run at most once.
    const bool single = s.chunk <= span * unroll;
    const bool deferred = single && vec > 1 && any_fast;
    const bool two_phase = !deferred && vec > 1 && any_two_phase;
    // Single pass: the first full_u sub-chunks are in range for every thread
    // of every split (the shortest split is the last), so they need no guard.
    int full_u = 0;
    if (single) {
      const int64_t min_len = s.row_len - (s.splits - 1) * s.chunk;
      while (full_u < unroll && full_u * span + span <= min_len) ++full_u;
    }
    out_ << pre_decl.str();
    if (deferred) deferred_decl(out_);
    if (single)
      out_ << "{\nconst idx_t c = c0 + threadIdx.x * " << vec << "u;\n";
    else
      out_ << "for (idx_t c = c0 + threadIdx.x * " << vec << "u; c < c1; c += " << span * unroll << "u) {\n";
    // Loads are unconditional (an out-of-range sub-chunk reads the split's
    // first one and is not folded), so they retire in issue order and each
    // sub-chunk waits only for its own.
    out_ << "#pragma unroll\nfor (int u = 0; u < " << unroll << "; ++u) {\n";
    out_ << "const idx_t cu = (u < " << full_u << " || c + (idx_t)u * " << span << "u < c1) ? c + (idx_t)u * " << span
         << "u : c0;\n";
    out_ << pre_load.str();
    out_ << "}\n";
    out_ << "#pragma unroll\nfor (int u = 0; u < " << unroll << "; ++u) {\n";
    out_ << "const idx_t cu = c + (idx_t)u * " << span << "u;\n";
    for (auto& [v, pname] : w.preload) out_ << "const auto& " << pname << " = pre_" << ptr_of[v] << "[u];\n";
    out_ << "if (u < " << full_u << " || cu < c1) {\n";
    if (two_phase) two_phase_decl(out_);
    if (deferred)
      for (size_t r = 0; r < accs.size(); ++r)
        if (fast_arg(r)) out_ << "mu" << r << "[u] = " << ident(r) << ";\n";
    const bool pairs = vec % 2 == 0;
    if (pairs)
      for (size_t r = 0; r < accs.size(); ++r)
        if (f16_sum[r] && accs[r].acc_t == "float") out_ << "float f16p" << r << " = 0.f;\n";
    out_ << "#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) {\n";
    out_ << "const idx_t col = cu + j;\nconst idx_t lin = row * " << s.row_len << "u + col;\n";
    out_ << col_digits.str() << elem_body;
    combine_elem(out_, deferred ? 2 : two_phase ? 1 : 0, pairs);
    out_ << "}\n";
    if (two_phase) two_phase_finish(out_);
    if (deferred)
      for (size_t r = 0; r < accs.size(); ++r)
        if (shares[r] >= 0)
          out_ << accs[r].v << " = " << (accs[r].kind == ReducerKind::kMax ? "max_r(" : "min_r(") << accs[r].v << ", mu"
               << shares[r] << "[u]);\n";
    out_ << "}\n";
    if (deferred && full_u < unroll) {
      out_ << "else {\n";
      for (size_t r = 0; r < accs.size(); ++r)
        if (fast_arg(r))
          out_ << "mu" << r << "[u] = " << ident(r) << ";\n#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) xa" << r
               << "[u][j] = 0.f;\n";
      out_ << "}\n";
    }
    out_ << "}\n";
    if (full_u < unroll && w.preload.size() > 0) {
      out_ << "#pragma unroll\nfor (int u = " << full_u << "; u < " << unroll << "; ++u) {\n";
      for (auto& [v, pname] : w.preload) out_ << "keep_live(pre_" << ptr_of[v] << "[u]);\n";
      out_ << "}\n";
    }
    out_ << "}\n";
    // Block reduction: wavefront all-reduce, then the wave results are
    // combined in wave order by thread 0 (fixed order: deterministic).
    // width: lanes that hold values (the fold of the split partials: one
    // lane per split).
    auto wave_reduce = [&](bool skip_done, int width) {
      for (size_t r = 0; r < accs.size(); ++r) {
        const Accum& a = accs[r];
        if (skip_done && wave_done[r]) continue;
        const bool am = a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin;
        if (am) {
          out_ << wave_allreduce_arg(a.kind, ait, a.v, a.i, width);
        } else {
          const ReducerKind k = a.kind;
          const DType vt = a.vt;
          out_ << wave_allreduce(a.acc_t, a.v, [&](const std::string& x, const std::string& y) { return combine_stmt(k, vt, x, y); },
                                 width);
        }
      }
    };
    if (deferred) deferred_finish(out_, full_u);
    // Shared slots for the cross-wave step of the block reductions.
    for (auto& a : accs) {
      out_ << "__shared__ " << a.acc_t << " sm_" << a.v << "[" << nwaves << "];\n";
      if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin)
        out_ << "__shared__ " << ait << " sm_" << a.i << "[" << nwaves << "];\n";
    }
    auto block_reduce = [&]() {
      wave_reduce(true, 64);
      out_ << "if ((threadIdx.x & 63) == 0) {\n";
      for (auto& a : accs) {
        out_ << "sm_" << a.v << "[threadIdx.x >> 6] = " << a.v << ";\n";
        if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin)
          out_ << "sm_" << a.i << "[threadIdx.x >> 6] = " << a.i << ";\n";
      }
      out_ << "}\n__syncthreads();\n";
      out_ << "if (threadIdx.x == 0) {\n";
      for (auto& a : accs) {
        const bool am = a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin;
        out_ << a.v << " = sm_" << a.v << "[0];\n";
        if (am) out_ << a.i << " = sm_" << a.i << "[0];\n";
        out_ << "for (int k = 1; k < " << nwaves << "; ++k) {\n";
        if (am) {
          out_ << "if (" << arg_better(a.kind) << "(sm_" << a.v << "[k], sm_" << a.i << "[k], " << a.v << ", " << a.i
               << ")) { " << a.v << " = sm_" << a.v << "[k]; " << a.i << " = sm_" << a.i << "[k]; }\n";
        } else {
          out_ << combine_stmt(a.kind, a.vt, a.v, "sm_" + a.v + "[k]") << "\n";
        }
        out_ << "}\n";
      }
      out_ << "}\n";
    };
    // Partial-slot layout in scratch: per reducer a [rows*splits] array of
    // 8-byte slots (argmax: value slots, then index slots).
    const int64_t slots = s.rows * s.splits;
    std::vector<size_t> offs;
    {
      size_t off = 0;
      for (auto& a : accs) {
        offs.push_back(off);
        off += static_cast<size_t>(slots) * 8;
        if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin) off += static_cast<size_t>(slots) * 8;
      }
    }
    block_reduce();
    // Fold of a row's partials by one wavefront, lane k reading split k
    // (wavefront all-reduce over the lanes: a fixed order, so the result does
    // not depend on which workgroup folds or on the launch).
    auto fold_partials = [&](bool coherent) {
      // coherent: loads that skip this CU's L1 and read the XCD's L2, where
      // the other workgroups' partial stores have landed.
      auto ld = [&](const std::string& addr) {
        return coherent ? "__hip_atomic_load(&" + addr + ", __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)" : addr;
      };
      for (size_t r = 0; r < accs.size(); ++r) {
        const Accum& a = accs[r];
        const bool am = a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin;
        out_ << a.v << " = " << identity_of(a.kind, a.vt, a.acc_t) << ";\n";
        if (am) out_ << a.i << " = " << aimax << ";\n";
        out_ << "if (lane < " << s.splits << "u) {\n";
        out_ << "uint64_t* slot = reinterpret_cast<uint64_t*>(scratch + " << offs[r] << "u);\n";
        out_ << "const uint64_t bits = " << ld("slot[row * " + std::to_string(s.splits) + "u + lane]") << ";\n";
        out_ << "__builtin_memcpy(&" << a.v << ", &bits, sizeof(" << a.v << "));\n";
        if (am)
          out_ << a.i << " = (" << ait << ")"
               << ld("slot[" + std::to_string(slots) + "u + row * " + std::to_string(s.splits) + "u + lane]") << ";\n";
        out_ << "}\n";
      }
      // Lanes at or past the split count hold identities: only the first
      // splits lanes need folding (lane 0 keeps the result).
      wave_reduce(false, static_cast<int>(s.splits));
      out_ << "if (lane != 0) return;\n";
    };
    if (split && s.fused_combine) {
      // Thread 0 stores this split's partials. In fused mode (the device
      // places workgroup b on XCD b % 8, probed at start-up) every split of
      // the row runs on this XCD: once the stores are acknowledged by its L2
      // (s_waitcnt), an L2 atomic counts the row's arrivals, and the
      // workgroup that arrives last folds every split with wavefront 0,
      // reading the slots past its L1, and puts the counter back to zero.
      // No device-scope fence (an L2 write-back on this GPU) is needed, and
      // no workgroup waits for another. Otherwise (fused_mode 0) the
      // partials stay for the `_combine` kernel launched next.
      // Only wavefront 0 takes part from here: the other wavefronts leave,
      // and lane 0's arrival verdict reaches its wavefront by readfirstlane
      // (no LDS round trip, no barrier).
      out_ << "if (threadIdx.x >= 64) return;\n";
      out_ << "uint32_t last = 0u;\n";
      out_ << "if (threadIdx.x == 0) {\n";
      for (size_t r = 0; r < accs.size(); ++r) {
        const Accum& a = accs[r];
        out_ << "{ uint64_t* slot = reinterpret_cast<uint64_t*>(scratch + " << offs[r] << "u);\n";
        out_ << "uint64_t bits = 0; __builtin_memcpy(&bits, &" << a.v << ", sizeof(" << a.v << "));\n";
        out_ << "slot[row * " << s.splits << "u + split] = bits;\n";
        if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin)
          out_ << "slot[" << slots << "u + row * " << s.splits << "u + split] = (uint64_t)" << a.i << ";\n";
        out_ << "}\n";
      }
      out_ << "if (fused_mode) {\n";
      // The workgroup-scope release fence keeps the compiler from moving the
      // slot stores past the counter RMW (it emits a wait for them, no cache
      // write-back); s_waitcnt(0) then has every store acknowledged by the
      // XCD's L2 before the RMW reaches that same L2.
      out_ << "__builtin_amdgcn_fence(__ATOMIC_RELEASE, \"workgroup\");\n";
      out_ << "__builtin_amdgcn_s_waitcnt(0);\n";
      // one counter per 128-byte line: rows do not contend for a line
      out_ << "uint32_t* ctr = reinterpret_cast<uint32_t*>(scratch + " << s.counter_offset << "u) + row * 32u;\n";
      out_ << "last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == " << s.splits - 1
           << "u;\n";
      out_ << "if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n";
      out_ << "}\n";
      out_ << "}\n";
      out_ << "if (!__builtin_amdgcn_readfirstlane(last)) return;\n";
      // Keeps the fold's slot loads after the RMW that decided `last`.
      out_ << "__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, \"workgroup\");\n";
      out_ << "const uint32_t lane = threadIdx.x;\n";
      fold_partials(true);
      epilogue_then_combine = true;
      {
        // text of the fallback combine kernel's fold (emitted after the epilogue)
        std::ostringstream saved;
        saved << out_.str();
        out_.str("");
        out_.clear();
        for (size_t r = 0; r < accs.size(); ++r) {
          const Accum& a = accs[r];
          out_ << a.acc_t << " " << a.v << ";\n";
          if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin) out_ << ait << " " << a.i << ";\n";
        }
        fold_partials(false);
        combine_fallback_body = out_.str();
        out_.str("");
        out_.clear();
        out_ << saved.str();
      }
    } else if (split) {
      // Partials of this split go to scratch with plain stores; the
      // `<name>_combine` kernel (launched next on the same stream) folds
      // them. The kernel boundary publishes the stores, so no per-workgroup
      // device-scope fence is needed.
      out_ << "if (threadIdx.x != 0) return;\n";
      for (size_t r = 0; r < accs.size(); ++r) {
        const Accum& a = accs[r];
        out_ << "{ uint64_t* slot = reinterpret_cast<uint64_t*>(scratch + " << offs[r] << "u);\n";
        out_ << "uint64_t bits = 0; __builtin_memcpy(&bits, &" << a.v << ", sizeof(" << a.v << "));\n";
        out_ << "slot[row * " << s.splits << "u + split] = bits;\n";
        if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin)
          out_ << "slot[" << slots << "u + row * " << s.splits << "u + split] = (uint64_t)" << a.i << ";\n";
        out_ << "}\n";
      }
      out_ << "}\n\n";
      // Combine kernel: one wavefront per row, lane k reads split k.
      signature(s, &ptr_of, true, "_combine");
      out_ << "typedef " << it << " idx_t;\n";
      out_ << "const idx_t row = (idx_t)blockIdx.x * 4u + (threadIdx.x >> 6);\n";
      out_ << "if (row >= " << s.rows << "u) return;\n";
      out_ << "const uint32_t lane = threadIdx.x & 63u;\n";
      for (size_t r = 0; r < accs.size(); ++r) {
        const Accum& a = accs[r];
        out_ << a.acc_t << " " << a.v << ";\n";
        if (a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin) out_ << ait << " " << a.i << ";\n";
      }
      fold_partials(false);
    } else {
      out_ << "if (threadIdx.x != 0) return;\n";
    }
  } else {
    // Column schedule: one thread per output, serial walk of reduced elements.
    out_ << "for (idx_t col = 0; col < " << s.row_len << "u; ++col) {\n";
    out_ << col_digits.str();
    // linear index of the full multi-index
    std::string lin;
    {
      int64_t stride = 1;
      for (int d = rank - 1; d >= 0; --d) {
        if (shape[d] != 1) {
          std::string term = stride == 1 ? "(" + root.multi[d] + ")" : "(" + root.multi[d] + ")*" + std::to_string(stride) + "u";
          lin = lin.empty() ? term : term + " + " + lin;
        }
        stride *= shape[d];
      }
      if (lin.empty()) lin = "0";
    }
    out_ << "const idx_t lin = " << lin << ";\n";
    out_ << elem_body;
    combine_elem(out_, 0);
    out_ << "}\n";
  }
  // Final: fold in the init values, evaluate the epilogue, store.
  Writer e(prog_, ptr_of, it);
  Idx oroot;
  oroot.key = "O";
  oroot.shape = kept_dims;
  oroot.lin = "row";
  const int oid = e.add_index(oroot);
  e.multi_of(oid);
  Idx sidx;
  sidx.key = "S";
  sidx.lin = "0";
  const int scal = e.add_index(sidx);
  std::ostringstream fin;
  for (size_t r = 0; r < accs.size(); ++r) {
    const Accum& a = accs[r];
    const ReduceSpec& rs = s.reduces[r];
    const bool am = a.kind == ReducerKind::kArgMax || a.kind == ReducerKind::kArgMin;
    std::string init0 = e.value(rs.inits[0], scal);
    if (am) {
      std::string init1 = e.value(rs.inits[1], scal);
      fin << "if (" << arg_better(a.kind) << "((float)" << init0 << ", (" << ait << ")" << init1 << ", " << a.v << ", " << a.i
          << ")) { " << a.v << " = " << init0 << "; " << a.i << " = (" << ait << ")" << init1 << "; }\n";
    } else {
      fin << combine_stmt(a.kind, a.vt, a.v, "(" + a.acc_t + ")(" + init0 + ")") << "\n";
    }
    // Seed the reduce results at the output index.
    const DType vt = a.vt;
    std::string rv = "fin" + std::to_string(r);
    if (a.kind == ReducerKind::kAnd || a.kind == ReducerKind::kOr) {
      fin << "const " << dtype_compute_ctype(vt) << " " << rv << " = (" << dtype_compute_ctype(vt) << ")" << a.v << ";\n";
    } else if (dtype_is_float(vt)) {
      fin << "const " << dtype_compute_ctype(vt) << " " << rv << " = " << round_to(vt, a.v) << ";\n";
    } else {
      fin << "const " << dtype_compute_ctype(vt) << " " << rv << " = (" << dtype_compute_ctype(vt) << ")" << a.v << ";\n";
    }
    e.seed(rs.results[0], oid, rv);
    if (am) {
      std::string ri = "fni" + std::to_string(r);
      fin << "const " << dtype_compute_ctype(a.it) << " " << ri << " = (" << dtype_compute_ctype(a.it) << ")" << a.i << ";\n";
      e.seed(rs.results[1], oid, ri);
    }
  }
  std::vector<std::string> outs;
  for (int v : s.outputs) outs.push_back(e.value(v, oid));
  std::ostringstream epi;
  epi << "{\n" << fin.str() << e.body.str();
  for (size_t o = 0; o < s.outputs.size(); ++o)
    epi << "out" << o << "[row] = " << to_storage(prog_.type(s.outputs[o]).dtype, outs[o]) << ";\n";
  epi << "}\n}\n\n";
  out_ << epi.str();
  if (epilogue_then_combine) {
    // The `_combine` kernel of the fallback (fused_mode 0): one wavefront per
    // row, lane k reads split k; the same epilogue.
    signature(s, &ptr_of, true, "_combine");
    out_ << "typedef " << it << " idx_t;\n";
    out_ << "const idx_t row = (idx_t)blockIdx.x * 4u + (threadIdx.x >> 6);\n";
    out_ << "if (row >= " << s.rows << "u) return;\n";
    out_ << "const uint32_t lane = threadIdx.x & 63u;\n";
    out_ << combine_fallback_body;
    out_ << epi.str();
  }
}

// Row-fused kernel: one workgroup (or one wave) per row. Each reduce phase
// walks the row, reduces across the workgroup, and every thread keeps the
// phase results as per-row scalars; the final elementwise phase writes the
// row outputs. When a thread's share of the row fits in registers
// (kRowCacheRegs 32-bit registers over all full-shape inputs) the whole share
// is loaded once, with every 16-byte load in flight together, and all phases
// read the registers; otherwise each phase streams the row again (the
// re-reads hit the cache).
constexpr int64_t kRowCacheRegs = 64;
constexpr int64_t kRowCacheSweeps = 16;

void KernelGen::row_fused(Step& s) {
  std::map<int, std::string> ptr_of;
  signature(s, &ptr_of, false);
  row_body(s, ptr_of, RowTarget());
  out_ << "}\n\n";
}

// The phases of a row-fused step for one row. By default the row is the
// workgroup's (or the wave's) and the outputs go to the kernel's `out`
// pointers; with `t.lds` the row is `t.row`, the block is one workgroup of
// 256 threads, and the final phase writes the row as float into the LDS
// array `t.lds` at t.row * row_len (a GEMV prologue).
void KernelGen::row_body(Step& s, std::map<int, std::string>& ptr_of, const RowTarget& t) {
  const std::string it = idx_type(s);
  out_ << "typedef " << it << " idx_t;\n";
  const Dims& shape = s.reduce_operand_shape;
  const int rank = static_cast<int>(shape.size());
  const int nred = static_cast<int>(s.reduce_dims.size());
  const int nkept = rank - nred;
  const int vec = s.vec;
  const int64_t row_len = s.row_len;
  const int64_t n_all = num_elements(shape);
  const bool wpr = s.wave_per_row && t.lds.empty();
  const int span = (wpr ? 64 : 256) * vec;     // elements per sweep of the row
  const std::string tix = wpr ? "(threadIdx.x & 63u)" : "threadIdx.x";
  if (!t.lds.empty()) {
    out_ << "const idx_t row = (idx_t)(" << t.row << ");\n";
  } else if (wpr) {
    out_ << "const idx_t row = (idx_t)blockIdx.x * 4u + (threadIdx.x >> 6);\n";
    out_ << "if (row >= " << s.rows << "u) return;\n";  // whole wave: no barriers follow
  } else {
    out_ << "const idx_t row = (idx_t)blockIdx.x;\n";
  }
  std::vector<std::string> multi(rank);
  {
    std::string rest = "row";
    for (int d = nkept - 1; d >= 0; --d) {
      if (d == 0) {
        multi[d] = rest;
      } else {
        out_ << "const idx_t kd" << d << " = " << rest << " % " << shape[d] << "u;\n";
        out_ << "const idx_t kq" << d << " = " << rest << " / " << shape[d] << "u;\n";
        multi[d] = "kd" + std::to_string(d);
        rest = "kq" + std::to_string(d);
      }
    }
  }
  std::ostringstream col_digits;
  {
    std::string rest = "col";
    for (int d = rank - 1; d >= nkept; --d) {
      if (d == nkept) {
        multi[d] = rest;
      } else {
        col_digits << "const idx_t rd" << d << " = " << rest << " % " << shape[d] << "u;\n";
        col_digits << "const idx_t rq" << d << " = " << rest << " / " << shape[d] << "u;\n";
        multi[d] = "rd" + std::to_string(d);
        rest = "rq" + std::to_string(d);
      }
    }
  }
  const Dims kept(shape.begin(), shape.begin() + nkept);
  std::map<int, std::string> scalars;
  // Register-resident share of the row: sweep k covers columns
  // tix*vec + k*span .. +vec (vec divides row_len, so a sweep that starts
  // inside the row is whole).
  const int64_t sweeps = (row_len + span - 1) / span;
  auto row_shaped = [&](int v) { return prog_.type(v).elements() == n_all && !t.lds_inputs.count(v); };
  int64_t cache_regs = 0;
  for (int v : s.inputs)
    if (row_shaped(v))
      cache_regs += sweeps * vec * static_cast<int64_t>(std::max<size_t>(dtype_size(prog_.type(v).dtype), 4)) / 4;
  const bool cached = sweeps <= kRowCacheSweeps && cache_regs <= kRowCacheRegs;
  const bool ragged = row_len % span != 0;
  auto sweep_open = [&](std::ostream& o) {
    if (cached) {
      o << "#pragma unroll\nfor (int k = 0; k < " << sweeps << "; ++k) {\n";
      o << "const idx_t c = " << tix << " * " << vec << "u + (idx_t)k * " << span << "u;\n";
      if (ragged) o << "if (c < " << row_len << "u) {\n";
    } else {
      o << "for (idx_t c = " << tix << " * " << vec << "u; c < " << row_len << "u; c += " << span << "u) {\n";
    }
  };
  auto sweep_close = [&](std::ostream& o) { o << ((cached && ragged) ? "}\n}\n" : "}\n"); };
  if (cached) {
    for (int v : s.inputs) {
      if (!row_shaped(v)) continue;
      const std::string st = dtype_storage_ctype(prog_.type(v).dtype);
      out_ << st << " pre_" << ptr_of[v] << "[" << sweeps << "][" << vec << "];\n";
    }
    sweep_open(out_);
    for (int v : s.inputs) {
      if (!row_shaped(v)) continue;
      const std::string st = dtype_storage_ctype(prog_.type(v).dtype);
      out_ << ldv_of(v, vec) << "(pre_" << ptr_of[v] << "[k], " << ptr_of[v] << ", row * " << row_len << "u + c, 0u, true);\n";
    }
    sweep_close(out_);
  }
  if (t.after_preload) t.after_preload();
  auto stage_hooks = [&](Writer& w) {
    for (auto& [v, name] : t.lds_inputs) {
      const DType dt = prog_.type(v).dtype;
      const std::string nm = name;
      w.lds_value[v] = [=](const std::string& lin) { return from_storage(dt, nm + "[" + lin + "]"); };
    }
  };
  auto preloads = [&](Writer& w, std::ostream& decl, std::ostream& load) {
    stage_hooks(w);
    for (int v : s.inputs) {
      if (!row_shaped(v)) continue;
      const std::string name = "pre_" + ptr_of[v];
      if (cached) {
        w.preload[v] = name + "[k]";
        continue;
      }
      const std::string st = dtype_storage_ctype(prog_.type(v).dtype);
      decl << st << " " << name << "[" << vec << "];\n";
      load << ldv_of(v, vec) << "(" << name << ", " << ptr_of[v] << ", row * " << row_len << "u + c, 0u, true);\n";
      w.preload[v] = name;
    }
  };
  int phase = 0;
  for (Step& ph : s.phases) {
    const std::string P = "p" + std::to_string(phase++);
    Writer w(prog_, ptr_of, it);
    w.row_scalar = scalars;
    Idx root;
    root.key = "R";
    root.shape = shape;
    root.lin = "lin";
    root.identity = true;
    root.multi = multi;
    const int rid = w.add_index(root);
    std::ostringstream pre_decl, pre_load;
    preloads(w, pre_decl, pre_load);
    if (ph.kind == StepKind::kReduce) {
      std::vector<Accum> accs;
      std::vector<std::string> xs;
      for (size_t r = 0; r < ph.reduces.size(); ++r) {
        const ReduceSpec& rs = ph.reduces[r];
        Accum a;
        a.kind = rs.kind;
        a.vt = prog_.type(rs.results[0]).dtype;
        a.acc_t = acc_ctype(rs.kind, a.vt);
        a.v = P + "_acc" + std::to_string(r);
        accs.push_back(a);
        xs.push_back(w.value(rs.inputs[0], rid));
      }
      const std::string body = w.body.str();
      for (auto& a : accs) {
        out_ << a.acc_t << " " << a.v << " = " << identity_of(a.kind, a.vt, a.acc_t) << ";\n";
        out_ << "__shared__ " << a.acc_t << " sm_" << a.v << "[4];\n";
      }
      sweep_open(out_);
      out_ << pre_decl.str() << pre_load.str();
      out_ << "#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) {\n";
      out_ << "const idx_t col = c + j;\nconst idx_t lin = row * " << row_len << "u + col;\n";
      out_ << col_digits.str() << body;
      for (size_t r = 0; r < accs.size(); ++r)
        out_ << combine_stmt(accs[r].kind, accs[r].vt, accs[r].v, "(" + accs[r].acc_t + ")(" + xs[r] + ")") << "\n";
      out_ << "}\n";
      sweep_close(out_);
      // Wavefront all-reduce (every lane ends with the same bits), then every
      // thread folds the 4 wave partials in wave order (deterministic).
      for (auto& a : accs) {
        const ReducerKind k = a.kind;
        const DType vt = a.vt;
        out_ << wave_allreduce(a.acc_t, a.v, [&](const std::string& x, const std::string& y) { return combine_stmt(k, vt, x, y); });
        if (!wpr) out_ << "if ((threadIdx.x & 63) == 0) sm_" << a.v << "[threadIdx.x >> 6] = " << a.v << ";\n";
      }
      if (!wpr) {
        out_ << "__syncthreads();\n";
        for (auto& a : accs) {
          out_ << a.v << " = sm_" << a.v << "[0];\n";
          out_ << "for (int k = 1; k < 4; ++k) { " << combine_stmt(a.kind, a.vt, a.v, "sm_" + a.v + "[k]") << " }\n";
        }
      }
      // Fold the init values, round, and evaluate this phase's outputs.
      Writer e(prog_, ptr_of, it);
      stage_hooks(e);
      e.row_scalar = scalars;
      Idx oroot;
      oroot.key = "O";
      oroot.shape = kept;
      oroot.lin = "row";
      oroot.multi.assign(multi.begin(), multi.begin() + nkept);
      const int oid = e.add_index(oroot);
      Idx sidx;
      sidx.key = "S";
      sidx.lin = "0";
      const int scal = e.add_index(sidx);
      std::ostringstream fin;
      for (size_t r = 0; r < accs.size(); ++r) {
        const Accum& a = accs[r];
        const ReduceSpec& rs = ph.reduces[r];
        fin << combine_stmt(a.kind, a.vt, a.v, "(" + a.acc_t + ")(" + e.value(rs.inits[0], scal) + ")") << "\n";
        const std::string rv = P + "_res" + std::to_string(r);
        const DType vt = a.vt;
        if (a.kind == ReducerKind::kAnd || a.kind == ReducerKind::kOr || !dtype_is_float(vt))
          fin << "const " << dtype_compute_ctype(vt) << " " << rv << " = (" << dtype_compute_ctype(vt) << ")" << a.v
              << ";\n";
        else
          fin << "const " << dtype_compute_ctype(vt) << " " << rv << " = " << round_to(vt, a.v) << ";\n";
        e.row_scalar[rs.results[0]] = rv;
      }
      std::vector<std::pair<int, std::string>> outs;
      for (int v : ph.outputs) outs.push_back({v, e.value(v, oid)});
      std::ostringstream decl, assign;
      for (auto& [v, expr] : outs) {
        const std::string name = P + "_v" + std::to_string(v);
        decl << dtype_compute_ctype(prog_.type(v).dtype) << " " << name << ";\n";
        assign << name << " = " << expr << ";\n";
        scalars[v] = name;
      }
      out_ << decl.str() << "{\n" << fin.str() << e.body.str() << assign.str() << "}\n";
      for (size_t o = 0; o < s.outputs.size() && t.lds.empty(); ++o)
        if (scalars.count(s.outputs[o]) && prog_.type(s.outputs[o]).dims == kept &&
            std::find(ph.outputs.begin(), ph.outputs.end(), s.outputs[o]) != ph.outputs.end())
          out_ << "if (" << tix << " == 0) out" << o << "[row] = "
               << to_storage(prog_.type(s.outputs[o]).dtype, scalars[s.outputs[o]]) << ";\n";
    } else {
      // Elementwise phase over the row.
      std::vector<std::pair<size_t, std::string>> outs;
      for (size_t o = 0; o < s.outputs.size(); ++o)
        if (std::find(ph.outputs.begin(), ph.outputs.end(), s.outputs[o]) != ph.outputs.end())
          outs.push_back({o, w.value(s.outputs[o], rid)});
      const std::string body = w.body.str();
      sweep_open(out_);
      out_ << pre_decl.str() << pre_load.str();
      for (auto& [o, expr] : outs)
        out_ << dtype_storage_ctype(prog_.type(s.outputs[o]).dtype) << " res" << o << "[" << vec << "];\n";
      out_ << "#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) {\n";
      out_ << "const idx_t col = c + j;\nconst idx_t lin = row * " << row_len << "u + col;\n";
      out_ << col_digits.str() << body;
      for (auto& [o, expr] : outs)
        out_ << "res" << o << "[j] = " << to_storage(prog_.type(s.outputs[o]).dtype, expr) << ";\n";
      out_ << "}\n";
      for (auto& [o, expr] : outs) {
        const DType ot = prog_.type(s.outputs[o]).dtype;
        if (!t.lds.empty()) {
          out_ << "#pragma unroll\nfor (int j = 0; j < " << vec << "; ++j) " << t.lds << "[row * " << row_len
               << "u + c + j] = " << from_storage(ot, "res" + std::to_string(o) + "[j]") << ";\n";
          continue;
        }
        out_ << "stv<" << dtype_storage_ctype(ot) << ", " << vec << ">(out" << o << ", row * " << row_len
             << "u + c, res" << o << ", 0u, true);\n";
      }
      sweep_close(out_);
    }
  }
}

// ----------------------------------------------------------------------------
// Decode GEMV (kGemv): Y_g[m][n] = sum_k X[m][k] * W_g[k][n] for the members
// g of the step, W_g [K][N_g] 16-bit with N contiguous, X [M][K].
//
// Work items: one item is `cols` columns of one member over one chunk of
// `kchunk` K rows; a segment (the unit whose partial sums are folded
// together) has wps items. Segment s belongs to XCD s % 8, and workgroup b
// runs on XCD b % 8 (the device places workgroups round-robin, probed at
// start-up; `fused_mode` says so): workgroup b takes items b / 8, b / 8 + P,
// b / 8 + 2P, ... of its XCD's list (P workgroups per XCD), segment by
// segment, so segments complete early and their folds overlap the streaming
// of later items; the next item's weight rows are loaded while the current
// one is reduced. Lanes take 16-byte pieces (8 columns) of a row, cols / 8
// lanes per row, so a wave reads 64 / (cols / 8) rows at once and each lane
// keeps `depth` rows in flight. X (or the prologue that produces it) is
// staged in LDS as float, whole or the one chunk a single-item workgroup
// needs. An item's column sums fold over the row lanes by xor shuffles and
// over the 4 waves in wave order.
//
// Unless an item is the whole result (direct: one K chunk, no epilogue), wave
// 0 stores the item's partial sums to scratch, waits until its L2 has them,
// and counts the segment's arrivals with an L2 atomic; the workgroup that
// completes a segment folds every partial in K-chunk order (reads past its
// L1), rounds to the result type, adds the residual, stores the results that
// are read elsewhere, keeps the segment's results in LDS, and evaluates the
// epilogue loop's elements of the segment from them. The fold order is fixed,
// so the result does not depend on which workgroup completes the segment.
// Without the XCD placement (fused_mode 0) agent-scope fences publish the
// partials instead.
void KernelGen::gemv(Step& s) {
  const GemvSpec& g = s.gemv;
  std::map<int, std::string> ptr_of;
  signature(s, &ptr_of, !g.direct);
  const int G = static_cast<int>(g.dots.size());
  const int M = g.M;
  const int64_t K = g.K;
  const int C = g.cols, LPR = C / 8, RPW = 64 / LPR, RS = 4 * RPW, D = g.depth;
  const int64_t iters = (g.kchunk + RS * D - 1) / (RS * D);
  const DType wt = prog_.type(prog_.ops[g.dots[0]].operands[1]).dtype;
  const bool f16 = wt == DType::kF16;
  const DType rt = prog_.type(g.result[0]).dtype;
  const bool pro = !s.prologue.empty();
  const bool all_x = g.stage_all_x;
  const int64_t XS = all_x ? K : g.kchunk;
  const int64_t S = g.seg_cols;
  const int64_t tps = S / C;
  const int64_t P = g.wgs / 8;  // workgroups per XCD
  std::vector<int64_t> N(G), tile0(G + 1, 0);
  for (int m = 0; m < G; ++m) {
    N[m] = prog_.type(g.result[m]).dims[1];
    tile0[m + 1] = tile0[m] + (N[m] + C - 1) / C;
  }
  auto out_of = [&](int v) {
    for (size_t o = 0; o < s.outputs.size(); ++o)
      if (s.outputs[o] == v) return "out" + std::to_string(o);
    return std::string();
  };
  auto by_member = [&](const std::string& gv, const std::function<std::string(int)>& f) {  // gv == 0 ? f(0) : ...
    std::string e = f(G - 1);
    for (int m = G - 2; m >= 0; --m) e = "(" + gv + " == " + std::to_string(m) + "u ? " + f(m) + " : " + e + ")";
    return e;
  };
  out_ << "typedef uint32_t idx_t;\n";
  out_ << "__shared__ float gv_xs[" << M * XS << "];\n";
  out_ << "__shared__ float gv_red[4][" << M << "][" << C << "];\n";
  if (g.joint) out_ << "__shared__ float gv_ys[" << G * M * S << "];\n";
  if (!g.direct) out_ << "__shared__ uint32_t gv_last;\n";
  out_ << "const uint32_t gv_lane = threadIdx.x & 63u, gv_wave = threadIdx.x >> 6;\n";
  out_ << "const uint32_t gv_x = blockIdx.x & 7u, gv_lb = blockIdx.x >> 3;\n";
  // items of this XCD: its segments x, x + 8, ... times wps
  out_ << "const uint32_t gv_nx = ((" << g.nseg << "u + 7u - gv_x) / 8u) * " << g.wps << "u;\n";
  out_ << "if (gv_lb >= gv_nx) return;\n";
  out_ << "const uint32_t gv_rg = gv_lane / " << LPR << "u, gv_cc = gv_lane % " << LPR << "u;\n";
  // The item being consumed (c_*) and the next one (n_*): plain registers
  // (a struct or a lambda taking pointers would put them on the stack and
  // turn the weight loads into flat loads).
  const char* fields[] = {"seg", "w", "g", "col0", "N", "k0", "k1", "r0"};
  for (const char* pre : {"c_", "n_"}) {
    out_ << "uint32_t";
    for (int f = 0; f < 8; ++f) out_ << (f ? ", " : " ") << pre << fields[f];
    out_ << ";\nconst uint16_t* " << pre << "W;\n";
  }
  auto assign_item = [&](const std::string& p, const std::string& it) {
    out_ << p << "seg = gv_x + 8u * ((" << it << ") / " << g.wps << "u);\n";
    out_ << p << "w = (" << it << ") % " << g.wps << "u;\n";
    out_ << "{\nconst uint32_t ks = " << p << "w % " << g.ksplit << "u;\n";
    if (g.joint) {
      out_ << "const uint32_t tg = " << p << "w / " << g.ksplit << "u;\n";
      out_ << p << "g = tg / " << tps << "u;\n";
      out_ << p << "col0 = " << p << "seg * " << S << "u + (tg % " << tps << "u) * " << C << "u;\n";
    } else {
      out_ << p << "g = 0u;\n";
      for (int m = 1; m < G; ++m) out_ << "if (" << p << "seg >= " << tile0[m] << "u) " << p << "g = " << m << "u;\n";
      out_ << p << "col0 = (" << p << "seg - " << by_member(p + "g", [&](int m) { return std::to_string(tile0[m]) + "u"; })
           << ") * " << C << "u;\n";
    }
    out_ << p << "N = " << by_member(p + "g", [&](int m) { return std::to_string(N[m]) + "u"; }) << ";\n";
    out_ << p << "W = " << by_member(p + "g", [&](int m) { return ptr_of.at(prog_.ops[g.dots[m]].operands[1]); })
         << ";\n";
    out_ << p << "k0 = ks * " << g.kchunk << "u;\n";
    out_ << p << "k1 = " << p << "k0 + " << g.kchunk << "u < " << K << "u ? " << p << "k0 + " << g.kchunk << "u : " << K
         << "u;\n";
    out_ << p << "r0 = " << p << "k0 + gv_wave * " << RPW << "u + gv_rg;\n}\n";
  };
  // Batch b of an item: rows r0 + (b * depth + i) * RS for i < depth. The
  // loads are unconditional (no branch between them, all in flight at once):
  // rows past the chunk read its last row and columns past N read the last
  // piece; the FMA loop skips those rows and the stores skip those columns.
  auto load_batch = [&](const std::string& p, const std::string& b, const std::string& dst) {
    out_ << "{\nconst uint32_t c0 = " << p << "col0 + gv_cc * 8u;\n";
    out_ << "const uint32_t c = c0 < " << p << "N ? c0 : " << p << "N - 8u;\n";
    out_ << "const uint16_t* wp = " << p << "W + c;\n";
    out_ << "#pragma unroll\nfor (int i = 0; i < " << D << "; ++i) {\n";
    out_ << "const uint32_t r = " << p << "r0 + ((" << b << ") * " << D << "u + (uint32_t)i) * " << RS << "u;\n";
    out_ << "const uint32_t rr = r < " << p << "k1 ? r : " << p << "k1 - 1u;\n";
    out_ << dst << "[i] = gv_load16<" << (g.weights_nt ? "true" : "false") << ">(wp + (size_t)rr * " << p << "N);\n";
    out_ << "}\n}\n";
  };
  assign_item("c_", "gv_lb");
  out_ << "gv_u32x4 gv_wv[" << D << "];\n";
  // X is requested before the first weight rows, so that the wait for X
  // (loads complete in order) does not include the weights.
  if (pro) {
    Step& Pst = s.prologue[0];
    RowTarget t;
    t.lds = "gv_xs";
    // The prologue's inputs (a few KB: the row and the norm weights) are
    // copied to LDS with 16-byte loads issued before the weight rows, so the
    // prologue never waits on a global load issued after them.
    int64_t staged_bytes = 0;
    bool stageable = true;
    for (int v : Pst.inputs) {
      staged_bytes += prog_.type(v).bytes();
      stageable &= prog_.type(v).bytes() % 16 == 0;
    }
    if (stageable && staged_bytes <= 32768) {
      int k = 0;
      std::vector<std::pair<int, int64_t>> pieces;  // value, 16-byte pieces
      for (int v : Pst.inputs) {
        const std::string name = "gv_pin" + std::to_string(k++);
        out_ << "__shared__ __attribute__((aligned(16))) " << dtype_storage_ctype(prog_.type(v).dtype) << " " << name
             << "[" << prog_.type(v).elements() << "];\n";
        t.lds_inputs[v] = name;
        pieces.push_back({v, prog_.type(v).bytes() / 16});
      }
      for (size_t q = 0; q < pieces.size(); ++q) {
        const int64_t per = (pieces[q].second + 255) / 256;
        out_ << "gv_u32x4 gv_pr" << q << "[" << per << "];\n";
        out_ << "#pragma unroll\nfor (int j = 0; j < " << per << "; ++j) {\n";
        out_ << "const uint32_t i = threadIdx.x + 256u * (uint32_t)j;\n";
        out_ << "if (i < " << pieces[q].second << "u) gv_pr" << q << "[j] = reinterpret_cast<const gv_u32x4*>("
             << ptr_of.at(pieces[q].first) << ")[i];\n}\n";
      }
      load_batch("c_", "0u", "gv_wv");
      for (size_t q = 0; q < pieces.size(); ++q) {
        const int64_t per = (pieces[q].second + 255) / 256;
        out_ << "#pragma unroll\nfor (int j = 0; j < " << per << "; ++j) {\n";
        out_ << "const uint32_t i = threadIdx.x + 256u * (uint32_t)j;\n";
        out_ << "if (i < " << pieces[q].second << "u) reinterpret_cast<gv_u32x4*>(" << t.lds_inputs[pieces[q].first]
             << ")[i] = gv_pr" << q << "[j];\n}\n";
      }
      out_ << "__syncthreads();\n";
      t.row = "gv_prow";
      out_ << "for (uint32_t gv_prow = 0; gv_prow < " << M << "u; ++gv_prow) {\n";
      row_body(Pst, ptr_of, t);
      out_ << "__syncthreads();\n}\n";
    } else if (M == 1) {
      t.row = "0u";
      t.after_preload = [&]() { load_batch("c_", "0u", "gv_wv"); };
      out_ << "{\n";
      row_body(Pst, ptr_of, t);
      out_ << "__syncthreads();\n}\n";
    } else {
      load_batch("c_", "0u", "gv_wv");
      t.row = "gv_prow";
      out_ << "for (uint32_t gv_prow = 0; gv_prow < " << M << "u; ++gv_prow) {\n";
      row_body(Pst, ptr_of, t);
      out_ << "__syncthreads();\n}\n";
    }
  } else {
    const std::string X = ptr_of.at(g.x);
    const int64_t nx = all_x ? M * K : M * g.kchunk;
    const int64_t per = (nx + 255) / 256;
    // X element i: read as is, or merged from a decode attention's split
    // partials (M == 1). A merged element's partials are requested before
    // the weight rows and folded after them when they fit in 96 registers a
    // lane; otherwise each element is merged before the weight rows are
    // requested.
    const std::string NS = std::to_string(g.attn_splits);
    const bool attn_late = g.attn_splits > 0 && per * g.attn_splits * 3 <= 96;
    auto x_elem = [&](const std::string& i) {
      if (g.attn_splits == 0) return load_expr(wt, X, i);
      return "gv_attn_merge<" + NS + ", " + std::to_string(g.attn_dim) + ", " + (f16 ? "true" : "false") +
             ">(reinterpret_cast<const float*>(" + X + "), " + i + ")";
    };
    const std::string valid = all_x ? "i < " + std::to_string(nx) + "u"
                                    : "i < " + std::to_string(nx) + "u && k < " + std::to_string(K) + "u";
    const std::string idx = all_x ? "i" : "m * " + std::to_string(K) + "u + k";
    out_ << "float gv_xr[" << per << "];\n";
    if (attn_late) out_ << "float gv_am[" << per << "][" << NS << "], gv_al[" << per << "][" << NS << "], gv_av[" << per
                        << "][" << NS << "];\n";
    out_ << "#pragma unroll\nfor (int j = 0; j < " << per << "; ++j) {\n";
    out_ << "const uint32_t i = threadIdx.x + 256u * (uint32_t)j;\n";
    if (!all_x) out_ << "const uint32_t m = i / " << g.kchunk << "u, k = c_k0 + i % " << g.kchunk << "u;\n";
    if (attn_late) {
      out_ << "if (" << valid << ") gv_attn_load<" << NS << ", " << g.attn_dim << ">(reinterpret_cast<const float*>(" << X
           << "), " << idx << ", gv_am[j], gv_al[j], gv_av[j]);\n";
    } else {
      out_ << "gv_xr[j] = (" << valid << ") ? " << x_elem(idx) << " : 0.0f;\n";
    }
    out_ << "}\n";
    load_batch("c_", "0u", "gv_wv");
    out_ << "#pragma unroll\nfor (int j = 0; j < " << per << "; ++j) {\n";
    out_ << "const uint32_t i = threadIdx.x + 256u * (uint32_t)j;\n";
    if (attn_late) {
      if (!all_x) out_ << "const uint32_t k = c_k0 + i % " << g.kchunk << "u;\n";
      out_ << "gv_xr[j] = (" << valid << ") ? gv_attn_fold<" << NS << ", " << (f16 ? "true" : "false")
           << ">(gv_am[j], gv_al[j], gv_av[j]) : 0.0f;\n";
    }
    out_ << "if (i < " << nx << "u) gv_xs[i] = gv_xr[j];\n}\n";
    out_ << "__syncthreads();\n";
  }
  out_ << "float gv_acc[" << M << "][8];\n";
  out_ << "#pragma unroll\nfor (int m = 0; m < " << M << "; ++m)\n#pragma unroll\nfor (int e = 0; e < 8; ++e) gv_acc[m][e] = 0.0f;\n";
  out_ << "uint32_t gv_it = gv_lb, gv_b = 0u;\n";
  out_ << "while (true) {\n";
  out_ << "uint32_t gv_nit = gv_it, gv_nb = gv_b + 1u;\n";
  out_ << "if (gv_nb == " << iters << "u) { gv_nit = gv_it + " << P << "u; gv_nb = 0u; }\n";
  out_ << "const bool gv_more = gv_nit < gv_nx;\n";
  out_ << "if (gv_more && gv_nb == 0u) {\n";
  assign_item("n_", "gv_nit");
  out_ << "} else {\n";
  for (const char* f : fields) out_ << "n_" << f << " = c_" << f << "; ";
  out_ << "n_W = c_W;\n}\n";
  out_ << "gv_u32x4 gv_nv[" << D << "];\n";
  out_ << "if (gv_more) ";
  load_batch("n_", "gv_nb", "gv_nv");
  out_ << "#pragma unroll\nfor (int i = 0; i < " << D << "; ++i) {\n";
  out_ << "const uint32_t r = c_r0 + (gv_b * " << D << "u + (uint32_t)i) * " << RS << "u;\n";
  out_ << "if (r < c_k1) {\n";
  out_ << "#pragma unroll\nfor (int m = 0; m < " << M << "; ++m) gv_fma8<" << (f16 ? "true" : "false")
       << ">(gv_acc[m], gv_xs[m * " << XS << "u + r" << (all_x ? "" : " - c_k0") << "], gv_wv[i]);\n";
  out_ << "}\n}\n";
  out_ << "if (gv_b + 1u == " << iters << "u) {\n";
  // ---- item done: fold the row lanes (xor over the row-group bits), then the waves
  out_ << "#pragma unroll\nfor (int m = 0; m < " << M << "; ++m)\n#pragma unroll\nfor (int e = 0; e < 8; ++e) {\n";
  out_ << "float v = gv_acc[m][e];\n";
  for (int sh = LPR; sh < 64; sh <<= 1) out_ << "v += wave_shfl_xor(v, " << sh << ");\n";
  out_ << "gv_acc[m][e] = 0.0f;\n";
  out_ << "if (gv_rg == 0u) gv_red[gv_wave][m][gv_cc * 8u + e] = v;\n}\n";
  out_ << "__syncthreads();\n";
  auto member_value = [&](const std::string& m_expr, const std::string& col, const std::string& sum, int m) {
    // rounded product, plus the residual when the member has one
    std::string y = round_to(rt, sum);
    if (g.add[m] >= 0) {
      const std::string a = load_expr(rt, ptr_of.at(g.add[m]), m_expr + " * " + std::to_string(N[m]) + "u + " + col);
      y = round_to(rt, a + " + " + y);
    }
    return y;
  };
  auto ld = [&](const std::string& addr) {
    return "__hip_atomic_load(&" + addr + ", __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)";
  };
  if (g.direct) {
    out_ << "for (uint32_t i = threadIdx.x; i < " << M * C << "u; i += 256u) {\n";
    out_ << "const uint32_t m = i / " << C << "u, c = i % " << C << "u, col = c_col0 + c;\n";
    out_ << "if (col < c_N) {\n";
    out_ << "const float p = ((gv_red[0][m][c] + gv_red[1][m][c]) + gv_red[2][m][c]) + gv_red[3][m][c];\n";
    for (int m = 0; m < G; ++m) {
      out_ << "if (c_g == " << m << "u) { const float y = " << member_value("m", "col", "p", m) << "; "
           << out_of(g.result[m]) << "[m * " << N[m] << "u + col] = " << to_storage(rt, "y") << "; }\n";
    }
    out_ << "}\n}\n";
    out_ << "__syncthreads();\n";  // gv_red is rewritten by the next item
  } else {
    out_ << "float* gv_part = reinterpret_cast<float*>(scratch);\n";
    out_ << "if (gv_wave == 0u) {\n";
    out_ << "for (uint32_t i = gv_lane; i < " << M * C << "u; i += 64u) {\n";
    out_ << "const uint32_t m = i / " << C << "u, c = i % " << C << "u;\n";
    out_ << "gv_part[((size_t)(c_seg * " << g.wps << "u + c_w) * " << M << "u + m) * " << C
         << "u + c] = ((gv_red[0][m][c] + gv_red[1][m][c]) + gv_red[2][m][c]) + gv_red[3][m][c];\n";
    out_ << "}\n";
    // Release fence at workgroup scope: a compiler barrier between the
    // partial stores and the counter RMW (no cache write-back); s_waitcnt(0)
    // has the stores acknowledged by the XCD's L2 first.
    out_ << "__builtin_amdgcn_fence(__ATOMIC_RELEASE, \"workgroup\");\n";
    out_ << "__builtin_amdgcn_s_waitcnt(0);\n";
    out_ << "if (!fused_mode) __threadfence();\n";
    out_ << "if (gv_lane == 0u) {\n";
    // one counter per 128-byte line
    out_ << "uint32_t* ctr = reinterpret_cast<uint32_t*>(scratch + " << s.counter_offset << "u) + c_seg * 32u;\n";
    out_ << "const uint32_t last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == "
         << g.wps - 1 << "u;\n";
    out_ << "if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n";
    out_ << "gv_last = last;\n}\n}\n";
    out_ << "__syncthreads();\n";
    out_ << "if (gv_last) {\n";
    out_ << "__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, \"workgroup\");\n";
    out_ << "if (!fused_mode) __threadfence();\n";
    if (g.joint) {
      // Up to Q passes of 256 threads over the segment's elements. When the
      // partials of every pass fit in registers, all of them are requested
      // first (one L2 round trip instead of one per pass), then summed in
      // the same K-chunk order.
      const int64_t n_el = G * M * S, Q = (n_el + 255) / 256;
      const bool batched = Q > 1 && Q * g.ksplit <= 64;
      const std::string decode = "const uint32_t gv_g = i / " + std::to_string(M * S) + "u, rem = i % " +
                                 std::to_string(M * S) + "u;\nconst uint32_t m = rem / " + std::to_string(S) +
                                 "u, c = rem % " + std::to_string(S) + "u;\nconst size_t base = (size_t)c_seg * " +
                                 std::to_string(g.wps) + "u + ((size_t)gv_g * " + std::to_string(tps) + "u + c / " +
                                 std::to_string(C) + "u) * " + std::to_string(g.ksplit) + "u;\n";
      const std::string part = ld("gv_part[((base + k) * " + std::to_string(M) + "u + m) * " + std::to_string(C) +
                                  "u + c % " + std::to_string(C) + "u]");
      if (batched) {
        out_ << "float gv_pv[" << Q << "][" << g.ksplit << "];\n";
        out_ << "#pragma unroll\nfor (int q = 0; q < " << Q << "; ++q) {\n";
        out_ << "const uint32_t i = threadIdx.x + 256u * (uint32_t)q;\n";
        out_ << "if (i < " << n_el << "u) {\n" << decode;
        out_ << "#pragma unroll\nfor (uint32_t k = 0; k < " << g.ksplit << "u; ++k) gv_pv[q][k] = " << part << ";\n";
        out_ << "}\n}\n";
        out_ << "#pragma unroll\nfor (int q = 0; q < " << Q << "; ++q) {\n";
        out_ << "const uint32_t i = threadIdx.x + 256u * (uint32_t)q;\n";
        out_ << "if (i >= " << n_el << "u) continue;\n" << decode;
        out_ << "float sum = 0.0f;\n";
        out_ << "#pragma unroll\nfor (uint32_t k = 0; k < " << g.ksplit << "u; ++k) sum += gv_pv[q][k];\n";
      } else {
        out_ << "for (uint32_t i = threadIdx.x; i < " << n_el << "u; i += 256u) {\n" << decode;
        out_ << "float sum = 0.0f;\n";
        out_ << "#pragma unroll\nfor (uint32_t k = 0; k < " << g.ksplit << "u; ++k) sum += " << part << ";\n";
      }
      out_ << "const uint32_t col = c_seg * " << S << "u + c;\n";
      out_ << "float y = 0.0f;\n";
      for (int m = 0; m < G; ++m) {
        out_ << "if (gv_g == " << m << "u) {\n";
        out_ << "y = " << member_value("m", "col", "sum", m) << ";\n";
        if (g.store[m]) out_ << out_of(g.result[m]) << "[m * " << N[m] << "u + col] = " << to_storage(rt, "y") << ";\n";
        out_ << "}\n";
      }
      out_ << "gv_ys[i] = y;\n";
      out_ << "}\n";
    } else {
      out_ << "for (uint32_t i = threadIdx.x; i < " << M * C << "u; i += 256u) {\n";
      out_ << "const uint32_t m = i / " << C << "u, c = i % " << C << "u, col = c_col0 + c;\n";
      out_ << "if (col < c_N) {\n";
      out_ << "const size_t base = (size_t)c_seg * " << g.wps << "u;\n";
      out_ << "float sum = 0.0f;\n";
      out_ << "#pragma unroll\nfor (uint32_t k = 0; k < " << g.ksplit << "u; ++k) sum += "
           << ld("gv_part[((base + k) * " + std::to_string(M) + "u + m) * " + std::to_string(C) + "u + c]") << ";\n";
      for (int m = 0; m < G; ++m) {
        out_ << "if (c_g == " << m << "u) { const float y = " << member_value("m", "col", "sum", m) << "; "
             << out_of(g.result[m]) << "[m * " << N[m] << "u + col] = " << to_storage(rt, "y") << "; }\n";
      }
      out_ << "}\n}\n";
    }
    if (!s.epilogue_loop.empty()) {
      out_ << "__syncthreads();\n";
      gemv_epilogue(s, ptr_of, "c_seg");
    }
    out_ << "}\n";  // gv_last
  }
  out_ << "}\n";  // item done
  out_ << "if (!gv_more) break;\n";
  out_ << "gv_it = gv_nit; gv_b = gv_nb;\n";
  for (const char* f : fields) out_ << "c_" << f << " = n_" << f << "; ";
  out_ << "c_W = n_W;\n";
  out_ << "#pragma unroll\nfor (int i = 0; i < " << D << "; ++i) gv_wv[i] = gv_nv[i];\n";
  out_ << "}\n";
  out_ << "}\n\n";
}

// The epilogue loop of a kGemv step over segment `seg`'s root elements
// [seg * R, (seg + 1) * R), one element per thread and pass. Reads of the
// step's results come from the segment's LDS copy (the planner checked that
// they stay inside the segment's columns); its outputs are the step's
// outputs after the stored results, window outputs written in place.
void KernelGen::gemv_epilogue(Step& s, const std::map<int, std::string>& ptr_of, const std::string& seg) {
  const GemvSpec& g = s.gemv;
  Step& L = s.epilogue_loop[0];
  const int G = static_cast<int>(g.dots.size());
  const int64_t S = g.seg_cols, R = g.root_per_seg;
  const int M = g.M;
  size_t base = 0;
  for (int m = 0; m < G; ++m) base += g.store[m] ? 1 : 0;
  out_ << "{\n";
  Writer w(prog_, ptr_of, "uint32_t");
  for (int m = 0; m < G; ++m) {
    const int64_t N = prog_.type(g.result[m]).dims[1];
    const std::string off = std::to_string(static_cast<int64_t>(m) * M * S);
    w.lds_value[g.result[m]] = [=](const std::string& lin) {
      if (M == 1) return "gv_ys[" + off + "u + (" + lin + ") - " + seg + " * " + std::to_string(S) + "u]";
      return "gv_ys[" + off + "u + ((" + lin + ") / " + std::to_string(N) + "u) * " + std::to_string(S) + "u + (" + lin +
             ") % " + std::to_string(N) + "u - " + seg + " * " + std::to_string(S) + "u]";
    };
  }
  Idx root;
  root.key = "R";
  root.shape = L.loop_shape;
  root.lin = "lin";
  root.identity = true;
  const int rid = w.add_index(root);
  std::vector<std::string> vals;
  for (size_t o = 0; o < L.outputs.size(); ++o) {
    auto ww = L.window_out.find(static_cast<int>(o));
    vals.push_back(w.value(ww == L.window_out.end() ? L.outputs[o] : ww->second.update, rid));
  }
  for (auto& [o, ww] : L.window_out) {
    const Dims& od = prog_.type(ww.operand).dims;
    for (size_t d = 0; d < ww.starts.size(); ++d) {
      const int sv = ww.starts[d];
      std::string e;
      auto pi = ptr_of.find(sv);
      if (pi != ptr_of.end()) {
        e = "(int64_t)" + pi->second + "[0]";
      } else {
        const Op* c = nullptr;
        for (const Op& op : prog_.ops)
          if (!op.results.empty() && op.results[0] == sv) c = &op;
        PJRTX_CHECK(c && c->kind == OpKind::kConstant, Code::kInternal, "window start is neither an input nor a constant");
        e = "(int64_t)(" + literal_expr(prog_, *c, 0) + ")";
      }
      const int64_t hi = od[d] - L.loop_shape[d];
      out_ << "int64_t ws" << o << "_" << d << " = " << e << ";\n";
      out_ << "ws" << o << "_" << d << " = ws" << o << "_" << d << " < 0 ? 0 : (ws" << o << "_" << d << " > " << hi
           << " ? " << hi << " : ws" << o << "_" << d << ");\n";
    }
  }
  out_ << "for (uint32_t lin = " << seg << " * " << R << "u + threadIdx.x; lin < (" << seg << " + 1u) * " << R
       << "u; lin += 256u) {\n";
  out_ << w.body.str();
  for (size_t o = 0; o < L.outputs.size(); ++o) {
    const DType t = prog_.type(L.outputs[o]).dtype;
    const std::string outp = "out" + std::to_string(base + o);
    auto ww = L.window_out.find(static_cast<int>(o));
    if (ww == L.window_out.end()) {
      out_ << outp << "[lin] = " << to_storage(t, vals[o]) << ";\n";
      continue;
    }
    const Dims& od = prog_.type(ww->second.operand).dims;
    out_ << "{ uint64_t rem = lin, dst = 0;\n";
    int64_t stride = 1;
    for (int d = static_cast<int>(od.size()) - 1; d >= 0; --d) {
      out_ << "{ const uint64_t c = rem % " << L.loop_shape[d] << "u; rem /= " << L.loop_shape[d]
           << "u; dst += (c + (uint64_t)ws" << o << "_" << d << ") * " << stride << "ull; }\n";
      stride *= od[d];
    }
    out_ << outp << "[dst] = " << to_storage(t, vals[o]) << "; }\n";
  }
  out_ << "}\n}\n";
}

}  // namespace

std::string generate_kernels(const Program& prog, Plan& plan) {
  std::ostringstream out;
  KernelGen gen(prog, out, plan.nt_min_bytes);
  for (Step& s : plan.steps) {
    if (s.kind == StepKind::kLoop) gen.loop(s);
    else if (s.kind == StepKind::kReduce) gen.reduce(s);
    else if (s.kind == StepKind::kRowFused) gen.row_fused(s);
    else if (s.kind == StepKind::kGemv) gen.gemv(s);
  }
  return out.str();
}

}  // namespace pjrtx
