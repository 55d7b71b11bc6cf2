// Custom-call target registry and the lowering of registered targets.
// Reference: src/backend/mlx_metal/custom_call.zig (registry, op names,
// built-ins) and lowering_custom_call.zig:17-215 (legality).
#include "custom_call.h"

#include <map>
#include <mutex>
#include <utility>

#include "common.h"

namespace pjrtx {

namespace {

// Op names accepted by the registration calls (reference:
// custom_call.zig:63-102, parseBinaryOp / parseUnaryOp).
const std::map<std::string, OpKind>& binary_ops() {
  static const std::map<std::string, OpKind> m = {
      {"add", OpKind::kAdd},
      {"subtract", OpKind::kSubtract},
      {"multiply", OpKind::kMultiply},
      {"divide", OpKind::kDivide},
      {"maximum", OpKind::kMaximum},
      {"minimum", OpKind::kMinimum},
      {"power", OpKind::kPower},
      {"atan2", OpKind::kAtan2},
      {"remainder", OpKind::kRemainder},
      {"and", OpKind::kAnd},
      {"or", OpKind::kOr},
      {"xor", OpKind::kXor},
      {"shift_left", OpKind::kShiftLeft},
      {"shift_right_logical", OpKind::kShiftRightLogical},
      {"shift_right_arithmetic", OpKind::kShiftRightArithmetic},
  };
  return m;
}

const std::map<std::string, OpKind>& unary_ops() {
  static const std::map<std::string, OpKind> m = {
      {"negate", OpKind::kNegate},
      {"exp", OpKind::kExp},
      {"expm1", OpKind::kExpm1},
      {"tanh", OpKind::kTanh},
      {"sqrt", OpKind::kSqrt},
      {"rsqrt", OpKind::kRsqrt},
      {"abs", OpKind::kAbs},
      {"cbrt", OpKind::kCbrt},
      {"ceil", OpKind::kCeil},
      {"floor", OpKind::kFloor},
      {"log", OpKind::kLog},
      {"log1p", OpKind::kLog1p},
      {"logistic", OpKind::kLogistic},
      {"sine", OpKind::kSine},
      {"cosine", OpKind::kCosine},
      {"not", OpKind::kNot},
      {"sign", OpKind::kSign},
      {"is_finite", OpKind::kIsFinite},
      {"round_nearest_afz", OpKind::kRoundAfz},
      {"round_nearest_even", OpKind::kRoundEven},
      {"popcnt", OpKind::kPopcnt},
      {"count_leading_zeros", OpKind::kClz},
  };
  return m;
}

std::string op_name_of(OpKind k) {
  for (const auto* m : {&binary_ops(), &unary_ops()})
    for (const auto& [name, op] : *m)
      if (op == k) return name;
  return "?";
}

struct Registry {
  std::mutex mu;
  std::map<std::string, CustomCallSpec> targets;
  uint64_t version = 0;
};

Registry& registry() {
  static Registry r;
  return r;
}

void put(const std::string& target, const CustomCallSpec& spec) {
  PJRTX_CHECK(!target.empty(), Code::kInvalidArgument, "custom call target is empty");
  Registry& r = registry();
  std::lock_guard<std::mutex> lk(r.mu);
  r.targets[target] = spec;
  ++r.version;
}

bool is_int(DType t) { return (dtype_is_signed_int(t) || dtype_is_unsigned_int(t)) && t != DType::kPred; }

}  // namespace

void register_custom_call_identity(const std::string& target) {
  CustomCallSpec s;
  s.kind = CustomCallKind::kIdentity;
  put(target, s);
}

void register_custom_call_unary(const std::string& target, const std::string& op_name) {
  auto it = unary_ops().find(op_name);
  PJRTX_CHECK(it != unary_ops().end(), Code::kInvalidArgument, "custom call unary op '" + op_name + "' is not known");
  CustomCallSpec s;
  s.kind = CustomCallKind::kUnary;
  s.op = it->second;
  put(target, s);
}

void register_custom_call_binary(const std::string& target, const std::string& op_name) {
  auto it = binary_ops().find(op_name);
  PJRTX_CHECK(it != binary_ops().end(), Code::kInvalidArgument, "custom call binary op '" + op_name + "' is not known");
  CustomCallSpec s;
  s.kind = CustomCallKind::kBinary;
  s.op = it->second;
  put(target, s);
}

void unregister_custom_call(const std::string& target) {
  Registry& r = registry();
  std::lock_guard<std::mutex> lk(r.mu);
  if (r.targets.erase(target)) ++r.version;
}

bool lookup_custom_call(const std::string& target, CustomCallSpec* spec) {
  // Built-ins (reference: custom_call.zig:222-229).
  if (target == "annotate_device_placement") {
    *spec = CustomCallSpec{CustomCallKind::kIdentity, OpKind::kParameter, false};
    return true;
  }
  if (target == "pjrtx.mlx_metal.custom_binary_add_f32") {
    *spec = CustomCallSpec{CustomCallKind::kBinary, OpKind::kAdd, true};
    return true;
  }
  Registry& r = registry();
  std::lock_guard<std::mutex> lk(r.mu);
  auto it = r.targets.find(target);
  if (it == r.targets.end()) return false;
  *spec = it->second;
  return true;
}

uint64_t custom_call_registry_version() {
  Registry& r = registry();
  std::lock_guard<std::mutex> lk(r.mu);
  return r.version;
}

void lower_registered_custom_call(const Program& prog, Op* op) {
  const std::string& target = op->target;
  CustomCallSpec spec;
  PJRTX_CHECK(lookup_custom_call(target, &spec), Code::kUnimplemented,
              "custom_call target '" + target + "' has no registered pjrtx implementation");
  const size_t nin = spec.kind == CustomCallKind::kBinary ? 2 : 1;
  const char* what = spec.kind == CustomCallKind::kIdentity ? "identity" : spec.kind == CustomCallKind::kUnary ? "unary" : "binary";
  PJRTX_CHECK(op->operands.size() == nin && op->results.size() == 1, Code::kInvalidArgument,
              std::string(what) + " custom_call '" + target + "' requires exactly " + (nin == 2 ? "two inputs" : "one input") +
                  " and one output");
  const TensorType& in = prog.type(op->operands[0]);
  const TensorType& out = prog.type(op->results[0]);
  PJRTX_CHECK(in.dims == out.dims, Code::kInvalidArgument,
              std::string(what) + " custom_call '" + target + "' requires matching input/output shapes");
  const DType t = in.dtype;
  auto need = [&](bool ok, const std::string& msg) {
    PJRTX_CHECK(ok, Code::kInvalidArgument, "custom_call '" + target + "': " + msg);
  };
  switch (spec.kind) {
    case CustomCallKind::kIdentity:
      need(out.dtype == t, "identity output must match input dtype and shape");
      op->kind = OpKind::kReshape;
      op->name = "stablehlo.reshape";
      break;
    case CustomCallKind::kUnary:
      switch (spec.op) {
        case OpKind::kIsFinite:
          need(dtype_is_float(t) && out.dtype == DType::kPred, "is_finite requires a floating input and a pred output");
          break;
        case OpKind::kNot:
          need((is_int(t) || t == DType::kPred) && out.dtype == t, "not requires a pred or integer dtype");
          break;
        case OpKind::kPopcnt:
        case OpKind::kClz:
          need(is_int(t) && out.dtype == t, op_name_of(spec.op) + " requires a matching integer dtype");
          break;
        case OpKind::kAbs:
        case OpKind::kNegate:
        case OpKind::kSign:
          need((dtype_is_float(t) || is_int(t)) && out.dtype == t, op_name_of(spec.op) + " requires a matching numeric dtype");
          break;
        default:  // exp, sqrt, the roundings, ...
          need(dtype_is_float(t) && out.dtype == t, op_name_of(spec.op) + " requires a matching floating dtype");
          break;
      }
      op->kind = spec.op;
      op->name = std::string("stablehlo.") + op_kind_name(spec.op);
      break;
    case CustomCallKind::kBinary: {
      const TensorType& rhs = prog.type(op->operands[1]);
      need(rhs.dtype == t && out.dtype == t && rhs.dims == in.dims,
           "binary custom_call requires matching input/output dtypes and shapes");
      if (spec.f32_only) need(t == DType::kF32, "the built-in binary add requires f32 tensors");
      switch (spec.op) {
        case OpKind::kAtan2:
          need(dtype_is_float(t), "atan2 requires a floating dtype");
          break;
        case OpKind::kAnd:
        case OpKind::kOr:
        case OpKind::kXor:
          need(is_int(t) || t == DType::kPred, "logical/bitwise ops require a pred or integer dtype");
          break;
        case OpKind::kShiftLeft:
        case OpKind::kShiftRightLogical:
        case OpKind::kShiftRightArithmetic:
          need(is_int(t), "shifts require an integer dtype");
          break;
        default:
          need(dtype_is_float(t) || is_int(t), op_name_of(spec.op) + " requires a numeric dtype");
          break;
      }
      op->kind = spec.op;
      op->name = std::string("stablehlo.") + op_kind_name(spec.op);
      break;
    }
  }
  op->target.clear();
}

}  // namespace pjrtx
