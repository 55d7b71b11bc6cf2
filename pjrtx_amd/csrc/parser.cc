// StableHLO text importer: MLIR text -> Program.
//
// Replaces the reference's ingestion path (reference:
// src/compiler/stablehlo_import.zig:81-110 analyzeProgramFromReader,
// src/compiler/mlir_session.zig:250-262 VHLO deserialization and :206-234
// inline/canonicalize, src/compiler/plan_instruction.zig:10-93 op walk).
// There is no MLIR library on this host, so the importer reads the textual
// form JAX prints for `jax.jit(f).lower(...).as_text()`: pretty stablehlo ops,
// the generic `"stablehlo.op"(...) <{...}> ({...}) : (...) -> ...` form, and
// `func.func` / `call` / `return`. Private functions are inlined into @main.
#include <cmath>
#include <cstring>
#include <functional>
#include <set>
#include <unordered_map>

#include "ir.h"

namespace pjrtx {

// ----------------------------------------------------------------------------
// Float format helpers (host side).

uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return static_cast<uint16_t>(u >> 16);
}

float bf16_bits_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) return static_cast<uint16_t>(sign | 0x7c00u | (man ? 0x200u : 0u));
  int32_t e = static_cast<int32_t>(exp) - 127 + 15;
  if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return static_cast<uint16_t>(sign);
    man |= 0x800000u;
    uint32_t shift = static_cast<uint32_t>(14 - e);
    uint32_t half = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) half++;
    return static_cast<uint16_t>(sign | half);
  }
  uint32_t half = sign | (static_cast<uint32_t>(e) << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
  return static_cast<uint16_t>(half);
}

float f16_bits_to_f32(uint16_t h) {
  uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t out;
  if (exp == 0) {
    if (man == 0) {
      out = sign;
    } else {
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      out = sign | (static_cast<uint32_t>(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (man << 13);
  } else {
    out = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &out, 4);
  return f;
}

// ----------------------------------------------------------------------------
// Op table.

namespace {

struct OpInfo {
  const char* mnemonic;
  OpKind kind;
};

const OpInfo kOpTable[] = {
    {"constant", OpKind::kConstant},
    {"abs", OpKind::kAbs},
    {"negate", OpKind::kNegate},
    {"exponential", OpKind::kExp},
    {"exponential_minus_one", OpKind::kExpm1},
    {"log", OpKind::kLog},
    {"log_plus_one", OpKind::kLog1p},
    {"logistic", OpKind::kLogistic},
    {"sqrt", OpKind::kSqrt},
    {"rsqrt", OpKind::kRsqrt},
    {"cbrt", OpKind::kCbrt},
    {"tanh", OpKind::kTanh},
    {"sine", OpKind::kSine},
    {"cosine", OpKind::kCosine},
    {"tan", OpKind::kTan},
    {"floor", OpKind::kFloor},
    {"ceil", OpKind::kCeil},
    {"round_nearest_afz", OpKind::kRoundAfz},
    {"round_nearest_even", OpKind::kRoundEven},
    {"sign", OpKind::kSign},
    {"not", OpKind::kNot},
    {"is_finite", OpKind::kIsFinite},
    {"popcnt", OpKind::kPopcnt},
    {"count_leading_zeros", OpKind::kClz},
    {"convert", OpKind::kConvert},
    {"bitcast_convert", OpKind::kBitcastConvert},
    {"reduce_precision", OpKind::kReducePrecision},
    {"add", OpKind::kAdd},
    {"subtract", OpKind::kSubtract},
    {"multiply", OpKind::kMultiply},
    {"divide", OpKind::kDivide},
    {"remainder", OpKind::kRemainder},
    {"power", OpKind::kPower},
    {"maximum", OpKind::kMaximum},
    {"minimum", OpKind::kMinimum},
    {"and", OpKind::kAnd},
    {"or", OpKind::kOr},
    {"xor", OpKind::kXor},
    {"shift_left", OpKind::kShiftLeft},
    {"shift_right_arithmetic", OpKind::kShiftRightArithmetic},
    {"shift_right_logical", OpKind::kShiftRightLogical},
    {"atan2", OpKind::kAtan2},
    {"compare", OpKind::kCompare},
    {"select", OpKind::kSelect},
    {"clamp", OpKind::kClamp},
    {"broadcast_in_dim", OpKind::kBroadcastInDim},
    {"reshape", OpKind::kReshape},
    {"transpose", OpKind::kTranspose},
    {"slice", OpKind::kSlice},
    {"iota", OpKind::kIota},
    {"reverse", OpKind::kReverse},
    {"concatenate", OpKind::kConcatenate},
    {"pad", OpKind::kPad},
    {"dynamic_slice", OpKind::kDynamicSlice},
    {"dynamic_update_slice", OpKind::kDynamicUpdateSlice},
    {"reduce", OpKind::kReduce},
    {"reduce_window", OpKind::kReduceWindow},
    {"dot_general", OpKind::kDotGeneral},
    {"dot", OpKind::kDotGeneral},
    {"gather", OpKind::kGather},
    {"scatter", OpKind::kScatter},
    {"while", OpKind::kWhile},
    {"sort", OpKind::kSort},
    {"top_k", OpKind::kTopK},
    {"custom_call", OpKind::kCustomCall},
    {"pjrtx.attention", OpKind::kAttention},
    {"return", OpKind::kReturn},
};

bool lookup_op(const std::string& mnemonic, OpKind* out) {
  for (const OpInfo& info : kOpTable) {
    if (mnemonic == info.mnemonic) {
      *out = info.kind;
      return true;
    }
  }
  return false;
}

}  // namespace

const char* op_kind_name(OpKind k) {
  if (k == OpKind::kParameter) return "parameter";
  for (const OpInfo& info : kOpTable) {
    if (info.kind == k) return info.mnemonic;
  }
  return "?";
}

bool op_is_elementwise(OpKind k) {
  return (k >= OpKind::kAbs && k <= OpKind::kClamp);
}

bool op_is_view(OpKind k) {
  return k == OpKind::kBroadcastInDim || k == OpKind::kReshape || k == OpKind::kTranspose ||
         k == OpKind::kSlice || k == OpKind::kIota || k == OpKind::kReverse;
}

std::string Program::describe() const {
  std::string s;
  for (const Op& op : ops) {
    for (size_t i = 0; i < op.results.size(); ++i) {
      s += (i ? ", %" : "%") + std::to_string(op.results[i]);
    }
    s += std::string(op.results.empty() ? "" : " = ") + op_kind_name(op.kind) + "(";
    for (size_t i = 0; i < op.operands.size(); ++i) {
      s += (i ? ", %" : "%") + std::to_string(op.operands[i]);
    }
    s += ")";
    if (!op.results.empty()) s += " : " + type(op.results[0]).str();
    s += "\n";
  }
  return s;
}

// ----------------------------------------------------------------------------
// Parser.

namespace {

// A function as written in the text, before inlining.
struct RawFunc {
  std::string name;
  std::vector<int> params;
  std::vector<int> param_alias;  // see Program::param_alias
  std::vector<TensorType> result_types;
  std::vector<Op> ops;  // includes call ops as kind kReturn+callee marker
};

struct CallMarker {
  std::string callee;
};

class Parser {
 public:
  explicit Parser(const std::string& text) : s_(text) {}

  Program run();

 private:
  // ---- low level cursor helpers ----
  const std::string& s_;
  size_t p_ = 0;

  [[noreturn]] void error(const std::string& msg, Code code = Code::kInvalidArgument) {
    size_t line = 1;
    for (size_t i = 0; i < p_ && i < s_.size(); ++i) line += s_[i] == '\n';
    size_t ls = s_.rfind('\n', p_ == 0 ? 0 : p_ - 1);
    ls = (ls == std::string::npos) ? 0 : ls + 1;
    size_t le = s_.find('\n', p_);
    std::string context = s_.substr(ls, (le == std::string::npos ? s_.size() : le) - ls);
    if (context.size() > 200) context = context.substr(0, 200) + "...";
    fail(code, strformat("stablehlo parse error at line %zu: %s\n  | %s", line, msg.c_str(),
                         context.c_str()));
  }

  void ws() {
    while (p_ < s_.size()) {
      char c = s_[p_];
      if (c == ' ' || c == '\t' || c == '\n' || c == '\r') {
        ++p_;
      } else if (c == '/' && p_ + 1 < s_.size() && s_[p_ + 1] == '/') {
        while (p_ < s_.size() && s_[p_] != '\n') ++p_;
      } else {
        break;
      }
    }
  }
  bool eof() {
    ws();
    return p_ >= s_.size();
  }
  char peek() {
    ws();
    return p_ < s_.size() ? s_[p_] : '\0';
  }
  bool starts(const char* lit) {
    ws();
    return s_.compare(p_, std::strlen(lit), lit) == 0;
  }
  bool try_lit(const char* lit) {
    if (starts(lit)) {
      p_ += std::strlen(lit);
      return true;
    }
    return false;
  }
  // Keyword match that does not eat a prefix of a longer identifier.
  bool try_word(const char* w) {
    ws();
    size_t n = std::strlen(w);
    if (s_.compare(p_, n, w) != 0) return false;
    if (p_ + n < s_.size() && is_ident_char(s_[p_ + n])) return false;
    p_ += n;
    return true;
  }
  void expect(const char* lit) {
    if (!try_lit(lit)) error(std::string("expected '") + lit + "'");
  }
  static bool is_ident_start(char c) { return std::isalpha(static_cast<unsigned char>(c)) || c == '_'; }
  static bool is_ident_char(char c) {
    return std::isalnum(static_cast<unsigned char>(c)) || c == '_' || c == '.' || c == '$';
  }
  std::string ident() {
    ws();
    size_t b = p_;
    if (p_ >= s_.size() || !is_ident_start(s_[p_])) error("expected identifier");
    while (p_ < s_.size() && is_ident_char(s_[p_])) ++p_;
    return s_.substr(b, p_ - b);
  }
  std::string ssa_name() {
    ws();
    if (p_ >= s_.size() || s_[p_] != '%') error("expected SSA value");
    size_t b = p_++;
    while (p_ < s_.size() && (is_ident_char(s_[p_]) || s_[p_] == '#' || s_[p_] == '-')) ++p_;
    return s_.substr(b, p_ - b);
  }
  std::string symbol() {
    ws();
    if (p_ >= s_.size() || s_[p_] != '@') error("expected @symbol");
    ++p_;
    if (p_ < s_.size() && s_[p_] == '"') return string_lit();
    size_t b = p_;
    while (p_ < s_.size() && is_ident_char(s_[p_])) ++p_;
    return s_.substr(b, p_ - b);
  }
  std::string string_lit() {
    ws();
    if (s_[p_] != '"') error("expected string");
    ++p_;
    std::string out;
    while (p_ < s_.size() && s_[p_] != '"') {
      if (s_[p_] == '\\' && p_ + 1 < s_.size()) {
        out += s_[p_ + 1];
        p_ += 2;
      } else {
        out += s_[p_++];
      }
    }
    expect("\"");
    return out;
  }
  int64_t integer() {
    ws();
    size_t b = p_;
    if (p_ < s_.size() && (s_[p_] == '-' || s_[p_] == '+')) ++p_;
    if (p_ >= s_.size() || !std::isdigit(static_cast<unsigned char>(s_[p_]))) error("expected integer");
    while (p_ < s_.size() && std::isdigit(static_cast<unsigned char>(s_[p_]))) ++p_;
    return std::stoll(s_.substr(b, p_ - b));
  }
  // Skips a balanced group starting at the current bracket character.
  std::string balanced() {
    ws();
    size_t b = p_;
    std::vector<char> stack;
    do {
      if (p_ >= s_.size()) error("unbalanced brackets");
      char c = s_[p_];
      if (c == '"') {
        string_lit();
        continue;
      }
      if (c == '-' && p_ + 1 < s_.size() && s_[p_ + 1] == '>') {
        p_ += 2;
        continue;
      }
      if (c == '(' || c == '[' || c == '{' || c == '<') stack.push_back(c);
      if (c == ')' || c == ']' || c == '}' || c == '>') {
        if (stack.empty()) error("unbalanced brackets");
        stack.pop_back();
      }
      ++p_;
    } while (!stack.empty());
    return s_.substr(b, p_ - b);
  }
  Dims int_list() {  // [1, 2, 3] or []
    Dims out;
    expect("[");
    if (try_lit("]")) return out;
    do {
      out.push_back(integer());
    } while (try_lit(","));
    expect("]");
    return out;
  }

  // tensor<4x8xf32>
  TensorType type() {
    ws();
    if (!try_lit("tensor<")) {
      if (starts("!stablehlo.token") || starts("tuple<")) error("token and tuple types are not supported", Code::kUnimplemented);
      error("expected tensor type");
    }
    size_t b = p_;
    int depth = 1;
    while (p_ < s_.size() && depth > 0) {
      if (s_[p_] == '<') depth++;
      if (s_[p_] == '>') depth--;
      ++p_;
    }
    std::string body = s_.substr(b, p_ - b - 1);
    size_t comma = body.find(',');  // encoding attribute
    if (comma != std::string::npos) body = body.substr(0, comma);
    TensorType t;
    size_t pos = 0;
    while (true) {
      size_t x = body.find('x', pos);
      if (x == std::string::npos || !std::isdigit(static_cast<unsigned char>(body[pos]))) break;
      std::string d = body.substr(pos, x - pos);
      if (d.empty() || d.find_first_not_of("0123456789") != std::string::npos) break;
      t.dims.push_back(std::stoll(d));
      pos = x + 1;
    }
    if (!body.empty() && body[pos] == '?') error("dynamic shapes are not supported", Code::kUnimplemented);
    t.dtype = dtype_from_mlir(body.substr(pos));
    if (t.dtype == DType::kInvalid) error("unsupported element type '" + body.substr(pos) + "'", Code::kUnimplemented);
    return t;
  }

  // Either `type` or `(type, ...)`, each optionally followed by an attr dict.
  std::vector<TensorType> type_list_maybe_parens() {
    std::vector<TensorType> out;
    if (try_lit("(")) {
      if (try_lit(")")) return out;
      do {
        out.push_back(type());
        if (peek() == '{') balanced();
      } while (try_lit(","));
      expect(")");
    } else {
      // A bare result type carries no attributes; a following '{' opens a body.
      out.push_back(type());
    }
    return out;
  }

  // ---- value scopes ----
  Program prog_;
  std::vector<std::unordered_map<std::string, int>> scopes_;

  int new_value(const TensorType& t, const std::string& name) {
    prog_.values.push_back(Value{t, name});
    return static_cast<int>(prog_.values.size()) - 1;
  }
  void bind(const std::string& name, int id) { scopes_.back()[name] = id; }
  int lookup(const std::string& name) {
    for (auto it = scopes_.rbegin(); it != scopes_.rend(); ++it) {
      auto f = it->find(name);
      if (f != it->end()) return f->second;
    }
    error("use of undefined value " + name);
  }

  // ---- structure ----
  std::map<std::string, RawFunc> funcs_;
  std::vector<std::string> func_order_;
  // Calls recorded as ops with kind kReturn and `name` = "call:@callee".

  void parse_module();
  void parse_mesh();
  bool try_identity_op(const std::vector<std::string>& names);
  void parse_func();
  void parse_block(std::vector<Op>* ops, std::vector<int>* ret_values, bool top_level);
  Op parse_op(const std::vector<std::string>& result_names, int result_count_hint,
              std::vector<std::string>* out_names);
  void parse_region_body(Region* region, const std::vector<std::pair<std::string, TensorType>>& args);
  void parse_dense(const TensorType& t, Op* op);
  void parse_generic_attrs(const std::string& dict, Op* op);
  Op parse_top_k(const std::vector<std::string>& result_names, std::vector<std::string>* out_names);
  Op parse_composite(const std::vector<std::string>& result_names, std::vector<std::string>* out_names);
  void bind_results(Op* op, const std::vector<TensorType>& types, const std::vector<std::string>& result_names,
                    std::vector<std::string>* out_names);
  void parse_dnums(const std::string& body, Op* op);
  void inline_region(Region* region, const std::function<int(int)>& outer, int depth);
  void close_over_captures(Op* op);
  void inline_into(const std::string& fname, const std::vector<int>& args, std::vector<int>* results,
                   std::vector<Op>* out, int depth);
};

// `sdy.mesh @name = <["x"=2, ...]>` (Shardy): the program runs whole on one
// device, so meshes and the shardings that name them are accepted and
// ignored; the mesh's device count is kept for diagnostics.
void Parser::parse_mesh() {
  symbol();
  expect("=");
  ws();
  const std::string body = balanced();
  int64_t devices = 1;
  for (size_t i = body.find('='); i != std::string::npos; i = body.find('=', i + 1)) {
    const long long n = std::strtoll(body.c_str() + i + 1, nullptr, 10);
    if (n > 0) devices *= n;
  }
  prog_.mesh_devices = std::max<int64_t>(prog_.mesh_devices, devices);
}

// Identity ops: stablehlo.optimization_barrier (results are its operands,
// the reference lowers it to an alias, lowering_rules.zig:136) and
// sdy.sharding_constraint (a no-op on one device). Binds the result names
// to the operand values; no op is emitted. Returns false (input untouched)
// when the next op is not one of them.
bool Parser::try_identity_op(const std::vector<std::string>& names) {
  const size_t save = p_;
  ws();
  std::string nm;
  if (peek() == '"') nm = string_lit();
  else if (is_ident_start(peek())) nm = ident();
  if (nm != "stablehlo.optimization_barrier" && nm != "mhlo.optimization_barrier" &&
      nm != "sdy.sharding_constraint") {
    p_ = save;
    return false;
  }
  std::vector<int> vals;
  while (true) {
    ws();
    const char c = peek();
    if (c == ':') break;
    if (c == '\0') error("unexpected end of input in " + nm);
    if (c == ',' || c == '(' || c == ')') {
      ++p_;
      continue;
    }
    if (c == '%') {
      vals.push_back(lookup(ssa_name()));
      continue;
    }
    if (c == '<' || c == '{' || c == '[') {
      balanced();
      continue;
    }
    error("unexpected token in " + nm);
  }
  expect(":");
  ws();
  if (peek() == '(') {
    balanced();
    if (try_lit("->")) type_list_maybe_parens();
  } else {
    do {
      type();
    } while (try_lit(","));
  }
  std::vector<std::string> rn;
  if (names.size() == 1 && vals.size() > 1) {
    for (size_t i = 0; i < vals.size(); ++i) rn.push_back(names[0] + "#" + std::to_string(i));
    bind(names[0], vals[0]);
  } else {
    rn = names;
  }
  if (rn.size() != vals.size()) error(nm + ": result count does not match its operands");
  for (size_t i = 0; i < vals.size(); ++i) bind(rn[i], vals[i]);
  return true;
}

Program Parser::run() {
  scopes_.emplace_back();
  ws();
  if (try_word("module")) {
    if (peek() == '@') symbol();
    if (try_word("attributes")) {
      std::string attrs = balanced();
      auto grab = [&](const char* key) -> int {
        size_t k = attrs.find(key);
        if (k == std::string::npos) return 1;
        size_t eq = attrs.find('=', k);
        return std::atoi(attrs.c_str() + eq + 1);
      };
      prog_.num_partitions = grab("mhlo.num_partitions");
      prog_.num_replicas = grab("mhlo.num_replicas");
    }
    expect("{");
    while (!try_lit("}")) {
      if (eof()) error("unexpected end of module");
      if (try_word("sdy.mesh")) {
        parse_mesh();
        continue;
      }
      parse_func();
    }
  } else {
    while (!eof()) {
      if (try_word("sdy.mesh")) {
        parse_mesh();
        continue;
      }
      parse_func();
    }
  }
  if (!funcs_.count("main")) error("module has no @main function");
  // Inline everything into main.
  RawFunc& main = funcs_["main"];
  prog_.params = main.params;
  prog_.param_alias = main.param_alias;
  std::vector<int> results;
  inline_into("main", main.params, &results, &prog_.ops, 0);
  for (Op& op : prog_.ops) close_over_captures(&op);
  prog_.results = results;
  Op ret;
  ret.kind = OpKind::kReturn;
  ret.name = "return";
  ret.operands = results;
  prog_.ops.push_back(ret);
  return std::move(prog_);
}

void Parser::inline_into(const std::string& fname, const std::vector<int>& args,
                         std::vector<int>* results, std::vector<Op>* out, int depth) {
  if (depth > 64) error("call depth exceeds 64 (recursive call?)");
  auto it = funcs_.find(fname);
  if (it == funcs_.end()) error("call to undefined function @" + fname);
  const RawFunc& f = it->second;
  if (args.size() != f.params.size()) error("call to @" + fname + " has wrong argument count");
  // Value remapping: the function's own value ids -> ids in the inlined copy.
  std::unordered_map<int, int> remap;
  for (size_t i = 0; i < args.size(); ++i) remap[f.params[i]] = args[i];
  std::function<int(int)> map_val = [&](int v) {
    auto r = remap.find(v);
    return r == remap.end() ? v : r->second;
  };
  const bool is_main = depth == 0;
  for (const Op& op0 : f.ops) {
    if (op0.name.rfind("call:", 0) == 0) {
      std::vector<int> call_args;
      for (int v : op0.operands) call_args.push_back(map_val(v));
      std::vector<int> call_results;
      inline_into(op0.name.substr(5), call_args, &call_results, out, depth + 1);
      if (call_results.size() != op0.results.size()) error("call result count mismatch for " + op0.name);
      for (size_t i = 0; i < call_results.size(); ++i) remap[op0.results[i]] = call_results[i];
      continue;
    }
    if (op0.kind == OpKind::kReturn) {
      for (int v : op0.operands) results->push_back(map_val(v));
      continue;
    }
    Op op = op0;
    for (int& v : op.operands) v = map_val(v);
    for (Region& r : op.regions) inline_region(&r, map_val, depth);
    if (!is_main) {
      // Fresh result ids so that a function called twice yields distinct values.
      for (int& v : op.results) {
        int nv = new_value(prog_.values[v].type, prog_.values[v].name);
        remap[v] = nv;
        v = nv;
      }
    }
    out->push_back(std::move(op));
  }
}

// Values a region reads that it does not define (its own block arguments
// and op results, nested regions included), in first-use order.
static void region_free_values(const Region& r, std::set<int>* defined, std::vector<int>* free_vals,
                               std::set<int>* seen) {
  for (int v : r.params) defined->insert(v);
  for (const Op& op : r.ops) {
    for (int v : op.operands)
      if (!defined->count(v) && seen->insert(v).second) free_vals->push_back(v);
    for (const Region& inner : op.regions) region_free_values(inner, defined, free_vals, seen);
    for (int v : op.results) defined->insert(v);
  }
}

// A while reads its regions' captured values as operands after the loop
// state (op.sizes = {state count}), so that liveness and scheduling see
// them like any other input; nested whiles first.
void Parser::close_over_captures(Op* op) {
  for (Region& r : op->regions)
    for (Op& inner : r.ops) close_over_captures(&inner);
  if (op->kind != OpKind::kWhile) return;
  if (op->regions.size() != 2) error("while needs a cond and a body region");
  const size_t n_state = op->operands.size();
  std::set<int> seen;
  std::vector<int> free_vals;
  for (const Region& r : op->regions) {
    std::set<int> defined;
    region_free_values(r, &defined, &free_vals, &seen);
  }
  op->sizes = {static_cast<int64_t>(n_state)};
  for (int v : free_vals) op->operands.push_back(v);
}

// Inside a region (a while's cond or body): values captured from the
// enclosing function are remapped like the function's own, and calls are
// inlined in place; the region keeps its own return.
void Parser::inline_region(Region* region, const std::function<int(int)>& outer, int depth) {
  std::unordered_map<int, int> remap;
  std::function<int(int)> map_val = [&](int v) {
    auto r = remap.find(v);
    return r == remap.end() ? outer(v) : r->second;
  };
  std::vector<Op> ops;
  for (const Op& op0 : region->ops) {
    if (op0.name.rfind("call:", 0) == 0) {
      std::vector<int> call_args;
      for (int v : op0.operands) call_args.push_back(map_val(v));
      std::vector<int> call_results;
      inline_into(op0.name.substr(5), call_args, &call_results, &ops, depth + 1);
      if (call_results.size() != op0.results.size()) error("call result count mismatch for " + op0.name);
      for (size_t i = 0; i < call_results.size(); ++i) remap[op0.results[i]] = call_results[i];
      continue;
    }
    Op op = op0;
    for (int& v : op.operands) v = map_val(v);
    for (Region& r : op.regions) inline_region(&r, map_val, depth);
    ops.push_back(std::move(op));
  }
  region->ops = std::move(ops);
}

// Donation attributes of an entry argument, as jax.jit(donate_argnums=...)
// lowers them: `tf.aliasing_output = N : i32` names the result that reuses
// the argument's buffer; `jax.buffer_donor = true` donates it without one.
static int donation_from_attrs(const std::string& attrs) {
  size_t p = attrs.find("tf.aliasing_output");
  if (p != std::string::npos) {
    p = attrs.find('=', p);
    if (p != std::string::npos) {
      ++p;
      while (p < attrs.size() && attrs[p] == ' ') ++p;
      size_t q = p;
      while (q < attrs.size() && isdigit(static_cast<unsigned char>(attrs[q]))) ++q;
      if (q > p) return std::stoi(attrs.substr(p, q - p));
    }
  }
  p = attrs.find("jax.buffer_donor");
  if (p != std::string::npos && attrs.find("true", p) != std::string::npos) return -2;
  return -1;
}

void Parser::parse_func() {
  ws();
  if (!try_word("func.func")) error("expected func.func");
  try_word("public") || try_word("private") || try_word("nested");
  RawFunc f;
  f.name = symbol();
  scopes_.emplace_back();
  expect("(");
  if (!try_lit(")")) {
    do {
      std::string n = ssa_name();
      expect(":");
      TensorType t = type();
      int alias = -1;
      if (peek() == '{') alias = donation_from_attrs(balanced());
      int id = new_value(t, n);
      bind(n, id);
      f.params.push_back(id);
      f.param_alias.push_back(alias);
    } while (try_lit(","));
    expect(")");
  }
  if (try_lit("->")) f.result_types = type_list_maybe_parens();
  if (try_word("attributes")) balanced();
  expect("{");
  std::vector<int> rets;
  parse_block(&f.ops, &rets, true);
  scopes_.pop_back();
  func_order_.push_back(f.name);
  funcs_[f.name] = std::move(f);
}

// Parses ops until the closing '}' (consumed).
void Parser::parse_block(std::vector<Op>* ops, std::vector<int>* ret_values, bool top_level) {
  (void)top_level;
  while (true) {
    ws();
    if (try_lit("}")) return;
    if (eof()) error("unexpected end of input in block");
    if (starts("^")) {  // block label of a generic region: ^bb0(%a: t, ...):
      error("unexpected block label");
    }
    std::vector<std::string> names;
    int count_hint = -1;
    if (peek() == '%') {
      names.push_back(ssa_name());
      if (try_lit(":")) count_hint = static_cast<int>(integer());
      while (try_lit(",")) names.push_back(ssa_name());
      expect("=");
    }
    // return forms
    if (names.empty() && (try_word("return") || try_word("func.return") || try_word("stablehlo.return") ||
                          try_lit("\"stablehlo.return\"") || try_lit("\"func.return\""))) {
      Op ret;
      ret.kind = OpKind::kReturn;
      ret.name = "return";
      bool generic = false;
      if (try_lit("(")) generic = true;
      if (peek() == '%') {
        do {
          ret.operands.push_back(lookup(ssa_name()));
        } while (try_lit(","));
      }
      if (generic) expect(")");
      if (try_lit(":")) {
        if (generic) {
          balanced();  // (types)
          if (try_lit("->")) type_list_maybe_parens();
        } else {
          do {
            type();
          } while (try_lit(","));
        }
      }
      *ret_values = ret.operands;
      ops->push_back(ret);
      continue;
    }
    if (try_identity_op(names)) continue;
    std::vector<std::string> out_names;
    Op op = parse_op(names, count_hint, &out_names);
    ops->push_back(std::move(op));
  }
}

void Parser::parse_region_body(Region* region,
                               const std::vector<std::pair<std::string, TensorType>>& args) {
  scopes_.emplace_back();
  for (const auto& a : args) {
    int id = new_value(a.second, a.first);
    bind(a.first, id);
    region->params.push_back(id);
  }
  std::vector<int> rets;
  parse_block(&region->ops, &rets, false);
  scopes_.pop_back();
}

static bool parse_dims_attr(const std::string& raw, Dims* out) {
  // "[1, 2]" or "array<i64: 1, 2>" or "array<i64>"
  out->clear();
  size_t b = raw.find_first_of("[:");
  if (b == std::string::npos) return raw.find("array<") != std::string::npos;
  size_t i = b + 1;
  while (i < raw.size()) {
    while (i < raw.size() && (raw[i] == ' ' || raw[i] == ',')) ++i;
    if (i >= raw.size() || raw[i] == ']' || raw[i] == '>') break;
    char* end = nullptr;
    long long v = std::strtoll(raw.c_str() + i, &end, 10);
    if (end == raw.c_str() + i) return false;
    out->push_back(v);
    i = end - raw.c_str();
  }
  return true;
}

// Splits "a = x, b = y<..., ...>, c = [1, 2]" at top-level commas into a map.
static std::map<std::string, std::string> split_attr_dict(const std::string& body) {
  std::map<std::string, std::string> out;
  size_t i = 0;
  while (i < body.size()) {
    while (i < body.size() && (body[i] == ' ' || body[i] == ',' || body[i] == '\n')) ++i;
    size_t kb = i;
    while (i < body.size() && body[i] != '=' && body[i] != ',') ++i;
    std::string key = body.substr(kb, i - kb);
    while (!key.empty() && key.back() == ' ') key.pop_back();
    if (i >= body.size() || body[i] == ',') {
      if (!key.empty()) out[key] = "";
      continue;
    }
    ++i;  // '='
    int depth = 0;
    size_t vb = i;
    bool in_str = false;
    while (i < body.size()) {
      char c = body[i];
      if (in_str) {
        if (c == '\\') ++i;
        else if (c == '"') in_str = false;
      } else if (c == '"') {
        in_str = true;
      } else if (c == '-' && i + 1 < body.size() && body[i + 1] == '>') {
        ++i;
      } else if (c == '(' || c == '[' || c == '{' || c == '<') {
        depth++;
      } else if (c == ')' || c == ']' || c == '}' || c == '>') {
        depth--;
      } else if (c == ',' && depth == 0) {
        break;
      }
      ++i;
    }
    std::string val = body.substr(vb, i - vb);
    size_t a = val.find_first_not_of(' ');
    size_t z = val.find_last_not_of(' ');
    out[key] = a == std::string::npos ? "" : val.substr(a, z - a + 1);
  }
  return out;
}

void Parser::parse_dnums(const std::string& raw, Op* op) {
  // raw: "#stablehlo.gather<offset_dims = [2], ...>" or "#stablehlo.scatter<...>"
  size_t lt = raw.find('<');
  size_t gt = raw.rfind('>');
  if (lt == std::string::npos || gt == std::string::npos) error("malformed dimension numbers");
  auto kv = split_attr_dict(raw.substr(lt + 1, gt - lt - 1));
  auto dims_of = [&](const char* key, Dims* d) {
    auto it = kv.find(key);
    if (it != kv.end()) parse_dims_attr(it->second, d);
  };
  dims_of("offset_dims", &op->offset_dims);
  dims_of("collapsed_slice_dims", &op->collapsed_slice_dims);
  dims_of("start_index_map", &op->start_index_map);
  dims_of("operand_batching_dims", &op->operand_batching_dims);
  dims_of("start_indices_batching_dims", &op->start_indices_batching_dims);
  dims_of("update_window_dims", &op->update_window_dims);
  dims_of("inserted_window_dims", &op->inserted_window_dims);
  dims_of("scatter_dims_to_operand_dims", &op->scatter_dims_to_operand_dims);
  dims_of("input_batching_dims", &op->input_batching_dims);
  dims_of("scatter_indices_batching_dims", &op->scatter_indices_batching_dims);
  auto ivd = kv.find("index_vector_dim");
  if (ivd != kv.end()) op->index_vector_dim = std::stoll(ivd->second);
}

void Parser::parse_generic_attrs(const std::string& dict, Op* op) {
  // dict includes the outer braces: "{...}" (from "<{...}>" or "{...}")
  size_t b = dict.find('{');
  size_t e = dict.rfind('}');
  if (b == std::string::npos || e == std::string::npos) return;
  auto kv = split_attr_dict(dict.substr(b + 1, e - b - 1));
  for (const auto& [key, val] : kv) {
    if (key == "dimension_numbers" || key == "scatter_dimension_numbers") {
      parse_dnums(val, op);
    } else if (key == "slice_sizes") {
      parse_dims_attr(val, &op->sizes);
    } else if (key == "indices_are_sorted") {
      op->indices_are_sorted = val == "true";
    } else if (key == "unique_indices") {
      op->unique_indices = val == "true";
    } else if (key == "start_indices") {
      parse_dims_attr(val, &op->start);
    } else if (key == "limit_indices") {
      parse_dims_attr(val, &op->limit);
    } else if (key == "strides") {
      parse_dims_attr(val, &op->strides);
    } else if (key == "dimensions" || key == "broadcast_dimensions" || key == "permutation") {
      parse_dims_attr(val, &op->dims);
    } else if (key == "iota_dimension" || key == "dimension") {
      op->dim = std::stoll(val.substr(0, val.find(':')));
    } else if (key == "slice_sizes") {
      parse_dims_attr(val, &op->sizes);
    } else if (key == "edge_padding_low") {
      parse_dims_attr(val, &op->pad_low);
    } else if (key == "edge_padding_high") {
      parse_dims_attr(val, &op->pad_high);
    } else if (key == "interior_padding") {
      parse_dims_attr(val, &op->pad_interior);
    } else if (key == "comparison_direction") {
      std::string d = val.substr(val.rfind(' ') + 1);
      d = d.substr(0, d.find('>'));
      static const std::pair<const char*, CmpDir> dirs[] = {
          {"EQ", CmpDir::kEQ}, {"NE", CmpDir::kNE}, {"LT", CmpDir::kLT},
          {"LE", CmpDir::kLE}, {"GT", CmpDir::kGT}, {"GE", CmpDir::kGE}};
      for (auto& dd : dirs)
        if (d == dd.first) op->cmp_dir = dd.second;
    } else if (key == "exponent_bits") {
      op->exponent_bits = std::stoll(val.substr(0, val.find(':')));
    } else if (key == "mantissa_bits") {
      op->mantissa_bits = std::stoll(val.substr(0, val.find(':')));
    } else if (key == "window_dimensions") {
      parse_dims_attr(val, &op->sizes);
    } else if (key == "window_strides") {
      parse_dims_attr(val, &op->strides);
    } else if (key == "base_dilations") {
      parse_dims_attr(val, &op->base_dilations);
    } else if (key == "window_dilations") {
      parse_dims_attr(val, &op->window_dilations);
    } else if (key == "padding") {
      // dense<[[lo, hi], ...]> : tensor<Nx2xi64>, or dense<0> (splat)
      Dims flat;
      const size_t lt = val.find('<');
      const size_t colon = val.rfind(':');
      std::string body = lt == std::string::npos ? val : val.substr(lt + 1, (colon == std::string::npos ? val.size() : colon) - lt - 1);
      for (char& ch : body)
        if (ch == '[' || ch == ']' || ch == '>' || ch == '<') ch = ' ';
      size_t i = 0;
      while (i < body.size()) {
        while (i < body.size() && (body[i] == ' ' || body[i] == ',')) ++i;
        if (i >= body.size()) break;
        char* end = nullptr;
        long long v = std::strtoll(body.c_str() + i, &end, 10);
        if (end == body.c_str() + i) break;
        flat.push_back(v);
        i = end - body.c_str();
      }
      op->pad_low.clear();
      op->pad_high.clear();
      if (flat.size() == 1) {  // splat: filled in once the rank is known
        op->pad_low.push_back(flat[0]);
        op->pad_high.push_back(-(flat[0] + 1));  // marker
      } else {
        for (size_t k = 0; k + 1 < flat.size(); k += 2) {
          op->pad_low.push_back(flat[k]);
          op->pad_high.push_back(flat[k + 1]);
        }
      }
    } else if (key == "call_target_name") {
      const size_t q0 = val.find('"'), q1 = val.rfind('"');
      if (q0 != std::string::npos && q1 > q0) op->target = val.substr(q0 + 1, q1 - q0 - 1);
    } else if (key == "dot_dimension_numbers") {
      size_t lt = val.find('<');
      size_t gt = val.rfind('>');
      auto dk = split_attr_dict(val.substr(lt + 1, gt - lt - 1));
      auto g = [&](const char* k, Dims* d) {
        auto it = dk.find(k);
        if (it != dk.end()) parse_dims_attr(it->second, d);
      };
      g("lhs_batching_dimensions", &op->lhs_batch);
      g("rhs_batching_dimensions", &op->rhs_batch);
      g("lhs_contracting_dimensions", &op->lhs_contract);
      g("rhs_contracting_dimensions", &op->rhs_contract);
    }
  }
}

// dense<...> literal for a tensor of type t.
void Parser::parse_dense(const TensorType& t, Op* op) {
  // cursor is just after "dense<"
  const size_t esz = dtype_size(t.dtype);
  const int64_t n = t.elements();
  ws();
  if (s_[p_] == '"') {
    std::string hex = string_lit();
    expect(">");
    if (hex.rfind("0x", 0) != 0) error("dense string literal must be hex");
    std::vector<uint8_t> bytes;
    for (size_t i = 2; i + 1 < hex.size(); i += 2) bytes.push_back(static_cast<uint8_t>(std::stoi(hex.substr(i, 2), nullptr, 16)));
    if (bytes.size() == esz && n != 1) {
      op->splat = true;
    } else if (bytes.size() != esz * static_cast<size_t>(n)) {
      error("hex literal size does not match tensor type");
    }
    op->literal = std::move(bytes);
    return;
  }
  // Flatten nested lists of scalars.
  std::vector<std::string> elems;
  int depth = 0;
  while (true) {
    ws();
    char c = s_[p_];
    if (c == '[') {
      depth++;
      p_++;
    } else if (c == ']') {
      depth--;
      p_++;
    } else if (c == ',') {
      p_++;
    } else if (c == '>' && depth == 0) {
      p_++;
      break;
    } else if (c == '(') {
      error("complex literals are not supported", Code::kUnimplemented);
    } else {
      size_t b = p_;
      while (p_ < s_.size() && s_[p_] != ',' && s_[p_] != ']' && s_[p_] != '>' && s_[p_] != ' ' && s_[p_] != '\n') ++p_;
      elems.push_back(s_.substr(b, p_ - b));
    }
  }
  if (elems.size() == 1 && n != 1) {
    op->splat = true;
  } else if (static_cast<int64_t>(elems.size()) != n) {
    error(strformat("dense literal has %zu elements, type needs %lld", elems.size(), static_cast<long long>(n)));
  }
  op->literal.resize(elems.size() * esz);
  for (size_t i = 0; i < elems.size(); ++i) {
    const std::string& e = elems[i];
    uint8_t* dst = op->literal.data() + i * esz;
    const bool is_hex = e.rfind("0x", 0) == 0 || e.rfind("0X", 0) == 0;
    if (is_hex) {
      uint64_t bits = std::stoull(e.substr(2), nullptr, 16);
      std::memcpy(dst, &bits, esz);  // little endian
      continue;
    }
    if (t.dtype == DType::kPred) {
      dst[0] = (e == "true" || e == "1") ? 1 : 0;
      continue;
    }
    if (dtype_is_float(t.dtype)) {
      double d;
      if (e == "inf" || e == "+inf") d = INFINITY;
      else if (e == "-inf") d = -INFINITY;
      else if (e == "nan") d = NAN;
      else d = std::strtod(e.c_str(), nullptr);
      if (t.dtype == DType::kF32) {
        float f = static_cast<float>(d);
        std::memcpy(dst, &f, 4);
      } else if (t.dtype == DType::kF64) {
        std::memcpy(dst, &d, 8);
      } else if (t.dtype == DType::kBF16) {
        uint16_t b = f32_to_bf16_bits(static_cast<float>(d));
        std::memcpy(dst, &b, 2);
      } else {
        uint16_t h = f32_to_f16_bits(static_cast<float>(d));
        std::memcpy(dst, &h, 2);
      }
      continue;
    }
    if (e == "true" || e == "false") {
      int64_t v = e == "true";
      std::memcpy(dst, &v, esz);
      continue;
    }
    if (dtype_is_unsigned_int(t.dtype)) {
      uint64_t v = std::stoull(e);
      std::memcpy(dst, &v, esz);
    } else {
      int64_t v = std::stoll(e);
      std::memcpy(dst, &v, esz);
    }
  }
}

void Parser::bind_results(Op* op, const std::vector<TensorType>& types, const std::vector<std::string>& result_names,
                          std::vector<std::string>* out_names) {
  std::vector<std::string> names;
  if (result_names.size() == 1 && types.size() > 1) {
    for (size_t i = 0; i < types.size(); ++i) names.push_back(result_names[0] + "#" + std::to_string(i));
  } else {
    names = result_names;
  }
  if (names.size() != types.size()) error("result name count does not match signature");
  for (size_t i = 0; i < types.size(); ++i) {
    int id = new_value(types[i], names[i]);
    bind(names[i], id);
    op->results.push_back(id);
  }
  if (out_names) *out_names = names;
}

// chlo.top_k(%x, k = K) : tensor<...xN> -> (tensor<...xK>, tensor<...xKxi32>)
// (reference: stablehlo_topk_import.zig:71-79).
Op Parser::parse_top_k(const std::vector<std::string>& result_names, std::vector<std::string>* out_names) {
  Op op;
  op.kind = OpKind::kTopK;
  op.name = "chlo.top_k";
  expect("(");
  op.operands.push_back(lookup(ssa_name()));
  expect(",");
  if (!try_word("k")) error("chlo.top_k: expected 'k = <int>'");
  expect("=");
  op.sizes = {integer()};
  expect(")");
  if (peek() == '{') balanced();
  expect(":");
  if (peek() == '(') {
    balanced();
  } else {
    type();
  }
  expect("->");
  bind_results(&op, type_list_maybe_parens(), result_names, out_names);
  if (op.results.size() != 2) error("chlo.top_k must have two results");
  return op;
}

// stablehlo.composite "name" %a, ... {composite_attributes = {...},
// decomposition = @f} : (...) -> ...: a top_k composite (name containing
// "top_k", as stablehlo_topk_import.zig:81-97 recognises) becomes the top_k
// op with k from the result type; any other composite is a call of its
// decomposition.
Op Parser::parse_composite(const std::vector<std::string>& result_names, std::vector<std::string>* out_names) {
  Op op;
  const std::string cname = string_lit();
  std::vector<int> operands;
  while (peek() == '%') {
    operands.push_back(lookup(ssa_name()));
    if (!try_lit(",")) break;
  }
  std::string decomposition;
  if (peek() == '{') {
    const std::string dict = balanced();
    const size_t d = dict.find("decomposition");
    if (d != std::string::npos) {
      const size_t at = dict.find('@', d);
      size_t e = at + 1;
      while (e < dict.size() && (std::isalnum(static_cast<unsigned char>(dict[e])) || dict[e] == '_' ||
                                 dict[e] == '.' || dict[e] == '$' || dict[e] == '-'))
        ++e;
      if (at != std::string::npos) decomposition = dict.substr(at + 1, e - at - 1);
    }
  }
  expect(":");
  balanced();  // (operand types)
  expect("->");
  std::vector<TensorType> rts = type_list_maybe_parens();
  op.operands = operands;
  if (cname.find("top_k") != std::string::npos && operands.size() == 1 && rts.size() == 2 &&
      rts[0].rank() >= 1) {
    op.kind = OpKind::kTopK;
    op.name = "chlo.top_k";
    op.sizes = {rts[0].dims.back()};
  } else {
    if (decomposition.empty()) error("stablehlo.composite without a decomposition", Code::kUnimplemented);
    op.name = "call:" + decomposition;
  }
  bind_results(&op, rts, result_names, out_names);
  if (rts.size() > 1 && op.name.rfind("call:", 0) == 0) bind(result_names[0], op.results[0]);
  return op;
}

Op Parser::parse_op(const std::vector<std::string>& result_names, int count_hint,
                    std::vector<std::string>* out_names) {
  Op op;
  ws();
  bool generic = false;
  std::string full;
  if (peek() == '"') {
    generic = true;
    full = string_lit();
  } else {
    full = ident();
  }
  // call / func.call
  if (full == "call" || full == "func.call") {
    std::string callee = symbol();
    op.name = "call:" + callee;
    expect("(");
    if (!try_lit(")")) {
      do {
        op.operands.push_back(lookup(ssa_name()));
      } while (try_lit(","));
      expect(")");
    }
    if (peek() == '{') balanced();
    expect(":");
    balanced();  // (arg types)
    expect("->");
    std::vector<TensorType> rts = type_list_maybe_parens();
    // bind results
    std::vector<std::string> names;
    if (result_names.size() == 1 && rts.size() > 1) {
      for (size_t i = 0; i < rts.size(); ++i) names.push_back(result_names[0] + "#" + std::to_string(i));
    } else {
      names = result_names;
    }
    if (names.size() != rts.size()) error("call result count mismatch");
    for (size_t i = 0; i < rts.size(); ++i) {
      int id = new_value(rts[i], names[i]);
      bind(names[i], id);
      op.results.push_back(id);
    }
    if (rts.size() > 1) bind(result_names[0], op.results[0]);
    return op;
  }
  if (full == "chlo.top_k") return parse_top_k(result_names, out_names);
  if (full == "stablehlo.composite") return parse_composite(result_names, out_names);
  std::string mnemonic = full;
  if (mnemonic.rfind("stablehlo.", 0) == 0) mnemonic = mnemonic.substr(10);
  else if (mnemonic.rfind("mhlo.", 0) == 0) mnemonic = mnemonic.substr(5);
  else error("unsupported op '" + full + "'", Code::kUnimplemented);
  if (!lookup_op(mnemonic, &op.kind) || op.kind == OpKind::kReturn) {
    error("unsupported stablehlo op '" + full + "'", Code::kUnimplemented);
  }
  op.name = "stablehlo." + mnemonic;

  std::vector<int> init_operands;  // reduce init values
  std::vector<TensorType> sig_inputs, sig_outputs;
  bool have_dense = false;
  TensorType dense_type;
  size_t dense_pos = 0;

  if (generic) {
    expect("(");
    if (!try_lit(")")) {
      do {
        op.operands.push_back(lookup(ssa_name()));
      } while (try_lit(","));
      expect(")");
    }
    if (try_lit("<")) {
      std::string dict = balanced();
      expect(">");
      parse_generic_attrs(dict, &op);
    }
    if (try_lit("(")) {  // regions
      do {
        expect("{");
        Region region;
        std::vector<std::pair<std::string, TensorType>> args;
        if (try_lit("^")) {
          ident();  // bb0
          expect("(");
          if (!try_lit(")")) {
            do {
              std::string n = ssa_name();
              expect(":");
              args.emplace_back(n, type());
            } while (try_lit(","));
            expect(")");
          }
          expect(":");
        }
        parse_region_body(&region, args);
        op.regions.push_back(std::move(region));
      } while (try_lit(","));
      expect(")");
    }
    if (peek() == '{') parse_generic_attrs(balanced(), &op);
    expect(":");
    expect("(");
    if (!try_lit(")")) {
      do {
        sig_inputs.push_back(type());
      } while (try_lit(","));
      expect(")");
    }
    expect("->");
    sig_outputs = type_list_maybe_parens();
  } else if (op.kind == OpKind::kWhile) {
    // while(%iterArg = %init, ...) : t, ... cond { ... } do { ... }: the
    // iteration names are the block arguments of both regions.
    std::vector<std::string> iter_names;
    expect("(");
    if (!try_lit(")")) {
      do {
        iter_names.push_back(ssa_name());
        expect("=");
        op.operands.push_back(lookup(ssa_name()));
      } while (try_lit(","));
      expect(")");
    }
    if (peek() == '{') parse_generic_attrs(balanced(), &op);
    if (!iter_names.empty()) {
      expect(":");
      do {
        sig_outputs.push_back(type());
      } while (try_lit(","));
    }
    if (sig_outputs.size() != iter_names.size()) error("while: state names and types differ in count");
    std::vector<std::pair<std::string, TensorType>> args;
    for (size_t i = 0; i < iter_names.size(); ++i) args.emplace_back(iter_names[i], sig_outputs[i]);
    for (const char* kw : {"cond", "do"}) {
      if (!try_word(kw)) error(std::string("while: expected '") + kw + "' region");
      expect("{");
      Region region;
      parse_region_body(&region, args);
      op.regions.push_back(std::move(region));
    }
  } else {
    if (op.kind == OpKind::kCustomCall) {  // custom_call @target(%a, ...) {attrs} : (...) -> ...
      op.target = symbol();
      expect("(");
      if (!try_lit(")")) {
        do {
          op.operands.push_back(lookup(ssa_name()));
        } while (try_lit(","));
        expect(")");
      }
    }
    // Pretty form: items until the top-level ':'.
    while (true) {
      ws();
      char c = peek();
      if (c == ':') break;
      if (c == '\0') error("unexpected end of input in op");
      if (c == ',') {
        ++p_;
        continue;
      }
      if (c == '%') {
        op.operands.push_back(lookup(ssa_name()));
        continue;
      }
      if (c == '(') {  // reduce operand group: (%x init: %y)
        ++p_;
        op.operands.push_back(lookup(ssa_name()));
        expect("init");
        expect(":");
        init_operands.push_back(lookup(ssa_name()));
        expect(")");
        continue;
      }
      if (c == '[') {  // slice ranges [a:b(:s), ...]
        ++p_;
        if (!try_lit("]")) {
          do {
            int64_t a = integer();
            expect(":");
            int64_t b = integer();
            int64_t st = 1;
            if (try_lit(":")) st = integer();
            op.start.push_back(a);
            op.limit.push_back(b);
            op.strides.push_back(st);
          } while (try_lit(","));
          expect("]");
        }
        continue;
      }
      if (c == '{') {
        parse_generic_attrs(balanced(), &op);
        continue;
      }
      if (c == '<') {
        std::string dict = balanced();
        parse_generic_attrs(dict, &op);
        continue;
      }
      std::string word = ident();
      if (word == "dense") {
        expect("<");
        have_dense = true;
        dense_pos = p_;
        // Skip now; decode after the type is known.
        int depth = 1;
        bool in_str = false;
        while (p_ < s_.size() && depth > 0) {
          char ch = s_[p_];
          if (in_str) {
            if (ch == '"') in_str = false;
          } else if (ch == '"') {
            in_str = true;
          } else if (ch == '<') {
            depth++;
          } else if (ch == '>') {
            depth--;
          }
          ++p_;
        }
        continue;
      }
      if (word == "across") {
        expect("dimensions");
        expect("=");
        op.dims = int_list();
        continue;
      }
      if (word == "applies") {
        std::string body_op = ident();
        // Synthesize a region "return body_op(a, b)".
        std::string m = body_op.rfind("stablehlo.", 0) == 0 ? body_op.substr(10) : body_op;
        OpKind bk;
        if (!lookup_op(m, &bk)) error("unsupported reducer " + body_op, Code::kUnimplemented);
        // Region is built after the types are known (needs the init type).
        op.name += "|applies:" + m;
        continue;
      }
      if (word == "init") error("unexpected 'init'");
      if (try_lit("=")) {
        if (word == "dims" || word == "dimensions" || word == "permutation") {
          op.dims = int_list();
        } else if (word == "dim") {
          op.dim = integer();
        } else if (word == "sizes") {
          op.sizes = int_list();
        } else if (word == "low") {
          op.pad_low = int_list();
        } else if (word == "high") {
          op.pad_high = int_list();
        } else if (word == "interior") {
          op.pad_interior = int_list();
        } else if (word == "batching_dims") {
          op.lhs_batch = int_list();
          expect("x");
          op.rhs_batch = int_list();
        } else if (word == "contracting_dims") {
          op.lhs_contract = int_list();
          expect("x");
          op.rhs_contract = int_list();
        } else if (word == "format") {  // reduce_precision: e<exponent>m<mantissa>
          const std::string f = ident();
          const size_t mpos = f.find('m');
          if (f.empty() || f[0] != 'e' || mpos == std::string::npos) error("bad reduce_precision format " + f);
          op.exponent_bits = std::stoll(f.substr(1, mpos - 1));
          op.mantissa_bits = std::stoll(f.substr(mpos + 1));
        } else if (word == "precision" || word == "algorithm") {
          if (peek() == '[' || peek() == '<' || peek() == '#') balanced();
          else ident();
          if (peek() == '<') balanced();
        } else {
          // Unknown keyword attribute: skip its value.
          if (peek() == '[' || peek() == '<' || peek() == '{' || peek() == '(') balanced();
          else if (peek() == '#') {
            ++p_;
            ident();
            if (peek() == '<') balanced();
          } else if (peek() == '"') string_lit();
          else if (peek() == '-' || std::isdigit(static_cast<unsigned char>(peek()))) integer();
          else ident();
        }
        continue;
      }
      // Bare words: comparison direction / type.
      static const std::pair<const char*, CmpDir> dirs[] = {
          {"EQ", CmpDir::kEQ}, {"NE", CmpDir::kNE}, {"LT", CmpDir::kLT},
          {"LE", CmpDir::kLE}, {"GT", CmpDir::kGT}, {"GE", CmpDir::kGE}};
      bool matched = false;
      for (auto& d : dirs) {
        if (word == d.first) {
          op.cmp_dir = d.second;
          matched = true;
        }
      }
      if (word == "FLOAT") op.cmp_type = CmpType::kFloat, matched = true;
      if (word == "TOTALORDER") op.cmp_type = CmpType::kTotalOrder, matched = true;
      if (word == "SIGNED") op.cmp_type = CmpType::kSigned, matched = true;
      if (word == "UNSIGNED") op.cmp_type = CmpType::kUnsigned, matched = true;
      if (!matched) error("unexpected token '" + word + "' in " + full);
    }
    expect(":");
    // Signature: "(ins) -> outs" | "t" | "t, t"
    if (peek() == '(') {
      expect("(");
      if (!try_lit(")")) {
        do {
          sig_inputs.push_back(type());
        } while (try_lit(","));
        expect(")");
      }
      expect("->");
      sig_outputs = type_list_maybe_parens();
    } else {
      std::vector<TensorType> ts;
      do {
        ts.push_back(type());
      } while (try_lit(","));
      // select prints "pred_type, result_type"; others print the result type.
      sig_outputs = {ts.back()};
      if (ts.size() > 1) sig_inputs = ts;
    }
    // reduce with a region in pretty form: reducer(%a: t, %b: t) (%c: t, %d: t) { ... }
    if (op.kind == OpKind::kReduce && try_word("reducer")) {
      std::vector<std::pair<std::string, TensorType>> lhs, rhs;
      while (try_lit("(")) {
        std::string a = ssa_name();
        expect(":");
        TensorType at = type();
        expect(",");
        std::string b = ssa_name();
        expect(":");
        TensorType bt = type();
        expect(")");
        lhs.emplace_back(a, at);
        rhs.emplace_back(b, bt);
      }
      expect("{");
      // Region block arguments are (acc_0..acc_n-1, x_0..x_n-1) in order.
      std::vector<std::pair<std::string, TensorType>> args = lhs;
      args.insert(args.end(), rhs.begin(), rhs.end());
      Region region;
      parse_region_body(&region, args);
      op.regions.push_back(std::move(region));
    }
  }

  // Reduce init operands follow the inputs.
  op.operands.insert(op.operands.end(), init_operands.begin(), init_operands.end());

  // Results.
  int nres = static_cast<int>(sig_outputs.size());
  if (count_hint > 0 && count_hint != nres) error("result count does not match signature");
  std::vector<std::string> names;
  if (result_names.size() == 1 && nres > 1) {
    for (int i = 0; i < nres; ++i) names.push_back(result_names[0] + "#" + std::to_string(i));
  } else {
    names = result_names;
  }
  if (static_cast<int>(names.size()) != nres) error("result name count does not match signature");
  for (int i = 0; i < nres; ++i) {
    int id = new_value(sig_outputs[i], names[i]);
    bind(names[i], id);
    op.results.push_back(id);
  }
  if (out_names) *out_names = names;
  if (op.kind == OpKind::kReduceWindow && !op.operands.empty()) {
    // Defaults of the optional window attributes, and a splat padding.
    const size_t r = prog_.values[op.operands[0]].type.dims.size();
    auto ones = [&](Dims* d) {
      if (d->empty()) d->assign(r, 1);
    };
    ones(&op.strides);
    ones(&op.base_dilations);
    ones(&op.window_dilations);
    if (op.pad_low.size() == 1 && op.pad_high.size() == 1 && op.pad_high[0] == -(op.pad_low[0] + 1)) {
      op.pad_high.assign(r, op.pad_low[0]);
      op.pad_low.assign(r, op.pad_low[0]);
    }
    if (op.pad_low.empty()) op.pad_low.assign(r, 0);
    if (op.pad_high.empty()) op.pad_high.assign(r, 0);
  }

  // Deferred pieces that need the result type.
  if (have_dense) {
    size_t save = p_;
    p_ = dense_pos;
    parse_dense(sig_outputs[0], &op);
    p_ = save;
  }
  size_t ap = op.name.find("|applies:");
  if (ap != std::string::npos) {
    std::string m = op.name.substr(ap + 9);
    op.name = op.name.substr(0, ap);
    // One region per reduce: params (acc..., x...) with scalar init types.
    Region region;
    const size_t n_in = op.operands.size() / 2;
    std::vector<int> accs, xs;
    for (size_t i = 0; i < n_in; ++i) {
      TensorType st{prog_.values[op.operands[n_in + i]].type.dtype, {}};
      accs.push_back(new_value(st, "%acc"));
    }
    for (size_t i = 0; i < n_in; ++i) {
      TensorType st{prog_.values[op.operands[n_in + i]].type.dtype, {}};
      xs.push_back(new_value(st, "%x"));
    }
    region.params = accs;
    region.params.insert(region.params.end(), xs.begin(), xs.end());
    Op body;
    lookup_op(m, &body.kind);
    body.name = "stablehlo." + m;
    std::vector<int> rets;
    for (size_t i = 0; i < n_in; ++i) {
      Op b = body;
      b.operands = {accs[i], xs[i]};
      b.results = {new_value(prog_.values[accs[i]].type, "%r")};
      rets.push_back(b.results[0]);
      region.ops.push_back(b);
    }
    Op ret;
    ret.kind = OpKind::kReturn;
    ret.name = "return";
    ret.operands = rets;
    region.ops.push_back(ret);
    op.regions.push_back(std::move(region));
  }
  if (op.kind == OpKind::kDotGeneral && op.name == "stablehlo.dot") {
    // Plain dot: contract lhs last dim with rhs first dim.
    const TensorType& lt = prog_.values[op.operands[0]].type;
    op.lhs_contract = {lt.rank() - 1};
    op.rhs_contract = {0};
    op.name = "stablehlo.dot_general";
  }
  return op;
}

}  // namespace

Program parse_stablehlo(const std::string& text) {
  if (text.size() >= 4 && text.compare(0, 4, "ML\xef" "R") == 0) {
    fail(Code::kUnimplemented,
         "program is MLIR bytecode (VHLO portable artifact); this host has no MLIR "
         "library to deserialize it. Pass the textual StableHLO module instead.");
  }
  Parser parser(text);
  return parser.run();
}

}  // namespace pjrtx
