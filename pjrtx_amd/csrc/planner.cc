// Fusion planner implementation. See planner.h for the contract.
#include "kernels/dot.h"
#include "planner.h"
#include "sort_op.h"

#include <algorithm>
#include <cstring>
#include <cstdio>
#include <functional>
#include <queue>
#include <sstream>

namespace pjrtx {

const char* reducer_name(ReducerKind k) {
  switch (k) {
    case ReducerKind::kSum: return "sum";
    case ReducerKind::kProd: return "prod";
    case ReducerKind::kMax: return "max";
    case ReducerKind::kMin: return "min";
    case ReducerKind::kAnd: return "and";
    case ReducerKind::kOr: return "or";
    case ReducerKind::kArgMax: return "argmax";
    case ReducerKind::kArgMin: return "argmin";
  }
  return "?";
}

const char* lib_kind_name(LibKind k) {
  switch (k) {
    case LibKind::kCopy: return "copy";
    case LibKind::kDot: return "dot_general";
    case LibKind::kGather: return "gather";
    case LibKind::kScatter: return "scatter";
    case LibKind::kDynamicSlice: return "dynamic_slice";
    case LibKind::kDynamicUpdateSlice: return "dynamic_update_slice";
    case LibKind::kConcatenate: return "concatenate";
    case LibKind::kPad: return "pad";
    case LibKind::kAttention: return "attention";
    case LibKind::kDotGroup: return "dot_group";
    case LibKind::kWhile: return "while";
    case LibKind::kSort: return "sort";
    case LibKind::kReduceWindow: return "reduce_window";
  }
  return "?";
}

ReducerKind classify_reducer(const Program& prog, const Op& op) {
  PJRTX_CHECK(op.regions.size() == 1, Code::kInvalidArgument, "reduce needs exactly one region");
  const Region& r = op.regions[0];
  const size_t n = op.results.size();
  if (n == 2) {
    // (values, indices) with a compare of the two value block arguments.
    const int v_acc = r.params[0], v_x = r.params[2];
    bool has_select = false;
    int dir = 0;  // +1 argmax, -1 argmin
    for (const Op& b : r.ops) {
      if (b.kind == OpKind::kSelect) has_select = true;
      if (b.kind == OpKind::kCompare && b.operands.size() == 2) {
        const bool vv = (b.operands[0] == v_acc && b.operands[1] == v_x) ||
                        (b.operands[0] == v_x && b.operands[1] == v_acc);
        if (vv && (b.cmp_dir == CmpDir::kGT || b.cmp_dir == CmpDir::kGE)) dir = dir ? dir : 1;
        if (vv && (b.cmp_dir == CmpDir::kLT || b.cmp_dir == CmpDir::kLE)) dir = dir ? dir : -1;
      }
    }
    const DType vt = prog.type(op.results[0]).dtype;
    const DType it = prog.type(op.results[1]).dtype;
    PJRTX_CHECK(has_select && dir != 0 && dtype_is_float(vt) &&
                    (it == DType::kS32 || it == DType::kS64 || it == DType::kU32),
                Code::kUnimplemented,
                "two-result reduce is supported only as argmax/argmin over float values with "
                "s32/s64/u32 indices");
    return dir > 0 ? ReducerKind::kArgMax : ReducerKind::kArgMin;
  }
  PJRTX_CHECK(n == 1, Code::kUnimplemented, "reduce with more than two results is not supported");
  // Single-result: body must be one binary op of the two block args.
  int kind_op = -1;
  for (size_t i = 0; i < r.ops.size(); ++i) {
    if (r.ops[i].kind != OpKind::kReturn) {
      PJRTX_CHECK(kind_op < 0, Code::kUnimplemented, "reduce region with more than one op is not supported");
      kind_op = static_cast<int>(i);
    }
  }
  PJRTX_CHECK(kind_op >= 0, Code::kUnimplemented, "empty reduce region");
  const Op& b = r.ops[kind_op];
  const DType t = prog.type(op.results[0]).dtype;
  switch (b.kind) {
    case OpKind::kAdd: return t == DType::kPred ? ReducerKind::kOr : ReducerKind::kSum;
    case OpKind::kMultiply: return t == DType::kPred ? ReducerKind::kAnd : ReducerKind::kProd;
    case OpKind::kMaximum: return ReducerKind::kMax;
    case OpKind::kMinimum: return ReducerKind::kMin;
    case OpKind::kAnd: return ReducerKind::kAnd;
    case OpKind::kOr: return ReducerKind::kOr;
    default:
      fail(Code::kUnimplemented, std::string("unsupported reduce region op ") + op_kind_name(b.kind));
  }
}

// reduce_window forms the library kernel runs (kernels/reduce_window.hip):
// one operand with a sum / product / max / min region, or two operands
// (values, indices) with an argmax / argmin pair region (the reference's
// max-pool-with-indices form, lowering_reduction.zig:96-140); any base
// dilation, window dilation and stride >= 1, padding of either sign, rank
// <= 8. Anything else fails closed at compile time (the reference accepts
// sum and max, and the max pair, with base dilation 1, api.cc:4324-4360,
// 4437-4480).
void check_reduce_window_supported(const Program& prog, const Op& op) {
  const size_t n = op.results.size();
  PJRTX_CHECK((n == 1 || n == 2) && op.operands.size() == 2 * n, Code::kUnimplemented,
              "reduce_window: one operand, or two (values and indices), are supported");
  const ReducerKind k = classify_reducer(prog, op);
  if (n == 1)
    PJRTX_CHECK(k == ReducerKind::kSum || k == ReducerKind::kProd || k == ReducerKind::kMax || k == ReducerKind::kMin,
                Code::kUnimplemented, "reduce_window: the region must be add, multiply, maximum or minimum");
  else
    PJRTX_CHECK(k == ReducerKind::kArgMax || k == ReducerKind::kArgMin, Code::kUnimplemented,
                "reduce_window: a two-operand region must be an argmax / argmin pair selection");
  const TensorType& in = prog.type(op.operands[0]);
  const TensorType& out = prog.type(op.results[0]);
  const size_t r = in.dims.size();
  PJRTX_CHECK(r >= 1 && r <= 8, Code::kUnimplemented, "reduce_window: rank must be 1..8");
  PJRTX_CHECK(op.sizes.size() == r && op.strides.size() == r && op.base_dilations.size() == r &&
                  op.window_dilations.size() == r && op.pad_low.size() == r && op.pad_high.size() == r,
              Code::kInvalidArgument, "reduce_window: window attributes do not match the operand rank");
  const DType t = in.dtype;
  if (n == 1) {
    PJRTX_CHECK(t == DType::kF32 || t == DType::kF64 || t == DType::kBF16 || t == DType::kF16 || t == DType::kS32 ||
                    t == DType::kS64,
                Code::kUnimplemented, std::string("reduce_window: element type ") + dtype_name(t) + " is not supported");
  } else {
    const TensorType& ix = prog.type(op.operands[1]);
    const TensorType& oi = prog.type(op.results[1]);
    PJRTX_CHECK(t == DType::kF32 || t == DType::kF64 || t == DType::kBF16 || t == DType::kF16, Code::kUnimplemented,
                std::string("reduce_window: value type ") + dtype_name(t) + " is not supported");
    PJRTX_CHECK(ix.dtype == DType::kS32 || ix.dtype == DType::kU32 || ix.dtype == DType::kS64, Code::kUnimplemented,
                std::string("reduce_window: index type ") + dtype_name(ix.dtype) + " is not supported");
    PJRTX_CHECK(ix.dims == in.dims && oi.dims == out.dims && oi.dtype == ix.dtype && out.dtype == t &&
                    prog.type(op.operands[2]).dtype == t && prog.type(op.operands[3]).dtype == ix.dtype,
                Code::kInvalidArgument, "reduce_window: values and indices must have matching shapes and types");
  }
  for (size_t d = 0; d < r; ++d) {
    PJRTX_CHECK(op.sizes[d] >= 1 && op.strides[d] >= 1 && op.window_dilations[d] >= 1 && op.base_dilations[d] >= 1,
                Code::kUnimplemented, "reduce_window: windows, strides and dilations must be positive");
    const int64_t dilated = in.dims[d] == 0 ? 0 : (in.dims[d] - 1) * op.base_dilations[d] + 1;
    const int64_t padded = op.pad_low[d] + dilated + op.pad_high[d];
    const int64_t span = (op.sizes[d] - 1) * op.window_dilations[d] + 1;
    const int64_t want = padded < span ? 0 : (padded - span) / op.strides[d] + 1;
    PJRTX_CHECK(out.dims[d] == want, Code::kInvalidArgument, "reduce_window: result shape does not match the window");
  }
}

namespace {

bool is_splat_constant(const Program& prog, const Op& op) {
  return op.kind == OpKind::kConstant && (op.splat || prog.type(op.results[0]).elements() == 1);
}

// A concatenate of a few operands fuses as an index select (each operand
// read at a clamped coordinate, the result picked by range); a long operand
// list runs as box copies instead.
constexpr size_t kMaxFusedConcatOperands = 8;

bool fusible_concat(const Op& op) {
  return op.kind == OpKind::kConcatenate && op.operands.size() <= kMaxFusedConcatOperands;
}

// Relative cost of recomputing an op per element, for the recompute-vs-
// materialize decision: trigonometric ops (argument reduction) and pow are
// much dearer than an add; exp/log-type ops somewhat.
int op_cost(OpKind k) {
  switch (k) {
    case OpKind::kSine: case OpKind::kCosine: case OpKind::kTan: case OpKind::kAtan2: case OpKind::kPower:
      return 12;
    case OpKind::kExp: case OpKind::kExpm1: case OpKind::kLog: case OpKind::kLog1p: case OpKind::kLogistic:
    case OpKind::kTanh: case OpKind::kCbrt: case OpKind::kDivide: case OpKind::kRemainder:
      return 4;
    case OpKind::kReducePrecision:
      return 2;
    default:
      return 1;
  }
}

bool is_library(const Op& op) {
  const OpKind k = op.kind;
  return k == OpKind::kDotGeneral || k == OpKind::kGather || k == OpKind::kScatter ||
         k == OpKind::kDynamicSlice || k == OpKind::kDynamicUpdateSlice ||
         (k == OpKind::kConcatenate && !fusible_concat(op)) || k == OpKind::kPad || k == OpKind::kAttention ||
         k == OpKind::kWhile || k == OpKind::kSort || k == OpKind::kTopK || k == OpKind::kReduceWindow;
}

LibKind lib_kind_of(OpKind k) {
  switch (k) {
    case OpKind::kDotGeneral: return LibKind::kDot;
    case OpKind::kGather: return LibKind::kGather;
    case OpKind::kScatter: return LibKind::kScatter;
    case OpKind::kAttention: return LibKind::kAttention;
    case OpKind::kDynamicSlice: return LibKind::kDynamicSlice;
    case OpKind::kDynamicUpdateSlice: return LibKind::kDynamicUpdateSlice;
    case OpKind::kConcatenate: return LibKind::kConcatenate;
    case OpKind::kPad: return LibKind::kPad;
    case OpKind::kWhile: return LibKind::kWhile;
    case OpKind::kSort:
    case OpKind::kTopK: return LibKind::kSort;
    case OpKind::kReduceWindow: return LibKind::kReduceWindow;
    default: return LibKind::kCopy;
  }
}

namespace {

// The value of a scalar integer constant op.
bool scalar_int_literal(const Program& prog, const Op& op, int64_t* out) {
  if (op.kind != OpKind::kConstant || op.results.size() != 1) return false;
  const TensorType& t = prog.type(op.results[0]);
  if (t.rank() != 0 || op.literal.size() < dtype_size(t.dtype)) return false;
  const uint8_t* b = op.literal.data();
  switch (t.dtype) {
    case DType::kS8: *out = static_cast<int8_t>(b[0]); return true;
    case DType::kU8: *out = b[0]; return true;
    case DType::kS16: { int16_t v; std::memcpy(&v, b, 2); *out = v; return true; }
    case DType::kU16: { uint16_t v; std::memcpy(&v, b, 2); *out = v; return true; }
    case DType::kS32: { int32_t v; std::memcpy(&v, b, 4); *out = v; return true; }
    case DType::kU32: { uint32_t v; std::memcpy(&v, b, 4); *out = v; return true; }
    case DType::kS64: { int64_t v; std::memcpy(&v, b, 8); *out = v; return true; }
    default: return false;
  }
}

// The integer constant a value holds, looking through the ops of `ops`.
bool value_int_constant(const Program& prog, const std::vector<Op>& ops, int v, int64_t* out) {
  for (const Op& op : ops)
    if (!op.results.empty() && op.results[0] == v) return scalar_int_literal(prog, op, out);
  return false;
}

// Iteration count of `while (i CMP bound) { ...; i += step }` when the
// counter's start, the bound and the step are integer constants (JAX's
// fori_loop / scan form), else -1. `outer` holds the ops that define the
// loop's operands.
int64_t static_trip_count(const Program& prog, const std::vector<Op>& outer, const Op& op) {
  if (op.regions.size() != 2 || op.sizes.empty()) return -1;
  const Region& cond = op.regions[0];
  const Region& body = op.regions[1];
  const size_t n_state = static_cast<size_t>(op.sizes[0]);
  // The cond: constants, one compare, and the return of its result.
  if (cond.ops.empty() || cond.ops.back().kind != OpKind::kReturn || cond.ops.back().operands.size() != 1) return -1;
  const Op* cmpp = nullptr;
  for (size_t i = 0; i + 1 < cond.ops.size(); ++i) {
    const Op& o = cond.ops[i];
    if (o.kind == OpKind::kConstant) continue;
    if (o.kind != OpKind::kCompare || cmpp) return -1;
    cmpp = &o;
  }
  if (!cmpp) return -1;
  const Op& cmp = *cmpp;
  if (cmp.results.size() != 1 || cmp.results[0] != cond.ops.back().operands[0]) return -1;
  if (cmp.cmp_dir != CmpDir::kLT && cmp.cmp_dir != CmpDir::kLE && cmp.cmp_dir != CmpDir::kGT &&
      cmp.cmp_dir != CmpDir::kGE)
    return -1;
  // The counter: a state element compared on the left.
  size_t ci = n_state;
  for (size_t i = 0; i < n_state; ++i)
    if (cond.params[i] == cmp.operands[0]) ci = i;
  if (ci == n_state) return -1;
  // The bound: a captured constant, or a state element the body passes
  // through unchanged whose initial value is constant.
  int64_t bound = 0, start = 0, step = 0;
  const int bv = cmp.operands[1];
  bool have_bound = value_int_constant(prog, cond.ops, bv, &bound) || value_int_constant(prog, outer, bv, &bound);
  if (!have_bound) {
    const Op& bret = body.ops.back();
    for (size_t j = 0; j < n_state && !have_bound; ++j)
      if (cond.params[j] == bv && bret.kind == OpKind::kReturn && j < bret.operands.size() &&
          bret.operands[j] == body.params[j])
        have_bound = value_int_constant(prog, outer, op.operands[j], &bound);
  }
  if (!have_bound || !value_int_constant(prog, outer, op.operands[ci], &start)) return -1;
  // The step: the body returns counter + constant (or constant + counter).
  const Op& ret = body.ops.back();
  if (ret.kind != OpKind::kReturn || ci >= ret.operands.size()) return -1;
  const int next = ret.operands[ci];
  bool have_step = false;
  for (const Op& o : body.ops) {
    if (o.results.empty() || o.results[0] != next) continue;
    if (o.kind != OpKind::kAdd || o.operands.size() != 2) return -1;
    const int other = o.operands[0] == body.params[ci] ? o.operands[1]
                      : o.operands[1] == body.params[ci] ? o.operands[0] : -1;
    if (other < 0) return -1;
    have_step = value_int_constant(prog, body.ops, other, &step) || value_int_constant(prog, outer, other, &step);
  }
  if (!have_step || step == 0) return -1;
  // Counts of at most 2^31 iterations; the counter must not wrap on the way.
  const CmpDir d = cmp.cmp_dir;
  int64_t trips = 0;
  if (d == CmpDir::kLT || d == CmpDir::kLE) {
    const int64_t last = d == CmpDir::kLT ? bound - 1 : bound;
    if (step < 0) return start > last ? 0 : -1;
    trips = start > last ? 0 : (last - start) / step + 1;
  } else {
    const int64_t last = d == CmpDir::kGT ? bound + 1 : bound;
    if (step > 0) return start < last ? 0 : -1;
    trips = start < last ? 0 : (start - last) / (-step) + 1;
  }
  if (trips > (int64_t(1) << 31)) return -1;
  const TensorType& ct = prog.type(op.operands[ci]);
  if (ct.dtype == DType::kS32 && (start + (trips + 1) * step > INT32_MAX || start + (trips + 1) * step < INT32_MIN))
    return -1;
  return trips;
}

}  // namespace

class Planner {
 public:
  Planner(const Program& prog, const PlanOptions& opts) : prog_(prog), opts_(opts) {}
  Plan run();

 private:
  const Program& prog_;
  const PlanOptions& opts_;
  Plan plan_;
  std::map<int, int>& producer_ = plan_.producer;
  std::map<int, std::vector<int>> users_;  // value -> ops using it
  std::set<int> outputs_;
  std::set<int>& mat_ = plan_.materialized;

  bool fusible_op(const Op& op) const {
    return op_is_elementwise(op.kind) || op_is_view(op.kind) || fusible_concat(op) || is_splat_constant(prog_, op);
  }
  void decide_materialization();
  // Collects the fused ops reachable backward from `roots` without crossing
  // materialized values. Fills ops (sorted) and inputs.
  // `roots_are_outputs`: the roots are the values this step produces (their
  // producers are fused even though the roots are materialized); otherwise
  // a materialized root is read as an input.
  void closure(const std::vector<int>& roots, std::vector<int>* ops, std::vector<int>* inputs,
               bool roots_are_outputs = true) const;
  void build_steps(std::vector<Step>* steps);
  int order_preserving_source(int v) const;
  void merge_siblings(std::vector<Step>* steps);
  void merge_epilogues(std::vector<Step>* steps);
  void merge_dot_residuals(std::vector<Step>* steps);
  void merge_sibling_loops(std::vector<Step>* steps);
  void absorb_window_updates();
  void fuse_row_chains(std::vector<Step>* steps);
  bool row_uses_ok(const Step& x, const std::set<int>& produced, const Dims& shape, size_t nkept) const;
  void shape_row_fused(Step* s);
  void schedule(std::vector<Step>* steps);
  void liveness();
  void shape_reduce(Step* s);
  void shape_loop(Step* s);
};

// Total inlined ops below which an expensive value is recomputed under a
// broadcast instead of being materialized.
constexpr int64_t kRecomputeBroadcastOps = int64_t(1) << 20;

void Planner::decide_materialization() {
  for (int p : prog_.params) mat_.insert(p);
  for (int r : prog_.results) outputs_.insert(r);
  for (size_t i = 0; i < prog_.ops.size(); ++i) {
    const Op& op = prog_.ops[i];
    for (int v : op.results) producer_[v] = static_cast<int>(i);
    for (int v : op.operands) users_[v].push_back(static_cast<int>(i));
  }
  std::map<int, int> cost;  // inlined op count of a non-materialized value
  // Materialized buffers that recomputing a non-materialized value reads.
  std::map<int, std::set<int>> reads;
  for (size_t i = 0; i < prog_.ops.size(); ++i) {
    const Op& op = prog_.ops[i];
    if (op.kind == OpKind::kReturn) {
      for (int v : op.operands) mat_.insert(v);
      continue;
    }
    if (op.kind == OpKind::kConstant) {
      if (!is_splat_constant(prog_, op)) {
        mat_.insert(op.results[0]);
        plan_.constants.push_back(op.results[0]);
      }
      cost[op.results[0]] = 0;
      continue;
    }
    if (op.kind == OpKind::kReduce) {
      const size_t n = op.results.size();
      for (size_t k = 0; k < n; ++k) {
        // Init values are scalars: literals when splat constants, else read.
        int init = op.operands[n + k];
        auto pi = producer_.find(init);
        const bool lit = pi != producer_.end() && is_splat_constant(prog_, prog_.ops[pi->second]);
        if (!lit) mat_.insert(init);
      }
      for (int v : op.results) mat_.insert(v);
      continue;
    }
    if (is_library(op)) {
      for (int v : op.operands) mat_.insert(v);
      for (int v : op.results) mat_.insert(v);
      continue;
    }
    PJRTX_CHECK(fusible_op(op), Code::kUnimplemented,
                std::string("op not supported by the HIP backend: ") + op.name);
    // Elementwise / view op.
    int c = (op_is_view(op.kind) || op.kind == OpKind::kConcatenate) ? 0 : op_cost(op.kind);
    for (int v : op.operands) {
      if (!mat_.count(v)) c += cost[v];
    }
    if (op.kind == OpKind::kBroadcastInDim && !op.operands.empty()) {
      const int u = op.operands[0];
      const bool expands = prog_.type(op.results[0]).elements() > prog_.type(u).elements();
      if (expands && !mat_.count(u) && cost[u] > 8 && prog_.type(u).elements() > 1 &&
          prog_.type(op.results[0]).elements() * cost[u] > kRecomputeBroadcastOps) {
        // Avoid recomputing an expensive value once per broadcast element
        // (unless the whole broadcast is small: a decode step's RoPE tables,
        // recomputed per head, cost less than the launch that would hold them).
        mat_.insert(u);
        c -= cost[u];
      }
    }
    std::set<int> rd;
    for (int u : op.operands) {
      if (mat_.count(u)) {
        rd.insert(u);
      } else {
        auto it = reads.find(u);
        if (it != reads.end()) rd.insert(it->second.begin(), it->second.end());
      }
    }
    // A value read by several kernels is recomputed in each unless that
    // costs too many ops, or reads half again as many bytes as the value
    // (a residual stream x + f(x) + g(...) would otherwise re-read every
    // earlier layer's output in every later kernel).
    const int v = op.results[0];
    int64_t rbytes = 0;
    for (int w : rd) rbytes += prog_.type(w).bytes();
    // Small values (the whole recomputation under 2^20 ops) are recomputed
    // whatever their per-element cost.
    const bool costly = c > opts_.recompute_limit &&
                        prog_.type(v).elements() * c * static_cast<int64_t>(users_[v].size()) > kRecomputeBroadcastOps;
    if (users_[v].size() > 1 && !is_splat_constant(prog_, op) &&
        (costly || (rd.size() > 1 && 2 * rbytes > 3 * prog_.type(v).bytes()))) {
      mat_.insert(v);
      c = 0;
      rd.clear();
    }
    cost[v] = c;
    reads[v] = std::move(rd);
  }
  // A splat constant that needs a buffer (library operand, program output,
  // non-literal reduce init) is uploaded once at load, like any constant.
  for (const Op& op : prog_.ops) {
    if (op.kind == OpKind::kConstant && is_splat_constant(prog_, op) && mat_.count(op.results[0]))
      plan_.constants.push_back(op.results[0]);
  }
}

void Planner::closure(const std::vector<int>& roots, std::vector<int>* ops, std::vector<int>* inputs,
                      bool roots_are_outputs) const {
  std::set<int> seen_ops, seen_inputs;
  std::function<void(int, bool)> visit = [&](int v, bool is_root) {
    if (!is_root && mat_.count(v)) {
      if (seen_inputs.insert(v).second) inputs->push_back(v);
      return;
    }
    auto pi = producer_.find(v);
    if (pi == producer_.end()) {  // parameter
      if (seen_inputs.insert(v).second) inputs->push_back(v);
      return;
    }
    const int oi = pi->second;
    if (!seen_ops.insert(oi).second) return;
    const Op& op = prog_.ops[oi];
    for (int u : op.operands) visit(u, false);
  };
  for (int r : roots) visit(r, roots_are_outputs);
  ops->assign(seen_ops.begin(), seen_ops.end());  // std::set is sorted: program order
}

// True if `op` is a view whose result has its operand's elements in the same
// row-major order.
static bool keeps_row_major_order(const Program& prog, const Op& op) {
  if (op.operands.empty()) return false;
  const TensorType& in = prog.type(op.operands[0]);
  const TensorType& out = prog.type(op.results[0]);
  if (in.elements() != out.elements()) return false;
  if (op.kind == OpKind::kReshape) return true;
  if (op.kind == OpKind::kBroadcastInDim) return std::is_sorted(op.dims.begin(), op.dims.end());
  if (op.kind == OpKind::kTranspose) {
    int64_t last = -1;
    for (int64_t d : op.dims) {  // result dim i reads operand dim op.dims[i]
      if (in.dims[d] == 1) continue;
      if (d < last) return false;
      last = d;
    }
    return true;
  }
  return false;
}

int Planner::order_preserving_source(int v) const {
  int cur = v;
  for (int hops = 0; hops < 64; ++hops) {
    auto pi = producer_.find(cur);
    if (pi == producer_.end()) return -1;
    const Op& op = prog_.ops[pi->second];
    if (!keeps_row_major_order(prog_, op)) return -1;
    const int u = op.operands[0];
    if (mat_.count(u)) return u;
    cur = u;
  }
  return -1;
}

// Decode-shaped dot (the reference's dot group candidates,
// executable_metal_graph_lowering_fusion.zig:394-424): [M, K] x [K, N] with
// M <= 4, 16-bit operands.
static bool group_candidate(const Program& prog, const Op& op) {
  if (op.kind != OpKind::kDotGeneral || op.operands.size() != 2) return false;
  const TensorType& l = prog.type(op.operands[0]);
  const TensorType& r = prog.type(op.operands[1]);
  return l.rank() == 2 && r.rank() == 2 && op.lhs_batch.empty() && op.rhs_batch.empty() &&
         op.lhs_contract == Dims{1} && op.rhs_contract == Dims{0} && l.dims[0] <= 4 && l.dtype == r.dtype &&
         (l.dtype == DType::kBF16 || l.dtype == DType::kF16);
}

void Planner::build_steps(std::vector<Step>* steps) {
  // Dots sharing one LHS, each RHS defined before the first of them (so no
  // member can depend on another), up to 4 per group.
  std::map<int, std::vector<int>> groups;
  std::set<int> grouped;
  if (opts_.group_dots) {
    for (size_t i = 0; i < prog_.ops.size(); ++i) {
      const Op& a = prog_.ops[i];
      if (grouped.count(static_cast<int>(i)) || !group_candidate(prog_, a)) continue;
      std::vector<int> members = {static_cast<int>(i)};
      for (size_t j = i + 1; j < prog_.ops.size() && members.size() < 4; ++j) {
        const Op& b = prog_.ops[j];
        if (grouped.count(static_cast<int>(j)) || !group_candidate(prog_, b) || b.operands[0] != a.operands[0]) continue;
        if (prog_.type(b.results[0]).dtype != prog_.type(a.results[0]).dtype) continue;
        auto pr = producer_.find(b.operands[1]);
        if (pr != producer_.end() && pr->second >= static_cast<int>(i)) continue;
        members.push_back(static_cast<int>(j));
      }
      if (members.size() < 2) continue;
      groups[static_cast<int>(i)] = members;
      grouped.insert(members.begin(), members.end());
    }
  }
  for (size_t i = 0; i < prog_.ops.size(); ++i) {
    const Op& op = prog_.ops[i];
    if (op.kind == OpKind::kReturn || op.kind == OpKind::kConstant) continue;  // constants: literals or resident
    if (grouped.count(static_cast<int>(i))) {
      auto g = groups.find(static_cast<int>(i));
      if (g == groups.end()) continue;  // a later member: emitted with its group
      Step s;
      s.kind = StepKind::kLibrary;
      s.lib = LibKind::kDotGroup;
      s.lib_op = static_cast<int>(i);
      s.group_ops = g->second;
      s.inputs.push_back(op.operands[0]);
      for (int m : g->second) {
        s.inputs.push_back(prog_.ops[m].operands[1]);
        s.outputs.push_back(prog_.ops[m].results[0]);
      }
      steps->push_back(std::move(s));
      continue;
    }
    if (op.kind == OpKind::kReduce) {
      Step s;
      s.kind = StepKind::kReduce;
      ReduceSpec rs;
      rs.op_index = static_cast<int>(i);
      rs.kind = classify_reducer(prog_, op);
      const size_t n = op.results.size();
      rs.inputs.assign(op.operands.begin(), op.operands.begin() + n);
      rs.inits.assign(op.operands.begin() + n, op.operands.end());
      rs.results = op.results;
      s.reduces.push_back(rs);
      s.reduce_operand_shape = prog_.type(rs.inputs[0]).dims;
      s.reduce_dims = op.dims;
      std::sort(s.reduce_dims.begin(), s.reduce_dims.end());
      std::vector<int> roots = rs.inputs;
      std::vector<int> init_inputs;
      for (int v : rs.inits) roots.push_back(v);
      closure(roots, &s.ops, &s.inputs, /*roots_are_outputs=*/false);
      s.outputs = op.results;
      steps->push_back(std::move(s));
      continue;
    }
    if (is_library(op)) {
      Step s;
      s.kind = StepKind::kLibrary;
      s.lib = lib_kind_of(op.kind);
      s.lib_op = static_cast<int>(i);
      s.inputs = op.operands;
      s.outputs = op.results;
      if (op.kind == OpKind::kWhile) s.while_trips = static_trip_count(prog_, prog_.ops, op);
      if (s.lib == LibKind::kSort) check_sort_supported(prog_, op);
      if (s.lib == LibKind::kReduceWindow) check_reduce_window_supported(prog_, op);
      steps->push_back(std::move(s));
      continue;
    }
    // Fusible op: a loop step only if its result is materialized.
    if (op.results.empty() || !mat_.count(op.results[0])) continue;
    const int v = op.results[0];
    Step s;
    // A chain of views that keeps the row-major order (reshapes, unit-dim
    // broadcasts, transposes that only move size-1 dims) over a materialized
    // value is that value's buffer under another type: no kernel.
    const int src = order_preserving_source(v);
    if (src >= 0) {
      s.kind = StepKind::kAlias;
      s.inputs = {src};
      s.outputs = {v};
      s.lib_op = static_cast<int>(i);
      steps->push_back(std::move(s));
      continue;
    }
    s.kind = StepKind::kLoop;
    closure({v}, &s.ops, &s.inputs);
    s.outputs = {v};
    s.loop_shape = prog_.type(v).dims;
    steps->push_back(std::move(s));
  }
}

// Producers of each materialized value, for dependency tests.
static std::map<int, int> value_to_step(const std::vector<Step>& steps) {
  std::map<int, int> m;
  for (size_t i = 0; i < steps.size(); ++i)
    for (int v : steps[i].outputs) m[v] = static_cast<int>(i);
  return m;
}

static bool depends_on(const std::vector<Step>& steps, const std::map<int, int>& v2s, int from, int target) {
  // true if step `from` (transitively) reads an output of step `target`.
  std::vector<int> stack = {from};
  std::set<int> seen;
  while (!stack.empty()) {
    int s = stack.back();
    stack.pop_back();
    if (!seen.insert(s).second) continue;
    for (int v : steps[s].inputs) {
      auto it = v2s.find(v);
      if (it == v2s.end()) continue;
      if (it->second == target) return true;
      stack.push_back(it->second);
    }
  }
  return false;
}

void Planner::merge_siblings(std::vector<Step>* steps) {
  bool changed = true;
  while (changed) {
    changed = false;
    auto v2s = value_to_step(*steps);
    for (size_t a = 0; a < steps->size() && !changed; ++a) {
      Step& A = (*steps)[a];
      if (A.kind != StepKind::kReduce) continue;
      for (size_t b = a + 1; b < steps->size() && !changed; ++b) {
        Step& B = (*steps)[b];
        if (B.kind != StepKind::kReduce) continue;
        if (A.reduce_operand_shape != B.reduce_operand_shape || A.reduce_dims != B.reduce_dims) continue;
        if (depends_on(*steps, v2s, static_cast<int>(a), static_cast<int>(b)) ||
            depends_on(*steps, v2s, static_cast<int>(b), static_cast<int>(a)))
          continue;
        // Merge B into A.
        for (auto& r : B.reduces) A.reduces.push_back(r);
        std::set<int> ops(A.ops.begin(), A.ops.end());
        ops.insert(B.ops.begin(), B.ops.end());
        A.ops.assign(ops.begin(), ops.end());
        for (int v : B.inputs)
          if (std::find(A.inputs.begin(), A.inputs.end(), v) == A.inputs.end()) A.inputs.push_back(v);
        for (int v : B.outputs) A.outputs.push_back(v);
        steps->erase(steps->begin() + b);
        changed = true;
      }
    }
  }
}

// True when run_dot_general takes the one-pass GEMV for this dot (shape
// conditions; buffer alignment is checked again at run time).
static bool one_pass_gemv(const Program& prog, const Op& op) {
  if (op.kind != OpKind::kDotGeneral || op.operands.size() != 2) return false;
  const TensorType& l = prog.type(op.operands[0]);
  const TensorType& r = prog.type(op.operands[1]);
  if (l.rank() != 2 || r.rank() != 2 || !op.lhs_batch.empty() || op.lhs_contract != Dims{1} ||
      op.rhs_contract != Dims{0} || l.dtype != r.dtype || (l.dtype != DType::kBF16 && l.dtype != DType::kF16))
    return false;
  const int64_t M = l.dims[0], K = l.dims[1], N = r.dims[1];
  if (M < 1 || M > 4 || K % 8 != 0 || N % 8 != 0 || N >= (int64_t(1) << 30)) return false;
  GemvGroup one;
  one.count = 1;
  one.m[0].N = static_cast<int>(N);
  return gemv_wide_fits(static_cast<int>(M), static_cast<int>(K), gemv_wide_tiles(one));
}

// Elementwise steps over the same shape that do not depend on each other
// become one multi-output kernel (RoPE of q and of k; the cos and sin
// tables): one launch, and inputs they share are read once per element.
// A later step joins an earlier one only when all its inputs are produced
// before that step, so it can run there.
void Planner::merge_sibling_loops(std::vector<Step>* steps) {
  constexpr size_t kMaxMergedOutputs = 8;
  auto v2s = value_to_step(*steps);
  for (size_t a = 0; a < steps->size(); ++a) {
    if ((*steps)[a].kind != StepKind::kLoop) continue;
    for (size_t b = a + 1; b < steps->size(); ++b) {
      Step& A = (*steps)[a];
      const Step& B = (*steps)[b];
      if (B.kind != StepKind::kLoop || B.loop_shape != A.loop_shape ||
          A.outputs.size() + B.outputs.size() > kMaxMergedOutputs)
        continue;
      bool early = true;
      for (int v : B.inputs) {
        auto it = v2s.find(v);
        if (it != v2s.end() && it->second >= static_cast<int>(a)) early = false;
      }
      if (!early) continue;
      std::set<int> ops(A.ops.begin(), A.ops.end());
      ops.insert(B.ops.begin(), B.ops.end());
      A.ops.assign(ops.begin(), ops.end());
      for (int v : B.inputs)
        if (std::find(A.inputs.begin(), A.inputs.end(), v) == A.inputs.end()) A.inputs.push_back(v);
      A.outputs.insert(A.outputs.end(), B.outputs.begin(), B.outputs.end());
      steps->erase(steps->begin() + b);
      v2s = value_to_step(*steps);
      --b;
    }
  }
}

// add(dot, x) where the dot's only reader is that add: the dot step writes
// x + round(dot) directly (the GEMV's epilogue), one launch and one buffer
// fewer (a residual connection after an output or down projection).
void Planner::merge_dot_residuals(std::vector<Step>* steps) {
  std::map<int, int> readers;
  for (const Step& s : *steps)
    for (int v : s.inputs) readers[v]++;
  auto v2s = value_to_step(*steps);
  for (size_t g = 0; g < steps->size(); ++g) {
    Step& G = (*steps)[g];
    if (G.kind != StepKind::kLoop || G.outputs.size() != 1 || G.ops.size() != 1 || G.inputs.size() != 2) continue;
    const Op& add = prog_.ops[G.ops[0]];
    if (add.kind != OpKind::kAdd || add.results[0] != G.outputs[0]) continue;
    for (int side = 0; side < 2; ++side) {
      const int d = add.operands[side], x = add.operands[1 - side];
      if (d == x || !v2s.count(d) || readers[d] != 1 || outputs_.count(d)) continue;
      Step& D = (*steps)[v2s[d]];
      if (D.kind != StepKind::kLibrary || D.lib != LibKind::kDot || D.dot_add >= 0 || D.outputs.size() != 1) continue;
      const Op& dot = prog_.ops[D.lib_op];
      if (!one_pass_gemv(prog_, dot) || prog_.type(x).dims != prog_.type(d).dims ||
          prog_.type(x).dtype != prog_.type(d).dtype || prog_.type(G.outputs[0]).dtype != prog_.type(d).dtype)
        continue;
      D.dot_add = x;
      D.inputs.push_back(x);
      D.outputs = G.outputs;
      mat_.erase(d);
      steps->erase(steps->begin() + g);
      --g;
      break;
    }
    v2s = value_to_step(*steps);
  }
}

void Planner::merge_epilogues(std::vector<Step>* steps) {
  bool changed = true;
  while (changed) {
    changed = false;
    auto v2s = value_to_step(*steps);
    for (size_t g = 0; g < steps->size() && !changed; ++g) {
      Step& G = (*steps)[g];
      if (G.kind != StepKind::kLoop || G.outputs.size() != 1) continue;
      // Which reduce step feeds G?
      int rs = -1;
      bool ok = true;
      for (int v : G.inputs) {
        auto it = v2s.find(v);
        const bool scalar = prog_.type(v).elements() == 1;
        if (it != v2s.end() && (*steps)[it->second].kind == StepKind::kReduce) {
          if (rs >= 0 && rs != it->second) ok = false;
          rs = it->second;
        } else if (!scalar) {
          ok = false;
        }
      }
      if (!ok || rs < 0) continue;
      Step& R = (*steps)[rs];
      Dims out_dims;
      for (size_t d = 0; d < R.reduce_operand_shape.size(); ++d)
        if (!std::binary_search(R.reduce_dims.begin(), R.reduce_dims.end(), static_cast<int64_t>(d)))
          out_dims.push_back(R.reduce_operand_shape[d]);
      if (G.loop_shape != out_dims) continue;
      // Every access to an R output must be at the output index: no view op
      // may sit between an R output and G's root, except over literals.
      bool identity_only = true;
      for (int oi : G.ops) {
        const Op& op = prog_.ops[oi];
        if ((!op_is_view(op.kind) && op.kind != OpKind::kConcatenate) || op.kind == OpKind::kIota) continue;
        for (int u : op.operands) {
          auto pi = producer_.find(u);
          const bool literal = pi != producer_.end() && is_splat_constant(prog_, prog_.ops[pi->second]);
          if (!literal) identity_only = false;
        }
      }
      if (!identity_only) continue;
      // Merge G into R as epilogue.
      std::set<int> eops(R.epilogue_ops.begin(), R.epilogue_ops.end());
      eops.insert(G.ops.begin(), G.ops.end());
      R.epilogue_ops.assign(eops.begin(), eops.end());
      for (int v : G.inputs) {
        if (v2s.count(v) && v2s[v] == rs) continue;
        if (std::find(R.inputs.begin(), R.inputs.end(), v) == R.inputs.end()) R.inputs.push_back(v);
      }
      R.outputs.push_back(G.outputs[0]);
      steps->erase(steps->begin() + g);
      changed = true;
    }
  }
  // Raw reduce results that only feed epilogues no longer need a buffer.
  std::map<int, int> readers;
  for (const Step& s : *steps)
    for (int v : s.inputs) readers[v]++;
  for (Step& s : *steps) {
    if (s.kind != StepKind::kReduce || s.epilogue_ops.empty()) continue;
    std::vector<int> keep;
    for (int v : s.outputs) {
      const bool raw = std::any_of(s.reduces.begin(), s.reduces.end(), [&](const ReduceSpec& r) {
        return std::find(r.results.begin(), r.results.end(), v) != r.results.end();
      });
      if (raw && !outputs_.count(v) && readers[v] == 0) {
        mat_.erase(v);
        continue;
      }
      keep.push_back(v);
    }
    s.outputs = keep;
  }
}

// Every use of a value derived from an earlier phase must be at the current
// row: elementwise ops over the kept shape, and broadcasts of the kept shape
// onto the leading dims of the row operand.
bool Planner::row_uses_ok(const Step& x, const std::set<int>& produced, const Dims& shape, size_t nkept) const {
  const Dims kept(shape.begin(), shape.begin() + nkept);
  std::set<int> derived(produced.begin(), produced.end());
  std::vector<int> ops = x.ops;
  ops.insert(ops.end(), x.epilogue_ops.begin(), x.epilogue_ops.end());
  std::sort(ops.begin(), ops.end());
  for (int oi : ops) {
    const Op& op = prog_.ops[oi];
    bool uses = false;
    for (int u : op.operands) uses = uses || derived.count(u);
    if (!uses) continue;
    if (op.kind == OpKind::kBroadcastInDim) {
      if (prog_.type(op.operands[0]).dims != kept || prog_.type(op.results[0]).dims != shape) return false;
      for (size_t k = 0; k < op.dims.size(); ++k)
        if (op.dims[k] != static_cast<int64_t>(k)) return false;
      continue;
    }
    if (!op_is_elementwise(op.kind) || op.results.empty() || prog_.type(op.results[0]).dims != kept) return false;
    for (int u : op.operands)  // other operands: kept-shaped derived values or scalars
      if (!derived.count(u) && prog_.type(u).rank() != 0 && prog_.type(u).dims != kept) return false;
    derived.insert(op.results[0]);
  }
  return true;
}

void Planner::fuse_row_chains(std::vector<Step>* steps) {
  auto reduce_shape_ok = [&](const Step& r, Dims* shape, size_t* nkept, int64_t* row_len) {
    if (r.kind != StepKind::kReduce) return false;
    const Dims& sh = r.reduce_operand_shape;
    const size_t rank = sh.size(), nred = r.reduce_dims.size();
    if (nred == 0 || nred > rank) return false;
    for (size_t k = 0; k < nred; ++k)
      if (r.reduce_dims[k] != static_cast<int64_t>(rank - nred + k)) return false;
    int64_t len = 1;
    for (size_t d = rank - nred; d < rank; ++d) len *= sh[d];
    if (len < 32 || len > opts_.row_fuse_max || num_elements(sh) >= (int64_t(1) << 32)) return false;
    for (const ReduceSpec& rs : r.reduces)
      if (rs.kind == ReducerKind::kArgMax || rs.kind == ReducerKind::kArgMin) return false;
    *shape = sh;
    *nkept = rank - nred;
    *row_len = len;
    return true;
  };
  for (size_t a = 0; a < steps->size(); ++a) {
    Dims shape;
    size_t nkept = 0;
    int64_t row_len = 0;
    if (!reduce_shape_ok((*steps)[a], &shape, &nkept, &row_len)) continue;
    std::vector<size_t> group = {a};
    std::set<int> produced((*steps)[a].outputs.begin(), (*steps)[a].outputs.end());
    for (size_t b = a + 1; b < steps->size(); ++b) {
      const Step& x = (*steps)[b];
      bool dep = false;
      for (int v : x.inputs) dep = dep || produced.count(v);
      if (!dep) continue;
      Dims xs;
      size_t xk = 0;
      int64_t xl = 0;
      const bool red = reduce_shape_ok(x, &xs, &xk, &xl) && xs == shape && xk == nkept;
      const bool loop = x.kind == StepKind::kLoop && x.loop_shape == shape;
      if ((!red && !loop) || !row_uses_ok(x, produced, shape, nkept)) break;
      group.push_back(b);
      produced.insert(x.outputs.begin(), x.outputs.end());
      if (loop) break;  // the elementwise pass ends a chain
    }
    if (group.size() < 2) continue;
    // A later member may read a value that an unfused step in between
    // produces from an earlier member: then the chain cannot be one kernel.
    std::set<int> member_outs;
    for (size_t g : group) member_outs.insert((*steps)[g].outputs.begin(), (*steps)[g].outputs.end());
    bool blocked = false;
    for (size_t b = a + 1; b <= group.back() && !blocked; ++b) {
      if (std::find(group.begin(), group.end(), b) != group.end()) continue;
      const Step& x = (*steps)[b];
      bool reads_group = false;
      for (int v : x.inputs) reads_group = reads_group || member_outs.count(v);
      if (!reads_group) continue;
      for (size_t g : group)
        for (int v : (*steps)[g].inputs)
          if (std::find(x.outputs.begin(), x.outputs.end(), v) != x.outputs.end()) blocked = true;
    }
    if (blocked) continue;
    Step f;
    f.kind = StepKind::kRowFused;
    f.reduce_operand_shape = shape;
    f.reduce_dims = (*steps)[a].reduce_dims;
    std::set<int> group_ops;
    for (size_t g : group) {
      const Step& x = (*steps)[g];
      group_ops.insert(x.ops.begin(), x.ops.end());
      group_ops.insert(x.epilogue_ops.begin(), x.epilogue_ops.end());
      for (const ReduceSpec& rs : x.reduces) group_ops.insert(rs.op_index);
    }
    for (size_t g : group) {
      const Step& x = (*steps)[g];
      for (int v : x.inputs)
        if (!member_outs.count(v) && std::find(f.inputs.begin(), f.inputs.end(), v) == f.inputs.end())
          f.inputs.push_back(v);
      for (int v : x.outputs) {  // stored only when read outside the kernel
        bool outside = outputs_.count(v) > 0;
        auto it = users_.find(v);
        if (it != users_.end())
          for (int u : it->second) outside = outside || !group_ops.count(u);
        if (outside) f.outputs.push_back(v);
      }
      f.phases.push_back(x);
    }
    if (f.outputs.empty()) continue;
    for (size_t k = group.size(); k-- > 0;) steps->erase(steps->begin() + group[k]);
    steps->insert(steps->begin() + a, std::move(f));
  }
}

void Planner::shape_row_fused(Step* s) {
  const Dims& shape = s->reduce_operand_shape;
  int64_t rows = 1, row_len = 1;
  const size_t nred = s->reduce_dims.size();
  for (size_t d = 0; d < shape.size(); ++d) (d + nred < shape.size() ? rows : row_len) *= shape[d];
  s->rows = rows;
  s->row_len = row_len;
  s->row_schedule = true;
  size_t min_size = 8;
  for (int v : s->inputs)
    if (prog_.type(v).elements() == num_elements(shape)) min_size = std::min(min_size, dtype_size(prog_.type(v).dtype));
  for (int v : s->outputs)
    if (prog_.type(v).elements() == num_elements(shape)) min_size = std::min(min_size, dtype_size(prog_.type(v).dtype));
  int vec = static_cast<int>(16 / std::max<size_t>(min_size, 1));
  vec = std::max(1, std::min(vec, 8));
  while (vec > 1 && row_len % vec != 0) vec /= 2;
  s->vec = vec;
  s->splits = 1;
  s->chunk = row_len;
  // Many short rows: a wave per row needs no workgroup barrier and packs
  // four rows per workgroup.
  s->wave_per_row = rows >= 1024 && row_len <= 4096;
  s->grid = static_cast<uint32_t>(s->wave_per_row ? (rows + 3) / 4 : rows);
  s->block = 256;
}

void Planner::schedule(std::vector<Step>* steps) {
  auto v2s = value_to_step(*steps);
  const size_t n = steps->size();
  std::vector<std::set<int>> deps(n);
  std::vector<std::vector<int>> rdeps(n);
  for (size_t i = 0; i < n; ++i) {
    for (int v : (*steps)[i].inputs) {
      auto it = v2s.find(v);
      if (it != v2s.end() && it->second != static_cast<int>(i) && deps[i].insert(it->second).second)
        rdeps[it->second].push_back(static_cast<int>(i));
    }
  }
  std::priority_queue<int, std::vector<int>, std::greater<int>> ready;
  std::vector<size_t> indeg(n);
  for (size_t i = 0; i < n; ++i) {
    indeg[i] = deps[i].size();
    if (!indeg[i]) ready.push(static_cast<int>(i));
  }
  std::vector<Step> out;
  while (!ready.empty()) {
    int i = ready.top();
    ready.pop();
    out.push_back(std::move((*steps)[i]));
    for (int j : rdeps[i])
      if (--indeg[j] == 0) ready.push(j);
  }
  PJRTX_CHECK(out.size() == n, Code::kInternal, "fusion planner produced a cyclic schedule");
  *steps = std::move(out);
}

void Planner::liveness() {
  std::set<int> persistent(prog_.params.begin(), prog_.params.end());
  for (int c : plan_.constants) persistent.insert(c);
  std::map<int, int> last_use;
  for (size_t i = 0; i < plan_.steps.size(); ++i)
    for (int v : plan_.steps[i].inputs) last_use[v] = static_cast<int>(i);
  for (auto& [v, i] : last_use) {
    if (persistent.count(v) || outputs_.count(v)) continue;
    plan_.steps[i].release_after.push_back(v);
  }
  // In-place dynamic_update_slice (reference: executable_metal_graph_slice.zig:
  // 129-144): allowed when the operand is an intermediate produced by a
  // kernel, or a donated entry argument, (not a view alias of another live
  // buffer) whose last reader is this step.
  std::map<int, int> donated_param;  // value id -> parameter position
  for (size_t k = 0; k < prog_.params.size(); ++k)
    if (k < prog_.param_alias.size() && prog_.param_alias[k] != -1)
      donated_param[prog_.params[k]] = static_cast<int>(k);
  std::set<int> aliased;
  std::map<int, StepKind> producer_kind;
  for (const Step& s : plan_.steps) {
    if (s.kind == StepKind::kAlias) aliased.insert(s.inputs[0]);
    for (int v : s.outputs) producer_kind[v] = s.kind;
  }
  for (size_t i = 0; i < plan_.steps.size(); ++i) {
    Step& s = plan_.steps[i];
    if (s.kind != StepKind::kLibrary || s.lib != LibKind::kDynamicUpdateSlice) continue;
    const int v0 = prog_.ops[s.lib_op].operands[0];
    const bool intermediate = !persistent.count(v0) && !outputs_.count(v0) && !aliased.count(v0) &&
                              producer_kind.count(v0) && producer_kind[v0] != StepKind::kAlias;
    const bool donated = donated_param.count(v0) && !outputs_.count(v0) && !aliased.count(v0);
    if ((intermediate || donated) && last_use[v0] == static_cast<int>(i)) {
      s.in_place = true;
      if (donated) plan_.written_params.push_back(donated_param[v0]);
    }
  }
}

// An in-place dynamic_update_slice whose update has the shape of an earlier
// elementwise kernel's root is written by that kernel, at the window's
// clamped offset, instead of by its own launch (a KV-cache row written where
// RoPE computes it; the value row copied by the same kernel). Requires the
// window to span the operand's innermost dim (the kernel's vector stores stay
// in one row) and nothing between the kernel and the update to touch the
// operand. Release lists are rebuilt afterwards.
void Planner::absorb_window_updates() {
  std::vector<Step>& steps = plan_.steps;
  std::map<int, int> v2s = value_to_step(steps);
  auto before = [&](int v, size_t j) {  // value available before step j
    auto it = v2s.find(v);
    if (it == v2s.end()) return true;  // parameter or resident constant
    return it->second < static_cast<int>(j);
  };
  bool changed = false;
  for (size_t i = 0; i < steps.size(); ++i) {
    Step& D = steps[i];
    if (D.kind != StepKind::kLibrary || D.lib != LibKind::kDynamicUpdateSlice || !D.in_place) continue;
    const Op& op = prog_.ops[D.lib_op];
    const int v0 = op.operands[0], u = op.operands[1], r = op.results[0];
    const TensorType& ut = prog_.type(u);
    const TensorType& ot = prog_.type(v0);
    if (ut.rank() == 0 || ut.dims.back() != ot.dims.back() || ut.elements() == 0) continue;
    std::vector<int> starts(op.operands.begin() + 2, op.operands.end());
    // The update's buffer, seen through order-preserving view aliases.
    int src = u;
    while (v2s.count(src) && steps[v2s[src]].kind == StepKind::kAlias) src = steps[v2s[src]].inputs[0];
    int target = -1;
    for (int j = static_cast<int>(i) - 1; j >= 0 && target < 0; --j) {
      const Step& L = steps[j];
      // Nothing from j to i may read or write the operand or the result.
      bool clear = true;
      for (size_t k = j + 1; k < i && clear; ++k) {
        for (int v : steps[k].inputs) clear &= v != v0 && v != r;
        for (int v : steps[k].outputs) clear &= v != v0;
      }
      if (!clear) break;
      // A kernel that reads the operand cannot also write the window into
      // it: other workgroups may overwrite elements before they are read
      // (a shift of the operand by one row, written back in place).
      for (int v : L.inputs) clear &= v != v0 && v != r;
      if (!clear) break;
      if (L.kind != StepKind::kLoop || L.loop_shape != ut.dims || L.window_out.size() >= 2) continue;
      if (ut.dims.back() % L.vec != 0) continue;
      const bool own = std::find(L.outputs.begin(), L.outputs.end(), u) != L.outputs.end();
      bool ok = own || before(src, j);
      for (int sv : starts) ok &= before(sv, j) || is_splat_constant(prog_, prog_.ops[producer_.at(sv)]);
      if (ok) target = j;
    }
    if (target < 0) continue;
    Step& L = steps[target];
    const bool own = std::find(L.outputs.begin(), L.outputs.end(), u) != L.outputs.end();
    Step::WindowWrite ww;
    ww.operand = v0;
    ww.update = own ? u : src;
    ww.starts = starts;
    if (!own && std::find(L.inputs.begin(), L.inputs.end(), src) == L.inputs.end()) L.inputs.push_back(src);
    for (int sv : starts) {
      auto pi = producer_.find(sv);
      const bool lit = pi != producer_.end() && is_splat_constant(prog_, prog_.ops[pi->second]);
      if (!lit && std::find(L.inputs.begin(), L.inputs.end(), sv) == L.inputs.end()) L.inputs.push_back(sv);
    }
    L.window_out[static_cast<int>(L.outputs.size())] = ww;
    L.outputs.push_back(r);
    // The update no longer needs its own buffer when the DUS was its only reader.
    if (own && !outputs_.count(u)) {
      bool read = false;
      for (size_t k = 0; k < steps.size(); ++k)
        if (k != i)
          for (int v : steps[k].inputs) read |= v == u;
      if (!read) {
        const int pos = static_cast<int>(std::find(L.outputs.begin(), L.outputs.end(), u) - L.outputs.begin());
        L.outputs.erase(L.outputs.begin() + pos);
        std::map<int, Step::WindowWrite> moved;
        for (auto& [k, w] : L.window_out) moved[k > pos ? k - 1 : k] = w;
        L.window_out = std::move(moved);
        mat_.erase(u);
      }
    }
    steps.erase(steps.begin() + i);
    --i;
    v2s = value_to_step(steps);
    changed = true;
  }
  if (!changed) return;
  for (Step& s : steps) s.release_after.clear();
  std::set<int> persistent(prog_.params.begin(), prog_.params.end());
  for (int c : plan_.constants) persistent.insert(c);
  std::map<int, int> last_use;
  for (size_t i = 0; i < steps.size(); ++i)
    for (int v : steps[i].inputs) last_use[v] = static_cast<int>(i);
  for (auto& [v, i] : last_use) {
    if (persistent.count(v) || outputs_.count(v)) continue;
    steps[i].release_after.push_back(v);
  }
}

void Planner::shape_loop(Step* s) {
  const int64_t n = num_elements(s->loop_shape);
  // 16-byte accesses for the narrowest element touched at the root index.
  size_t min_size = dtype_size(prog_.type(s->outputs[0]).dtype);
  for (int v : s->inputs)
    if (prog_.type(v).elements() == n) min_size = std::min(min_size, dtype_size(prog_.type(v).dtype));
  int vec = static_cast<int>(16 / std::max<size_t>(min_size, 1));
  vec = std::max(1, std::min(vec, 8));
  s->vec = vec;
  const int64_t per_block = 256 * vec;
  s->grid = static_cast<uint32_t>(std::max<int64_t>(1, (n + per_block - 1) / per_block));
  s->block = 256;
}

void Planner::shape_reduce(Step* s) {
  const Dims& shape = s->reduce_operand_shape;
  const int rank = static_cast<int>(shape.size());
  const int nred = static_cast<int>(s->reduce_dims.size());
  bool trailing = true;
  for (int k = 0; k < nred; ++k)
    if (s->reduce_dims[k] != rank - nred + k) trailing = false;
  int64_t rows = 1, row_len = 1;
  for (int d = 0; d < rank; ++d) {
    if (std::binary_search(s->reduce_dims.begin(), s->reduce_dims.end(), static_cast<int64_t>(d))) row_len *= shape[d];
    else rows *= shape[d];
  }
  s->rows = rows;
  s->row_len = row_len;
  // Row schedule needs enough work per row to fill a workgroup; otherwise a
  // thread per output walks its reduced elements serially.
  s->row_schedule = trailing && row_len >= 64;
  if (!s->row_schedule) {
    s->vec = 1;
    s->splits = 1;
    s->grid = static_cast<uint32_t>(std::max<int64_t>(1, (rows + 255) / 256));
    s->block = 256;
    return;
  }
  size_t min_size = 8;
  for (int v : s->inputs)
    if (prog_.type(v).elements() == num_elements(shape)) min_size = std::min(min_size, dtype_size(prog_.type(v).dtype));
  int vec = static_cast<int>(16 / std::max<size_t>(min_size, 1));
  vec = std::max(1, std::min(vec, 8));
  while (vec > 1 && row_len % vec != 0) vec /= 2;
  s->vec = vec;
  const int block = opts_.reduce_block >= 1024 ? 1024 : opts_.reduce_block >= 512 ? 512 : 256;
  const int64_t per_iter = block * vec;
  // Few long rows: split each row over several workgroups so the launch
  // reaches the target block count, keeping at least one full 256*vec span
  // per split.
  int64_t splits = (opts_.reduce_target_blocks + rows - 1) / rows;
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, row_len / per_iter));
  splits = std::max<int64_t>(1, std::min<int64_t>(splits, 64));
  int64_t chunk = (row_len + splits - 1) / splits;
  chunk = (chunk + vec - 1) / vec * vec;
  splits = (row_len + chunk - 1) / chunk;
  s->splits = splits;
  s->chunk = chunk;
  s->unroll = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(8, (chunk + per_iter - 1) / per_iter)));
  s->grid = static_cast<uint32_t>(rows * splits);
  s->block = block;
  if (splits > 1) {
    size_t per_slot = 0;
    for (const ReduceSpec& r : s->reduces) per_slot += (r.kind == ReducerKind::kArgMax || r.kind == ReducerKind::kArgMin) ? 16 : 8;
    s->scratch_bytes = static_cast<size_t>(rows * splits) * per_slot;
    // The `_combine` kernel folds the partials in a second launch; with a
    // fused combine (rows a multiple of 8, so that every split of a row runs
    // on one XCD) the last-arriving workgroup of each row folds them inside
    // the same launch, and the combine kernel remains the fallback for a
    // device that does not place workgroups round-robin on its XCDs.
    s->combine_grid = static_cast<uint32_t>((rows + 3) / 4);
    if (opts_.reduce_fused_combine) {
      // One 32-bit arrival counter per row, each on a 128-byte line of its
      // own, after the 8-byte slots. With rows a multiple of 8, row = b %
      // rows keeps a row's splits on one XCD; otherwise the grid is padded to
      // 8 * ceil(rows / 8) * splits workgroups, row (b % 8) + 8 * ((b / 8) /
      // splits) (the rest exit at once).
      s->fused_combine = true;
      if (rows % 8 != 0) s->grid = static_cast<uint32_t>(8 * ((rows + 7) / 8) * splits);
      s->counter_offset = (s->scratch_bytes + 127) / 128 * 128;
      s->scratch_bytes = s->counter_offset + static_cast<size_t>(rows) * 128;
    }
  }
}

Plan Planner::run() {
  decide_materialization();
  std::vector<Step> steps;
  build_steps(&steps);
  if (opts_.fuse_siblings) merge_siblings(&steps);
  if (opts_.fuse_epilogues) merge_epilogues(&steps);
  if (opts_.dot_residual) merge_dot_residuals(&steps);
  if (opts_.row_fuse_max > 0) fuse_row_chains(&steps);
  if (opts_.fuse_siblings) merge_sibling_loops(&steps);
  schedule(&steps);
  int kernel_id = 0;
  for (Step& s : steps) {
    if (s.kind == StepKind::kLoop) {
      shape_loop(&s);
      s.name = strformat("pjrtx_fusion_loop_%d", kernel_id++);
    } else if (s.kind == StepKind::kReduce) {
      shape_reduce(&s);
      s.name = strformat("pjrtx_fusion_reduce_%d", kernel_id++);
    } else if (s.kind == StepKind::kRowFused) {
      shape_row_fused(&s);
      s.name = strformat("pjrtx_fusion_row_%d", kernel_id++);
    }
  }
  plan_.steps = std::move(steps);
  plan_.num_fusion_kernels = kernel_id;
  liveness();
  if (opts_.fuse_siblings) absorb_window_updates();
  fuse_gemv_steps(prog_, &plan_, outputs_, opts_);
  return std::move(plan_);
}

}  // namespace

std::string Plan::describe(const Program& prog) const {
  std::ostringstream o;
  auto list = [&](const std::vector<int>& v) {
    std::string s = "[";
    for (size_t i = 0; i < v.size(); ++i) s += (i ? "," : "") + std::to_string(v[i]);
    return s + "]";
  };
  o << "{\"steps\":[";
  for (size_t i = 0; i < steps.size(); ++i) {
    const Step& s = steps[i];
    if (i) o << ",";
    const char* kind = s.kind == StepKind::kLoop ? "loop" : s.kind == StepKind::kReduce ? "reduce"
                     : s.kind == StepKind::kAlias ? "alias" : s.kind == StepKind::kRowFused ? "rowfused"
                     : s.kind == StepKind::kGemv ? "gemv" : "library";
    o << "{\"kind\":\"" << kind << "\",\"name\":\"" << s.name << "\"";
    o << ",\"inputs\":" << list(s.inputs) << ",\"outputs\":" << list(s.outputs);
    auto bytes_of = [&](const std::vector<int>& vs) {
      std::string b = "[";
      for (size_t k = 0; k < vs.size(); ++k) b += (k ? "," : "") + std::to_string(prog.type(vs[k]).bytes());
      return b + "]";
    };
    o << ",\"in_bytes\":" << bytes_of(s.inputs) << ",\"out_bytes\":" << bytes_of(s.outputs);
    // Bytes the step must move at minimum: every input read once and every
    // output written once, except where a library op touches only part of an
    // input (gather and dynamic_slice read the selected rows; an in-place
    // dynamic_update_slice reads and writes only the update's window).
    int64_t alg = 0;
    for (int v : s.inputs) alg += prog.type(v).bytes();
    for (int v : s.outputs) alg += prog.type(v).bytes();
    if (s.kind == StepKind::kLibrary) {
      const Op& d = prog.ops[s.lib_op];
      const int64_t out = prog.type(d.results[0]).bytes();
      if (s.lib == LibKind::kGather) {
        alg = 2 * out + prog.type(d.operands[1]).bytes();
      } else if (s.lib == LibKind::kDynamicSlice) {
        alg = 2 * out;
        for (size_t k = 1; k < d.operands.size(); ++k) alg += prog.type(d.operands[k]).bytes();
      } else if (s.lib == LibKind::kDynamicUpdateSlice && s.in_place) {
        alg = 2 * prog.type(d.operands[1]).bytes();
        for (size_t k = 2; k < d.operands.size(); ++k) alg += prog.type(d.operands[k]).bytes();
      }
    }
    if (s.kind == StepKind::kGemv) {
      // Window outputs move only their window (the update's elements).
      for (auto& [k, w] : s.window_out)
        alg += prog.type(w.update).bytes() - prog.type(s.outputs[k]).bytes();
    }
    o << ",\"algorithmic_bytes\":" << alg;
    std::vector<std::string> names;
    o << ",\"ops\":[";
    for (size_t k = 0; k < s.ops.size(); ++k) o << (k ? "," : "") << "\"" << op_kind_name(prog.ops[s.ops[k]].kind) << "\"";
    o << "],\"epilogue\":[";
    for (size_t k = 0; k < s.epilogue_ops.size(); ++k) o << (k ? "," : "") << "\"" << op_kind_name(prog.ops[s.epilogue_ops[k]].kind) << "\"";
    o << "]";
    if (!s.window_out.empty()) {
      o << ",\"window_outputs\":[";
      bool first = true;
      for (auto& [k, w] : s.window_out) {
        o << (first ? "" : ",") << "{\"output\":" << s.outputs[k] << ",\"operand\":" << w.operand << "}";
        first = false;
      }
      o << "]";
    }
    if (s.kind == StepKind::kRowFused)
      o << ",\"phases\":" << s.phases.size() << ",\"rows\":" << s.rows << ",\"row_len\":" << s.row_len
        << ",\"wave_per_row\":" << (s.wave_per_row ? "true" : "false");
    if (s.kind == StepKind::kGemv) {
      const GemvSpec& g = s.gemv;
      int64_t flops = 0;
      std::string ns = "[";
      for (size_t m = 0; m < g.dots.size(); ++m) {
        const int64_t n = prog.type(g.result[m]).dims[1];
        flops += 2 * g.M * g.K * n;
        ns += (m ? "," : "") + std::to_string(n);
      }
      o << ",\"flops\":" << flops << ",\"members\":" << g.dots.size() << ",\"M\":" << g.M << ",\"K\":" << g.K
        << ",\"N\":" << ns << "],\"cols\":" << g.cols << ",\"depth\":" << g.depth << ",\"ksplit\":" << g.ksplit
        << ",\"kchunk\":" << g.kchunk << ",\"joint\":" << (g.joint ? "true" : "false")
        << ",\"seg_cols\":" << g.seg_cols << ",\"segments\":" << g.nseg << ",\"items_per_segment\":" << g.wps << ",\"workgroups\":" << g.wgs
        << ",\"stage_all_x\":" << (g.stage_all_x ? "true" : "false")
        << ",\"direct\":" << (g.direct ? "true" : "false") << ",\"fused_combine\":" << (s.fused_combine ? "true" : "false")
        << ",\"prologue\":" << (s.prologue.empty() ? "null" : "\"" + std::string("rowfused") + "\"")
        << ",\"epilogue_loop\":[";
      if (!s.epilogue_loop.empty())
        for (size_t k = 0; k < s.epilogue_loop[0].ops.size(); ++k)
          o << (k ? "," : "") << "\"" << op_kind_name(prog.ops[s.epilogue_loop[0].ops[k]].kind) << "\"";
      o << "]";
      for (size_t m = 0; m < g.add.size(); ++m)
        if (g.add[m] >= 0) o << ",\"residual_add\":" << g.add[m];
      if (g.attn_splits) o << ",\"attention_splits_merged\":" << g.attn_splits;
    }
    if (s.kind == StepKind::kReduce) {
      o << ",\"reducers\":[";
      for (size_t k = 0; k < s.reduces.size(); ++k) o << (k ? "," : "") << "\"" << reducer_name(s.reduces[k].kind) << "\"";
      o << "],\"row_schedule\":" << (s.row_schedule ? "true" : "false") << ",\"rows\":" << s.rows
        << ",\"row_len\":" << s.row_len << ",\"splits\":" << s.splits << ",\"chunk\":" << s.chunk
        << ",\"fused_combine\":" << (s.fused_combine ? "true" : "false");
    }
    if (s.kind == StepKind::kLibrary) {
      o << ",\"library\":\"" << lib_kind_name(s.lib) << "\",\"in_place\":" << (s.in_place ? "true" : "false");
      if (s.lib == LibKind::kDot || s.lib == LibKind::kDotGroup) {  // 2 * output elements * contracted size
        int64_t flops = 0;
        const std::vector<int> ops = s.lib == LibKind::kDot ? std::vector<int>{s.lib_op} : s.group_ops;
        for (int oi : ops) {
          const Op& d = prog.ops[oi];
          int64_t kc = 1;
          for (int64_t c : d.lhs_contract) kc *= prog.type(d.operands[0]).dims[c];
          flops += 2 * prog.type(d.results[0]).elements() * kc;
        }
        o << ",\"flops\":" << flops;
        if (s.lib == LibKind::kDotGroup) o << ",\"group_size\":" << s.group_ops.size();
        if (s.dot_add >= 0) o << ",\"residual_add\":" << s.dot_add;
      }
      if (s.lib == LibKind::kWhile) o << ",\"while_trips\":" << s.while_trips;
      if (s.lib == LibKind::kAttention) {  // q.k and p.v over every (query, key) pair
        const Op& d = prog.ops[s.lib_op];
        const TensorType& q = prog.type(d.operands[0]);
        const TensorType& k = prog.type(d.operands[1]);
        const int sa = d.attn.layout == 0 ? 2 : d.attn.layout == 1 ? 1 : 0;
        // Pairs the mask allows (static masks only; a runtime offset leaves
        // the count at every pair).
        const int64_t sq = q.dims[sa], skv = k.dims[sa];
        int64_t pairs = sq * skv;
        if (d.attn.causal && !d.attn.has_offset_operand) {
          pairs = 0;
          for (int64_t i = 0; i < sq; ++i)
            pairs += std::max<int64_t>(0, std::min<int64_t>(skv, d.attn.q_coef * i + d.attn.offset + 1));
        }
        o << ",\"flops\":" << 4 * q.elements() * skv << ",\"effective_flops\":" << 4 * (q.elements() / sq) * pairs
          << ",\"causal\":" << (d.attn.causal ? "true" : "false")
          << ",\"q_coef\":" << d.attn.q_coef << ",\"offset\":" << d.attn.offset
          << ",\"partials_out\":" << (s.attn_partials ? "true" : "false")
          << ",\"offset_operand\":" << (d.attn.has_offset_operand ? "true" : "false") << ",\"scale\":" << strformat("%.17g", d.attn.scale)
          << ",\"layout\":" << d.attn.layout;
      }
    }
    o << ",\"vec\":" << s.vec << ",\"grid\":" << s.grid << ",\"block\":" << s.block;
    o << ",\"release_after\":" << list(s.release_after) << "}";
  }
  o << "],\"constants\":" << list(constants) << ",\"fusion_kernels\":" << num_fusion_kernels
    << ",\"param_alias\":" << list(prog.param_alias) << ",\"written_params\":" << list(written_params) << "}";
  return o.str();
}

Plan make_plan(const Program& prog, const PlanOptions& opts) {
  Planner p(prog, opts);
  Plan plan = p.run();
  if (env_flag("PJRTX_PLAN_DEBUG")) std::fprintf(stderr, "pjrtx plan: %s\n", plan.describe(prog).c_str());
  plan.nt_min_bytes = opts.nt_min_bytes;
  plan.kernel_source = generate_kernels(prog, plan);
  return plan;
}

}  // namespace pjrtx
