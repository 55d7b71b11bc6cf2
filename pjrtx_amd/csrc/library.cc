// Dispatch of library steps: StableHLO ops that materialize their result
// through a precompiled kernel instead of a generated fusion.
#include "kernels/library.h"
#include "kernels/reduce_window.h"

#include <cstring>
#include <map>

#include "runtime.h"
#include "sort_op.h"

namespace pjrtx {

namespace {

void row_major_strides(const Dims& d, int64_t* out) {
  int64_t s = 1;
  for (int i = static_cast<int>(d.size()) - 1; i >= 0; --i) {
    out[i] = s;
    s *= d[i];
  }
}

void check_rank(const Dims& d, const char* what) {
  PJRTX_CHECK(d.size() <= static_cast<size_t>(kMaxRank), Code::kUnimplemented,
              strformat("%s: rank %zu exceeds %d", what, d.size(), kMaxRank));
}

void* ptr(std::vector<MemRef>& vals, int v) { return vals[v] ? vals[v]->ptr : nullptr; }

void run_dynamic_slice(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals) {
  const TensorType& x = prog.type(op.operands[0]);
  const TensorType& out = prog.type(op.results[0]);
  check_rank(x.dims, "dynamic_slice");
  BoxCopy b;
  b.rank = x.rank();
  row_major_strides(x.dims, b.src_stride);
  row_major_strides(out.dims, b.dst_stride);
  for (int d = 0; d < b.rank; ++d) {
    b.dims[d] = out.dims[d];
    b.dyn_start[d] = ptr(vals, op.operands[1 + d]);
    b.dyn_limit[d] = x.dims[d];
  }
  const DType it = prog.type(op.operands[1]).dtype;
  b.dyn_start_bytes = static_cast<int>(dtype_size(it));
  b.dyn_start_signed = dtype_is_signed_int(it);
  b.dyn_on_dst = 0;
  launch_box_copy(dev->stream(), b, ptr(vals, op.operands[0]), ptr(vals, op.results[0]),
                  static_cast<int>(dtype_size(x.dtype)));
}

void run_dynamic_update_slice(Device* dev, const Program& prog, const Step& step, const Op& op,
                              std::vector<MemRef>& vals) {
  const TensorType& x = prog.type(op.operands[0]);
  const TensorType& u = prog.type(op.operands[1]);
  check_rank(x.dims, "dynamic_update_slice");
  const int esz = static_cast<int>(dtype_size(x.dtype));
  if (!step.in_place) {
    // Copy the operand into the fresh output, then write the update.
    if (x.bytes())
      hip_check(hipMemcpyAsync(ptr(vals, op.results[0]), ptr(vals, op.operands[0]), x.bytes(), hipMemcpyDeviceToDevice,
                               dev->stream()),
                "hipMemcpyAsync(DUS operand)");
  }
  BoxCopy b;
  b.rank = x.rank();
  row_major_strides(u.dims, b.src_stride);
  row_major_strides(x.dims, b.dst_stride);
  for (int d = 0; d < b.rank; ++d) {
    b.dims[d] = u.dims[d];
    b.dyn_start[d] = ptr(vals, op.operands[2 + d]);
    b.dyn_limit[d] = x.dims[d];
  }
  const DType it = prog.type(op.operands[2]).dtype;
  b.dyn_start_bytes = static_cast<int>(dtype_size(it));
  b.dyn_start_signed = dtype_is_signed_int(it);
  b.dyn_on_dst = 1;
  launch_box_copy(dev->stream(), b, ptr(vals, op.operands[1]), ptr(vals, op.results[0]), esz);
}

void run_concatenate(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals) {
  const TensorType& out = prog.type(op.results[0]);
  check_rank(out.dims, "concatenate");
  int64_t ost[kMaxRank];
  row_major_strides(out.dims, ost);
  int64_t offset = 0;
  for (int src : op.operands) {
    const TensorType& t = prog.type(src);
    BoxCopy b;
    b.rank = t.rank();
    row_major_strides(t.dims, b.src_stride);
    for (int d = 0; d < b.rank; ++d) {
      b.dims[d] = t.dims[d];
      b.dst_stride[d] = ost[d];
    }
    b.dst_off = offset * ost[op.dim];
    launch_box_copy(dev->stream(), b, ptr(vals, src), ptr(vals, op.results[0]), static_cast<int>(dtype_size(t.dtype)));
    offset += t.dims[op.dim];
  }
}

void run_pad(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals) {
  const TensorType& x = prog.type(op.operands[0]);
  const TensorType& out = prog.type(op.results[0]);
  check_rank(out.dims, "pad");
  for (size_t d = 0; d < x.dims.size(); ++d)
    PJRTX_CHECK(op.pad_low[d] >= 0 && op.pad_high[d] >= 0 && op.pad_interior[d] >= 0, Code::kUnimplemented,
                "pad with negative (cropping) padding is not supported");
  const int esz = static_cast<int>(dtype_size(x.dtype));
  launch_fill(dev->stream(), ptr(vals, op.results[0]), ptr(vals, op.operands[1]), out.elements(), esz);
  int64_t ost[kMaxRank];
  row_major_strides(out.dims, ost);
  BoxCopy b;
  b.rank = x.rank();
  row_major_strides(x.dims, b.src_stride);
  for (int d = 0; d < b.rank; ++d) {
    b.dims[d] = x.dims[d];
    b.dst_stride[d] = ost[d] * (op.pad_interior[d] + 1);
    b.dst_off += op.pad_low[d] * ost[d];
  }
  launch_box_copy(dev->stream(), b, ptr(vals, op.operands[0]), ptr(vals, op.results[0]), esz);
}

}  // namespace

// Translates StableHLO gather dimension numbers into the kernel's mapping
// (semantics: StableHLO spec `gather`; start indices are clamped so the slice
// stays in bounds, as reference executable_metal_graph_gather.zig:61-65).
// JAX normalizes a negative gather index i to i + N before the gather
// (select(compare(LT, i, 0), add(i, N), i), N the gathered dimension's size,
// as `table[i]` lowers); the gather kernels apply the same rule while they
// read the index (Op::index_wrap), so the normalization's elementwise launch
// goes away (PJRTX_GATHER_WRAP=0 keeps it). Matched for a one-component
// index vector whose value reaches the gather through reshapes and
// broadcasts that only add unit dimensions (the flat order unchanged): the
// gather then reads i through one reshape to its index shape.
bool fold_gather_index_wrap(Program* prog) {
  if (env_int("PJRTX_GATHER_WRAP", 1) == 0) return false;
  std::map<int, size_t> producer;
  for (size_t i = 0; i < prog->ops.size(); ++i)
    for (int r : prog->ops[i].results) producer[r] = i;
  auto op_of = [&](int v) -> const Op* {
    auto it = producer.find(v);
    return it == producer.end() ? nullptr : &prog->ops[it->second];
  };
  auto is_int = [](DType t) { return (dtype_is_signed_int(t) || dtype_is_unsigned_int(t)) && t != DType::kPred; };
  // A splat integer constant, directly or broadcast from a one-element one.
  auto splat_int = [&](int v, int64_t* out) {
    const Op* o = op_of(v);
    if (o && o->kind == OpKind::kBroadcastInDim && prog->type(o->operands[0]).elements() == 1) o = op_of(o->operands[0]);
    if (!o || o->kind != OpKind::kConstant || o->results.size() != 1) return false;
    const TensorType& t = prog->type(o->results[0]);
    const size_t es = dtype_size(t.dtype);
    if (!is_int(t.dtype) || !(o->splat || t.elements() == 1) || o->literal.size() < es) return false;
    uint64_t u = 0;
    std::memcpy(&u, o->literal.data(), es);
    const int sh = 64 - 8 * static_cast<int>(es);
    *out = dtype_is_signed_int(t.dtype) && sh > 0 ? static_cast<int64_t>(u << sh) >> sh : static_cast<int64_t>(u);
    return true;
  };
  // Views that keep the flat element order.
  auto order_view = [&](const Op* o) {
    if (o->kind == OpKind::kReshape) return true;
    if (o->kind != OpKind::kBroadcastInDim) return false;
    const TensorType& in = prog->type(o->operands[0]);
    const TensorType& out = prog->type(o->results[0]);
    if (in.elements() != out.elements()) return false;
    for (size_t k = 1; k < o->dims.size(); ++k)
      if (o->dims[k] <= o->dims[k - 1]) return false;
    return true;
  };
  // The reshapes to insert, each before its gather (ops are not moved while
  // producers are still looked up).
  std::vector<std::pair<size_t, Op>> inserts;
  for (size_t gi = 0; gi < prog->ops.size(); ++gi) {
    Op& g = prog->ops[gi];
    if (g.kind == OpKind::kGather && g.index_wrap == 0 && g.start_index_map.size() == 1) {
      const int idx = g.operands[1];
      int v = idx;
      const Op* o = op_of(v);
      while (o && order_view(o)) {
        v = o->operands[0];
        o = op_of(v);
      }
      int64_t zero = -1, n = 0;
      const int64_t N = prog->type(g.operands[0]).dims.at(g.start_index_map[0]);
      if (o && o->kind == OpKind::kSelect) {
        const int x = o->operands[2];
        const Op* cmp = op_of(o->operands[0]);
        const Op* add = op_of(o->operands[1]);
        const bool cmp_ok = cmp && cmp->kind == OpKind::kCompare && cmp->cmp_dir == CmpDir::kLT &&
                            cmp->cmp_type != CmpType::kUnsigned && cmp->cmp_type != CmpType::kFloat &&
                            cmp->operands[0] == x && splat_int(cmp->operands[1], &zero) && zero == 0;
        int other = -1;
        if (add && add->kind == OpKind::kAdd) other = add->operands[0] == x ? add->operands[1] : add->operands[1] == x ? add->operands[0] : -1;
        const bool add_ok = other >= 0 && splat_int(other, &n) && n == N;
        const DType xt = prog->type(x).dtype;
        if (cmp_ok && add_ok && dtype_is_signed_int(xt) && xt == prog->type(idx).dtype && N > 0 &&
            prog->type(x).elements() == prog->type(idx).elements()) {
          // the gather's index operand: x through one reshape to its shape
          Value nv;
          nv.type = prog->type(idx);
          nv.name = prog->values[x].name + ".gather_index";
          prog->values.push_back(nv);
          const int r = static_cast<int>(prog->values.size()) - 1;
          Op rs;
          rs.kind = OpKind::kReshape;
          rs.name = "stablehlo.reshape";
          rs.operands = {x};
          rs.results = {r};
          g.operands[1] = r;
          g.index_wrap = N;
          inserts.emplace_back(gi, std::move(rs));
        }
      }
    }
  }
  if (inserts.empty()) return false;
  std::vector<Op> ops;
  ops.reserve(prog->ops.size() + inserts.size());
  size_t next = 0;
  for (size_t i = 0; i < prog->ops.size(); ++i) {
    while (next < inserts.size() && inserts[next].first == i) ops.push_back(std::move(inserts[next++].second));
    ops.push_back(std::move(prog->ops[i]));
  }
  prog->ops = std::move(ops);
  return true;
}

GatherParams make_gather_params(const Program& prog, const Op& op) {
  const TensorType& x = prog.type(op.operands[0]);
  const TensorType& idx = prog.type(op.operands[1]);
  const TensorType& out = prog.type(op.results[0]);
  check_rank(x.dims, "gather");
  check_rank(out.dims, "gather");
  check_rank(idx.dims, "gather");
  GatherParams g;
  g.out_rank = out.rank();
  g.op_rank = x.rank();
  g.idx_rank = idx.rank();
  for (int d = 0; d < g.out_rank; ++d) g.out_dims[d] = out.dims[d];
  for (int d = 0; d < g.op_rank; ++d) {
    g.op_dims[d] = x.dims[d];
    g.slice[d] = op.sizes.at(d);
  }
  row_major_strides(x.dims, g.op_stride);
  row_major_strides(idx.dims, g.idx_stride);
  g.ivd = static_cast<int>(op.index_vector_dim < 0 ? idx.rank() : op.index_vector_dim);
  g.n_index = static_cast<int>(op.start_index_map.size());
  PJRTX_CHECK(g.ivd == g.idx_rank || idx.dims[g.ivd] == g.n_index, Code::kInvalidArgument,
              "gather: index vector length does not match start_index_map");
  for (int k = 0; k < g.n_index; ++k) g.start_map[k] = static_cast<int>(op.start_index_map[k]);
  g.n_batching = static_cast<int>(op.operand_batching_dims.size());
  for (int k = 0; k < g.n_batching; ++k) {
    g.op_batch_dim[k] = static_cast<int>(op.operand_batching_dims[k]);
    g.idx_batch_dim[k] = static_cast<int>(op.start_indices_batching_dims[k]);
  }
  // Output dims: offset_dims are window dims (operand dims that are neither
  // collapsed nor batching, in increasing order); the rest are batch dims
  // (start_indices dims except index_vector_dim, in order).
  std::vector<int> window_operand_dims;
  for (int d = 0; d < g.op_rank; ++d) {
    bool collapsed = false;
    for (int64_t c : op.collapsed_slice_dims) collapsed |= c == d;
    for (int64_t c : op.operand_batching_dims) collapsed |= c == d;
    if (!collapsed) window_operand_dims.push_back(d);
  }
  std::vector<int> batch_idx_dims;
  for (int d = 0; d < g.idx_rank; ++d)
    if (d != g.ivd) batch_idx_dims.push_back(d);
  size_t wi = 0, bi = 0;
  for (int d = 0; d < g.out_rank; ++d) {
    bool is_offset = false;
    for (int64_t o : op.offset_dims) is_offset |= o == d;
    if (is_offset) {
      PJRTX_CHECK(wi < window_operand_dims.size(), Code::kInvalidArgument, "gather: too many offset dims");
      g.out_map[d] = -window_operand_dims[wi++] - 1;
    } else {
      PJRTX_CHECK(bi < batch_idx_dims.size(), Code::kInvalidArgument, "gather: too many batch dims");
      g.out_map[d] = batch_idx_dims[bi++];
    }
  }
  g.idx_bytes = static_cast<int>(dtype_size(idx.dtype));
  g.idx_signed = dtype_is_signed_int(idx.dtype);
  g.wrap = op.index_wrap;
  return g;
}

void run_dot_general(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals);
void run_scatter(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals);
void run_attention(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals, bool partials_out);
void run_dot_group(Device* dev, const Program& prog, const std::vector<int>& ops, std::vector<MemRef>& vals);
void run_dot_residual(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals, int add, int out);

// stablehlo.reduce_window (the planner checked the supported forms).
// Replaces pjrtx_mlx_metal_buffer_reduce_window and
// pjrtx_mlx_metal_buffer_reduce_window_max_with_indices (reference:
// src/backend/mlx_metal/api.cc:4324-4620).
void run_reduce_window(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals) {
  ReduceWindowParams p;
  const TensorType& in = prog.type(op.operands[0]);
  const TensorType& out = prog.type(op.results[0]);
  p.rank = static_cast<int>(in.dims.size());
  switch (classify_reducer(prog, op)) {
    case ReducerKind::kProd: p.op = 1; break;
    case ReducerKind::kMax: p.op = 2; break;
    case ReducerKind::kMin: p.op = 3; break;
    case ReducerKind::kArgMax: p.op = 4; break;
    case ReducerKind::kArgMin: p.op = 5; break;
    default: p.op = 0; break;
  }
  for (int d = 0; d < p.rank; ++d) {
    p.in_dims[d] = in.dims[d];
    p.out_dims[d] = out.dims[d];
    p.window[d] = op.sizes[d];
    p.stride[d] = op.strides[d];
    p.dilation[d] = op.window_dilations[d];
    p.base_dilation[d] = op.base_dilations[d];
    p.pad_low[d] = op.pad_low[d];
  }
  if (op.results.size() == 2) {
    launch_reduce_window_arg(dev->stream(), p, in.dtype, prog.type(op.operands[1]).dtype, ptr(vals, op.operands[0]),
                             ptr(vals, op.operands[1]), ptr(vals, op.operands[2]), ptr(vals, op.operands[3]),
                             ptr(vals, op.results[0]), ptr(vals, op.results[1]));
    return;
  }
  launch_reduce_window(dev->stream(), p, in.dtype, ptr(vals, op.operands[0]), ptr(vals, op.operands[1]),
                       ptr(vals, op.results[0]));
}

void run_library_step(Device* dev, const Program& prog, const Step& step, std::vector<MemRef>& vals) {
  const Op& op = prog.ops.at(step.lib_op);
  switch (step.lib) {
    case LibKind::kDynamicSlice:
      run_dynamic_slice(dev, prog, op, vals);
      return;
    case LibKind::kDynamicUpdateSlice:
      run_dynamic_update_slice(dev, prog, step, op, vals);
      return;
    case LibKind::kConcatenate:
      run_concatenate(dev, prog, op, vals);
      return;
    case LibKind::kPad:
      run_pad(dev, prog, op, vals);
      return;
    case LibKind::kGather: {
      GatherParams g = make_gather_params(prog, op);
      launch_gather(dev->stream(), g, ptr(vals, op.operands[0]), ptr(vals, op.operands[1]), ptr(vals, op.results[0]),
                    static_cast<int>(dtype_size(prog.type(op.operands[0]).dtype)));
      return;
    }
    case LibKind::kDot:
      if (step.dot_add >= 0) run_dot_residual(dev, prog, op, vals, step.dot_add, step.outputs[0]);
      else run_dot_general(dev, prog, op, vals);
      return;
    case LibKind::kScatter:
      run_scatter(dev, prog, op, vals);
      return;
    case LibKind::kAttention:
      run_attention(dev, prog, op, vals, step.attn_partials);
      return;
    case LibKind::kDotGroup:
      run_dot_group(dev, prog, step.group_ops, vals);
      return;
    case LibKind::kSort:
      run_sort(dev, prog, op, vals);
      return;
    case LibKind::kReduceWindow:
      run_reduce_window(dev, prog, op, vals);
      return;
    default:
      fail(Code::kUnimplemented, std::string("library op not available: ") + lib_kind_name(step.lib));
  }
}

}  // namespace pjrtx
