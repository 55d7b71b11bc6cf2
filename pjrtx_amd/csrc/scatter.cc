// scatter: StableHLO dimension numbers -> key / sort / segment / fold launches.
//
// Semantics: StableHLO `scatter` with one operand; the update computation is
// classified as add / set (returns the update) / max / min / multiply. A
// window whose start is out of bounds is skipped as a whole, as XLA does.
// Updates to the same target are applied in update order, the order of a
// sequential scatter loop.
#include <algorithm>

#include "kernels/scatter.h"
#include "runtime.h"

namespace pjrtx {

namespace {

ScatterOp classify_scatter_region(const Program& prog, const Op& op) {
  PJRTX_CHECK(op.regions.size() == 1, Code::kInvalidArgument, "scatter needs one update computation");
  const Region& r = op.regions[0];
  PJRTX_CHECK(r.params.size() == 2, Code::kUnimplemented, "scatter with more than one operand is not supported");
  const Op& ret = r.ops.back();
  PJRTX_CHECK(ret.kind == OpKind::kReturn && ret.operands.size() == 1, Code::kInvalidArgument, "malformed scatter region");
  const int res = ret.operands[0];
  if (res == r.params[1]) return ScatterOp::kSet;
  for (const Op& b : r.ops) {
    if (b.results.empty() || b.results[0] != res) continue;
    const bool args = b.operands.size() == 2 &&
                      ((b.operands[0] == r.params[0] && b.operands[1] == r.params[1]) ||
                       (b.operands[0] == r.params[1] && b.operands[1] == r.params[0]));
    PJRTX_CHECK(args, Code::kUnimplemented, "scatter region must combine the two block arguments directly");
    switch (b.kind) {
      case OpKind::kAdd: return ScatterOp::kAdd;
      case OpKind::kMultiply: return ScatterOp::kMul;
      case OpKind::kMaximum: return ScatterOp::kMax;
      case OpKind::kMinimum: return ScatterOp::kMin;
      default: break;
    }
  }
  (void)prog;
  fail(Code::kUnimplemented, "scatter update computation is not add/set/max/min/multiply");
}

void strides_of(const Dims& d, int64_t* out) {
  int64_t s = 1;
  for (int i = static_cast<int>(d.size()) - 1; i >= 0; --i) {
    out[i] = s;
    s *= d[i];
  }
}

}  // namespace

void run_scatter(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals) {
  PJRTX_CHECK(op.operands.size() == 3, Code::kUnimplemented, "scatter with more than one operand is not supported");
  const TensorType& xt = prog.type(op.operands[0]);
  const TensorType& it = prog.type(op.operands[1]);
  const TensorType& ut = prog.type(op.operands[2]);
  PJRTX_CHECK(xt.rank() <= kMaxRank && it.rank() <= kMaxRank && ut.rank() <= kMaxRank, Code::kUnimplemented,
              "scatter: rank too large");
  const ScatterOp sop = classify_scatter_region(prog, op);
  hipStream_t s = dev->stream();
  void* out = vals[op.results[0]]->ptr;
  const void* X = vals[op.operands[0]]->ptr;
  const void* I = vals[op.operands[1]]->ptr;
  const void* U = vals[op.operands[2]]->ptr;

  ScatterKeyParams p;
  p.op_rank = xt.rank();
  p.idx_rank = it.rank();
  p.ivd = static_cast<int>(op.index_vector_dim < 0 ? it.rank() : op.index_vector_dim);
  p.n_index = static_cast<int>(op.scatter_dims_to_operand_dims.size());
  for (int k = 0; k < p.n_index; ++k) p.start_map[k] = static_cast<int>(op.scatter_dims_to_operand_dims[k]);
  for (int d = 0; d < p.op_rank; ++d) p.op_dims[d] = xt.dims[d];
  strides_of(xt.dims, p.op_stride);
  strides_of(it.dims, p.idx_stride);
  p.idx_bytes = static_cast<int>(dtype_size(it.dtype));
  p.idx_signed = dtype_is_signed_int(it.dtype);

  int64_t ust[kMaxRank];
  strides_of(ut.dims, ust);
  // Update scatter dims (not window dims), in order; their scatter_indices dims.
  std::vector<int> upd_scatter;
  for (int d = 0; d < ut.rank(); ++d)
    if (std::find(op.update_window_dims.begin(), op.update_window_dims.end(), d) == op.update_window_dims.end())
      upd_scatter.push_back(d);
  std::vector<int> idx_batch_dims;
  for (int d = 0; d < it.rank(); ++d)
    if (d != p.ivd) idx_batch_dims.push_back(d);
  PJRTX_CHECK(upd_scatter.size() == idx_batch_dims.size(), Code::kInvalidArgument,
              "scatter: update scatter dims do not match the indices");
  p.n_scatter_dims = static_cast<int>(upd_scatter.size());
  int64_t n_scatter = 1;
  for (int j = 0; j < p.n_scatter_dims; ++j) {
    p.scatter_dims[j] = ut.dims[upd_scatter[j]];
    p.scatter_idx_dim[j] = idx_batch_dims[j];
    p.upd_stride_scatter[j] = ust[upd_scatter[j]];
    n_scatter *= p.scatter_dims[j];
  }
  p.n_batching = static_cast<int>(op.input_batching_dims.size());
  for (int k = 0; k < p.n_batching; ++k) {
    p.op_batch_dim[k] = static_cast<int>(op.input_batching_dims[k]);
    const int idim = static_cast<int>(op.scatter_indices_batching_dims[k]);
    const auto pos = std::find(idx_batch_dims.begin(), idx_batch_dims.end(), idim) - idx_batch_dims.begin();
    p.idx_batch_dim[k] = static_cast<int>(pos);
  }
  // Window dims of the operand: not inserted and not batching, increasing.
  std::vector<int> window_op;
  for (int d = 0; d < p.op_rank; ++d) {
    const bool ins = std::find(op.inserted_window_dims.begin(), op.inserted_window_dims.end(), d) !=
                     op.inserted_window_dims.end();
    const bool bat = std::find(op.input_batching_dims.begin(), op.input_batching_dims.end(), d) !=
                     op.input_batching_dims.end();
    p.window[d] = 1;
    if (!ins && !bat) window_op.push_back(d);
  }
  PJRTX_CHECK(window_op.size() == op.update_window_dims.size(), Code::kInvalidArgument,
              "scatter: update window dims do not match the operand");
  p.n_window_dims = static_cast<int>(window_op.size());
  int64_t window_elems = 1;
  for (int j = 0; j < p.n_window_dims; ++j) {
    const int wd = static_cast<int>(op.update_window_dims[j]);
    p.window[window_op[j]] = ut.dims[wd];
    p.window_op_dim[j] = window_op[j];
    p.window_extent[j] = ut.dims[wd];
    p.upd_stride_window[j] = ust[wd];
    window_elems *= ut.dims[wd];
  }
  // Row mode: the window is a whole trailing block of the operand and the
  // trailing block of each update.
  bool row_mode = true;
  const int nw = p.n_window_dims;
  for (int j = 0; j < nw; ++j) {
    if (window_op[j] != p.op_rank - nw + j) row_mode = false;
    if (op.update_window_dims[j] != ut.rank() - nw + j) row_mode = false;
    if (p.window[window_op[j]] != xt.dims[window_op[j]]) row_mode = false;
  }
  p.row_mode = row_mode ? 1 : 0;
  p.row_elems = row_mode ? window_elems : 1;
  p.window_items = row_mode ? 1 : window_elems;
  p.items = n_scatter * p.window_items;
  const int64_t rows = row_mode ? (window_elems ? xt.elements() / window_elems : 0) : xt.elements();
  PJRTX_CHECK(rows < (int64_t(1) << 32) - 1 && p.items < (int64_t(1) << 32) && ut.elements() < (int64_t(1) << 32),
              Code::kUnimplemented, "scatter: more than 2^32 targets or updates");
  p.invalid = static_cast<uint32_t>(rows);

  const size_t esz = dtype_size(xt.dtype);
  if (xt.elements() == 0) return;
  if (p.items == 0 || window_elems == 0) {
    hip_check(hipMemcpyAsync(out, X, xt.bytes(), hipMemcpyDeviceToDevice, s), "hipMemcpyAsync(scatter copy)");
    return;
  }
  const int64_t n = p.items;
  MemRef keys = dev->allocate(n * 4), vals_a = dev->allocate(n * 4);
  MemRef tkeys = dev->allocate(n * 4), tvals = dev->allocate(n * 4);
  MemRef scratch = dev->allocate(radix_sort_scratch_bytes(n));
  // seg_start, seg_end, then the 32 hot-class counters: zeroed by one launch.
  MemRef seg = dev->allocate(static_cast<size_t>(rows) * 8 + 32 * 4);
  uint32_t* K = static_cast<uint32_t*>(keys->ptr);
  uint32_t* V = static_cast<uint32_t*>(vals_a->ptr);
  // Early rows (the longest, found from a sample of the keys) are folded on
  // the second stream while the keys are sorted (environment:
  // PJRTX_SCATTER_EARLY=0 disables). Only where the hot rows fold in update
  // order by 16-byte slices (the integer add / max / min chunks are exact in
  // any order and need no early start).
  const bool int_type = xt.dtype == DType::kS32 || xt.dtype == DType::kU32 || xt.dtype == DType::kS64;
  const bool chunked = int_type && (sop == ScatterOp::kAdd || sop == ScatterOp::kMax || sop == ScatterOp::kMin);
  const bool vec16 = (p.row_elems * static_cast<int64_t>(esz)) % 16 == 0 && reinterpret_cast<uintptr_t>(X) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(U) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
  // Slices of one row on one XCD (PJRTX_SCATTER_XCD=0 turns it off): only
  // where workgroup b is known to run on XCD b % 8.
  const int xcd_group = dev->xcd_round_robin() && env_int("PJRTX_SCATTER_XCD", 1) != 0 ? 1 : 0;
  ScatterEarly early;
  MemRef early_mem;
  const bool use_early = p.row_mode && !chunked && vec16 && n >= (int64_t(1) << 16) && n < (int64_t(1) << 31) &&
                         env_int("PJRTX_SCATTER_EARLY", 1) != 0;
  if (use_early) {
    early.blocks = scatter_early_blocks(n);
    early.xcd_group = xcd_group;
    const int64_t words = (1 + kEarlyRows) + 2 * (kEarlyRows * early.blocks + 1) + 2 * n + 2048;
    early_mem = dev->allocate(static_cast<size_t>(words) * 4);
    uint32_t* w = static_cast<uint32_t*>(early_mem->ptr);
    early.rows = w;
    early.counts = early.rows + (1 + kEarlyRows);
    early.offsets = early.counts + (kEarlyRows * early.blocks + 1);
    early.scan_tmp = early.offsets + (kEarlyRows * early.blocks + 1);
    early.list = early.scan_tmp + 2048;
    // The sort rewrites K in place: the early path reads its own copy of
    // the keys, written by the same key kernel.
    uint32_t* keys_copy = early.list + n;
    launch_scatter_keys(s, p, I, K, V, keys_copy, static_cast<uint32_t*>(seg->ptr), 2 * rows + 32);
    hipStream_t aux = dev->aux_stream();
    hip_check(hipEventRecord(dev->fork_event(), s), "hipEventRecord(scatter early fork)");
    hip_check(hipStreamWaitEvent(aux, dev->fork_event(), 0), "hipStreamWaitEvent(scatter early fork)");
    launch_scatter_early(aux, dev->side_event(), early, keys_copy, n, p.invalid, p.row_elems,
                         static_cast<int>(sop), xt.dtype, X, U, out);
  } else {
    launch_scatter_keys(s, p, I, K, V, nullptr, static_cast<uint32_t*>(seg->ptr), 2 * rows + 32);
  }
  int bits = 1;
  while ((int64_t(1) << bits) <= rows) ++bits;  // keys are in [0, rows]
  launch_radix_sort(s, K, V, static_cast<uint32_t*>(tkeys->ptr), static_cast<uint32_t*>(tvals->ptr), scratch->ptr, n, bits);
  uint32_t* seg_start = static_cast<uint32_t*>(seg->ptr);
  uint32_t* seg_end = seg_start + rows;
  uint32_t* hot_counts = seg_end + rows;
  launch_scatter_segments(s, K, n, p.invalid, seg_start, seg_end, rows, 32, /*zeroed=*/true);
  if (p.row_mode) {
    // Segments longer than kHotMinUpdates fold by column slices on
    // persistent workgroups (two per CU) on the device's second stream; the
    // hot list lives in the sort's temporary key array, free again after
    // the sort.
    int64_t hot_wgs = 0;
    ScatterHotList h;
    if (n > kHotMinUpdates && scatter_hot_list_words(n) <= static_cast<size_t>(n)) {
      h = scatter_hot_list(n, hot_counts, static_cast<uint32_t*>(tkeys->ptr));
      h.xcd_group = xcd_group;
      const int64_t cols = kHotSliceBytes / static_cast<int64_t>(dtype_size(xt.dtype));
      const int64_t slices = (p.row_elems + cols - 1) / cols;
      const int64_t max_items = (n / (kHotMinUpdates + 1)) * slices;
      hot_wgs = std::min<int64_t>(max_items, env_int("PJRTX_SCATTER_HOT_PER_CU", 2) *
                                                 static_cast<int64_t>(dev->compute_units()));
    }
    if (use_early) {
      // classify and the bulk fold skip the early rows: wait for the list.
      hip_check(hipStreamWaitEvent(s, dev->side_event(), 0), "hipStreamWaitEvent(scatter early selected)");
      launch_scatter_rows(s, dev->aux2_stream(), dev->fork2_event(), dev->join2_event(), rows, p.row_elems,
                          static_cast<int>(sop), xt.dtype, X, U, V, seg_start, seg_end, h, hot_wgs, out, early.rows);
      hip_check(hipEventRecord(dev->join_event(), dev->aux_stream()), "hipEventRecord(scatter early join)");
      hip_check(hipStreamWaitEvent(s, dev->join_event(), 0), "hipStreamWaitEvent(scatter early join)");
      return;
    }
    launch_scatter_rows(s, dev->aux_stream(), dev->fork_event(), dev->join_event(), rows, p.row_elems,
                        static_cast<int>(sop), xt.dtype, X, U, V, seg_start, seg_end, h,
                        hot_wgs, out);
    return;
  }
  ScatterFoldParams f;
  f.rows = rows;
  f.row_elems = p.row_elems;
  f.row_mode = p.row_mode;
  f.op = sop;
  launch_scatter_fold(s, f, xt.dtype, X, U, V, seg_start, seg_end, out);
  (void)esz;
}

}  // namespace pjrtx
