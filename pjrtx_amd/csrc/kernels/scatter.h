// Launchers of the scatter / sort kernels (kernels/scatter.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"
#include "kernels/library.h"

namespace pjrtx {

// Key generation for scatter. For each "item" (row mode: one scatter index;
// element mode: one update element) compute the operand row / element it
// targets, or `invalid` when its window is out of bounds (skipped).
struct ScatterKeyParams {
  int64_t items = 0;        // number of keys
  int64_t window_items = 1; // element mode: window elements per scatter index; row mode: 1
  // scatter index -> coordinates in scatter_indices (without index_vector_dim)
  int n_scatter_dims = 0;
  int64_t scatter_dims[kMaxRank] = {};     // extents of the update scatter dims (in order)
  int scatter_idx_dim[kMaxRank] = {};      // matching scatter_indices dim
  int64_t idx_stride[kMaxRank] = {};       // strides of scatter_indices
  int ivd = 0, idx_rank = 0, n_index = 1;
  int start_map[kMaxRank] = {};            // index component -> operand dim
  int n_batching = 0;
  int op_batch_dim[kMaxRank] = {};
  int idx_batch_dim[kMaxRank] = {};        // position among the update scatter dims
  int idx_bytes = 4, idx_signed = 1;
  int op_rank = 0;
  int64_t op_dims[kMaxRank] = {};
  int64_t op_stride[kMaxRank] = {};
  int64_t window[kMaxRank] = {};           // window size per operand dim (1 for inserted/batching)
  // element mode: window coords -> update offset
  int n_window_dims = 0;
  int window_op_dim[kMaxRank] = {};        // operand dim of each update window dim
  int64_t window_extent[kMaxRank] = {};
  int64_t upd_stride_scatter[kMaxRank] = {};  // update strides of the scatter dims
  int64_t upd_stride_window[kMaxRank] = {};   // update strides of the window dims
  int row_mode = 1;
  int64_t row_elems = 1;   // row mode: elements per operand row (window size)
  uint32_t invalid = 0;    // key for skipped items (= number of rows)
};

// Stable LSD radix sort of (key, value) pairs by key (uint32, < 2^bits).
// `tmp_*` are scratch arrays of n elements; `hist` holds 256 * ceil(n/2048)
// uint32 entries plus scan scratch. Result lands in keys/vals.
size_t radix_sort_scratch_bytes(int64_t n);
void launch_radix_sort(hipStream_t s, uint32_t* keys, uint32_t* vals, uint32_t* tmp_keys, uint32_t* tmp_vals,
                       void* scratch, int64_t n, int bits);

// Combiner of the scatter region.
enum class ScatterOp { kAdd, kSet, kMax, kMin, kMul };

// Row mode, long segments: a segment (the updates of one operand row, in
// update order) is cut into chunks of kScatterChunk updates. Chunk 0 folds
// from the operand row, later chunks from their own first update; a row
// with one chunk writes its result directly (the exact sequential fold),
// otherwise the chunk partials are folded in chunk order.
constexpr int kScatterChunk = 256;
size_t scatter_chunk_scratch_bytes(int64_t rows, int64_t n, int64_t row_elems, DType t);
void launch_scatter_chunked(hipStream_t s, int64_t rows, int64_t row_elems, int64_t n, int op, DType t,
                            const void* operand, const void* updates, const uint32_t* perm,
                            const uint32_t* seg_start, const uint32_t* seg_end, void* scratch, void* out);

struct ScatterFoldParams {
  int64_t rows = 0;       // operand rows (element mode: operand elements)
  int64_t row_elems = 1;  // elements per row (element mode: 1)
  int row_mode = 1;
  ScatterOp op = ScatterOp::kAdd;
};

void launch_scatter_keys(hipStream_t s, const ScatterKeyParams& p, const void* indices, uint32_t* keys,
                         uint32_t* vals);
// seg_start/seg_end: `rows` uint32 each (zeroed by this launcher).
void launch_scatter_segments(hipStream_t s, const uint32_t* sorted_keys, int64_t n, uint32_t invalid,
                             uint32_t* seg_start, uint32_t* seg_end, int64_t rows);
// out = fold(operand, updates in order) per target; `operand` may equal `out`.
void launch_scatter_fold(hipStream_t s, const ScatterFoldParams& p, DType t, const void* operand,
                         const void* updates, const uint32_t* perm, const uint32_t* seg_start,
                         const uint32_t* seg_end, void* out);

}  // namespace pjrtx
