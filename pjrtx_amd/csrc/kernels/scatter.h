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

// Row mode: each operand row folds its updates in update order (bit-exact
// against a sequential scatter loop for every type). Segments longer than
// kHotMinUpdates are folded by 64-byte column slices on persistent
// workgroups of their own (a list of hot rows, bucketed by
// floor(log2(length)) so the longest start first), on the second stream
// `aux` (joined back into `s` before return); the other rows one wave per row.
// Integer add / max / min (exact in any order) fold hot rows in parallel
// chunks merged with atomics instead. `h.counts` must be zero on entry (the
// launcher lists the hot rows itself).
constexpr int kHotMinUpdates = 256;
constexpr int kHotSliceBytes = 64;

struct ScatterHotList {
  uint32_t* counts = nullptr;  // [32] rows per length class (zeroed before classify)
  uint32_t* rows = nullptr;    // class k's rows at base[k] ..
  int64_t base[32] = {};
  int kmin = 0;                // lowest class that can hold a hot row
  // 1 when workgroup b runs on XCD b % 8 and the grid is a multiple of 8:
  // consecutive items (the slices of one row) then go to workgroups of one
  // XCD, so the two 64-byte halves of an update row's 128-byte line are
  // read through the same L2.
  int xcd_group = 0;
};
// Early rows: the longest rows, found from a sample of the keys, are folded
// while the keys are still being sorted. `select` (one workgroup) sorts
// kEarlySample keys taken at even strides and lists up to kEarlyRows rows
// that fill at least kEarlyMinRun of them (longest first); the rows' update
// indices are then listed in update order by a count / write pass over the
// keys (a scan of the counts in between only for more than
// kEarlyInlineBlocks blocks), and their slices folded like hot rows. The sorted path
// skips these rows (classify and the bulk fold read the list).
constexpr int kEarlyRows = 8;
constexpr int kEarlySample = 4096;
constexpr int kEarlyMinRun = 32;
constexpr int kEarlyBlockItems = 4096;  // keys per count / write workgroup
constexpr int kEarlyInlineBlocks = 1024;  // up to this many, the write kernel scans the counts itself
struct ScatterEarly {
  uint32_t* rows = nullptr;     // [1 + kEarlyRows]: count, then the rows
  uint32_t* counts = nullptr;   // [kEarlyRows * blocks + 1]
  // [kEarlyRows * blocks + 1]: the scan of `counts`, or (up to
  // kEarlyInlineBlocks blocks) the rows' starts and the total in its first
  // kEarlyRows + 1 words
  uint32_t* offsets = nullptr;
  uint32_t* list = nullptr;     // [n] update indices, row by row
  uint32_t* scan_tmp = nullptr; // [2048]
  int64_t blocks = 0;
  // 1 when workgroup b runs on XCD b % 8: all slices of one early row run on
  // one XCD (ScatterHotList::xcd_group).
  int xcd_group = 0;
};
inline int64_t scatter_early_blocks(int64_t n) { return (n + kEarlyBlockItems - 1) / kEarlyBlockItems; }
// Queues the selection on `aux` (records `selected` after it, which the
// sorted path's classify waits on), then the listing and the early folds.
void launch_scatter_early(hipStream_t aux, hipEvent_t selected, const ScatterEarly& e, const uint32_t* keys, int64_t n,
                          uint32_t invalid, int64_t row_elems, int op, DType t, const void* operand,
                          const void* updates, void* out);

struct ScatterRowsParams {
  int64_t rows = 0;
  int64_t row_elems = 0;
  int64_t hot_wgs = 0;  // persistent hot-slice workgroups (0: every row in bulk)
};
// Class layout for n updates; the list needs scatter_hot_list_words(n) words.
ScatterHotList scatter_hot_list(int64_t n, uint32_t* counts, uint32_t* rows_list);
size_t scatter_hot_list_words(int64_t n);
void launch_scatter_rows(hipStream_t s, hipStream_t aux, hipEvent_t fork, hipEvent_t join, int64_t rows,
                         int64_t row_elems, int op, DType t, const void* operand, const void* updates,
                         const uint32_t* perm, const uint32_t* seg_start, const uint32_t* seg_end,
                         const ScatterHotList& h, int64_t hot_wgs, void* out,
                         const uint32_t* early_rows = nullptr);

struct ScatterFoldParams {
  int64_t rows = 0;       // operand rows (element mode: operand elements)
  int64_t row_elems = 1;  // elements per row (element mode: 1)
  int row_mode = 1;
  ScatterOp op = ScatterOp::kAdd;
};

// keys2, when not null, receives a second copy of the keys.
// `zero`: zero_n words the key kernel also zeroes (may be null).
void launch_scatter_keys(hipStream_t s, const ScatterKeyParams& p, const void* indices, uint32_t* keys,
                         uint32_t* vals, uint32_t* keys2 = nullptr, uint32_t* zero = nullptr, int64_t zero_n = 0);
// seg_start/seg_end: `rows` uint32 each; they and `extra_zero` words after
// seg_end are zeroed by this launcher unless `zeroed` (the key kernel did).
void launch_scatter_segments(hipStream_t s, const uint32_t* sorted_keys, int64_t n, uint32_t invalid,
                             uint32_t* seg_start, uint32_t* seg_end, int64_t rows, int64_t extra_zero = 0,
                             bool zeroed = false);
// out = fold(operand, updates in order) per target; `operand` may equal `out`.
void launch_scatter_fold(hipStream_t s, const ScatterFoldParams& p, DType t, const void* operand,
                         const void* updates, const uint32_t* perm, const uint32_t* seg_start,
                         const uint32_t* seg_end, void* out);

}  // namespace pjrtx
