// Host-side launchers of the precompiled library kernels (kernels/*.hip).
// All launches go to the given stream; shapes are validated by the caller.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.h"

namespace pjrtx {

constexpr int kMaxRank = 8;

// N-d box copy: dst[dst_off + sum(i_d * dst_stride_d)] = src[src_off + sum(i_d * src_stride_d)]
// for i in box `dims`. Strides in elements. Element size 1, 2, 4 or 8 bytes.
// When dyn_src/dyn_dst are non-null, they hold `rank` device pointers to
// int32/int64 scalar start indices (clamped to [0, limit_d - dims_d]) that
// are added to the source / destination offsets on the device.
struct BoxCopy {
  int rank = 0;
  int64_t dims[kMaxRank] = {};
  int64_t src_stride[kMaxRank] = {};
  int64_t dst_stride[kMaxRank] = {};
  int64_t src_off = 0, dst_off = 0;
  // dynamic starts (dynamic_slice: source side; dynamic_update_slice: dest side)
  const void* dyn_start[kMaxRank] = {};
  int dyn_start_bytes = 4;    // 4 (i32/u32) or 8 (i64)
  int dyn_start_signed = 1;
  int dyn_on_dst = 0;         // 0: starts offset the source, 1: the destination
  int64_t dyn_limit[kMaxRank] = {};  // full extent of the dynamically indexed tensor
};
void launch_box_copy(hipStream_t s, const BoxCopy& p, const void* src, void* dst, int elem_bytes);

// Fills `n` elements of `dst` with the element at `value` (device pointer).
void launch_fill(hipStream_t s, void* dst, const void* value, int64_t n, int elem_bytes);

// Zeroes `bytes` bytes of `dst` with a kernel (no memset node, no host value:
// safe under graph capture and in the allocation-free execute).
void launch_zero(hipStream_t s, void* dst, int64_t bytes);

// True when workgroup b of a launch runs on the same XCD as workgroup
// b % 8 (the round-robin placement that XCD-local cooperation between the
// workgroups of one launch relies on). Runs a probe kernel and waits.
bool probe_xcd_round_robin(hipStream_t s);

// StableHLO gather with full dimension numbers (clamped starts).
struct GatherParams {
  int out_rank = 0;
  int64_t out_dims[kMaxRank] = {};
  // per output dim: >= 0 -> indices batch dim position (in the indices
  // tensor); < 0 -> window dim: -(operand dim) - 1
  int out_map[kMaxRank] = {};
  int op_rank = 0;
  int64_t op_dims[kMaxRank] = {};
  int64_t op_stride[kMaxRank] = {};
  int64_t slice[kMaxRank] = {};
  int idx_rank = 0;  // rank of start_indices
  int64_t idx_stride[kMaxRank] = {};
  int ivd = 0;        // index_vector_dim (== idx_rank: implicit trailing 1)
  int n_index = 1;    // index vector length
  int start_map[kMaxRank] = {};  // index vector component -> operand dim
  int n_batching = 0;
  int op_batch_dim[kMaxRank] = {};   // operand_batching_dims
  int idx_batch_dim[kMaxRank] = {};  // matching start_indices_batching_dims
  int idx_bytes = 4;
  int idx_signed = 1;
  // > 0: a negative start index i becomes i + wrap (wrapping in idx_bytes)
  // before the clamp (Op::index_wrap).
  int64_t wrap = 0;
};
void launch_gather(hipStream_t s, const GatherParams& p, const void* operand, const void* indices, void* out,
                   int elem_bytes);

// out[i] = a[i] + y[i] computed in f32 and rounded to the element type
// (bf16, f16 or f32): the unfused elementwise add.
void launch_add(hipStream_t s, const void* a, const void* y, void* out, int64_t n, DType t);

// Copies up to kMaxCopySegments independent byte ranges in one launch (used
// to stage small arguments into, and results out of, a replayed graph).
constexpr int kMaxCopySegments = 16;
struct CopySegments {
  int n = 0;
  const void* src[kMaxCopySegments] = {};
  void* dst[kMaxCopySegments] = {};
  int64_t bytes[kMaxCopySegments] = {};
};
void launch_copy_segments(hipStream_t s, const CopySegments& c);

// Dense bf16 MFMA throughput this GPU sustains (TFLOP/s): two waves per SIMD
// on every CU issuing independent v_mfma_f32_16x16x32_bf16 (shape 0) or
// v_mfma_f32_32x32x16_bf16 (shape 1), best of five timed runs. Synchronizes
// the stream.
double measure_mfma_peak_tflops(hipStream_t s, int shape, int compute_units);

}  // namespace pjrtx
