// Windowed reductions (stablehlo.reduce_window) on the GPU.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace pjrtx {

constexpr int kReduceWindowMaxRank = 8;

// out[o] = init (+) in[window of o] in row-major window order, where window
// position w of output o reads input coordinate o * stride + w * dilation -
// pad_low per dimension; coordinates outside the input (padding) contribute
// `init`. (+) is the reducer `op`: 0 sum, 1 product, 2 max, 3 min.
struct ReduceWindowParams {
  int rank = 0;
  int op = 0;
  int64_t in_dims[kReduceWindowMaxRank] = {};
  int64_t out_dims[kReduceWindowMaxRank] = {};
  int64_t window[kReduceWindowMaxRank] = {};
  int64_t stride[kReduceWindowMaxRank] = {};
  int64_t dilation[kReduceWindowMaxRank] = {};
  int64_t pad_low[kReduceWindowMaxRank] = {};
};

// `init` is a device scalar of the element type. Element types: f32, f64,
// bf16, f16 (16-bit floats accumulate in f32, rounded once at the end), s32,
// s64.
void launch_reduce_window(hipStream_t s, const ReduceWindowParams& p, DType t, const void* in, const void* init,
                          void* out);

}  // namespace pjrtx
